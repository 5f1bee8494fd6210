// nanovllm_shim.cpp -- PyTorch-ROCm binding of libmimoe.so with the schema of
// the reference extension (Int8-gemm/nanovllm_ops.cpp:349-412):
//   torch.classes.nanovllm.MoEInfer(E, H, I, quant_type)
//   torch.ops.nanovllm.moe_forward(hidden, topk_ids, topk_w, moe) -> Tensor
// plus the build-defined W4A16 loader store_awq_repack, the out variant
// moe_forward_out, and the router step the reference runs in its Python
// harness (make_topk_from_logits_cpu, Int8-gemm/test/fused_moe_cpu.py:20-37)
// as moe_topk_softmax / moe_forward_logits.  Only this file sees torch types; it calls the C ABI of
// include/mi_moe.h on the current HIP stream.
#include <c10/hip/HIPStream.h>
#include <torch/custom_class.h>
#include <tuple>
#include <vector>
#include <torch/library.h>
#include <ATen/ATen.h>

#include <string>

#include "mi_moe.h"

namespace {

void check_status(int rc, const char* what) {
  TORCH_CHECK(rc == MI_MOE_OK, what, ": ", mi_moe_last_error(), " (status ", rc, ")");
}

int act_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kBFloat16) return MI_MOE_BF16;
  TORCH_CHECK(t.scalar_type() == at::kHalf, "expected float16 or bfloat16, got ", t.scalar_type());
  return MI_MOE_F16;
}

void* stream_of(const at::Tensor& ref) {
  if (ref.is_cuda()) return (void*)c10::hip::getCurrentHIPStream(ref.get_device()).stream();
  return (void*)c10::hip::getCurrentHIPStream().stream();
}

struct MoEInferHandle : torch::CustomClassHolder {
  int64_t quant_type;
  mi_moe_handle* h = nullptr;

  // Int8-gemm/nanovllm_ops.cpp:28-30 (quant_type: 0 Q8_0, 1 Q4_0; 2 W4A16)
  MoEInferHandle(int64_t E, int64_t H, int64_t I, int64_t qt) : quant_type(qt) {
    check_status(mi_moe_create(E, H, I, (int)qt, &h), "MoEInfer");
  }
  ~MoEInferHandle() override {
    if (h) mi_moe_destroy(h);
  }
  std::string get_quant_type() const {
    return quant_type == 1 ? "Q4_0" : (quant_type == 2 ? "W4A16" : "Q8_0");
  }
  int64_t info(int which) const {
    int64_t E = 0, H = 0, I = 0;
    check_status(mi_moe_get_info(h, &E, &H, &I, nullptr, nullptr), "get_info");
    return which == 0 ? E : (which == 1 ? H : I);
  }
};

at::Tensor contig(const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

void forward_into(const at::Tensor& hidden, const at::Tensor& topk_ids, const at::Tensor& topk_w,
                  const c10::intrusive_ptr<MoEInferHandle>& moe, at::Tensor& out) {
  TORCH_CHECK(hidden.is_cuda(), "moe_forward: hidden must be a HIP (cuda) tensor on MI355X; "
              "this build has no CPU path");
  TORCH_CHECK(hidden.dim() == 2 && topk_ids.dim() == 2 && topk_w.dim() == 2,
              "moe_forward: expected hidden [T,H], topk_ids [T,K], topk_w [T,K]");
  TORCH_CHECK(topk_ids.scalar_type() == at::kInt, "topk_ids must be int32");
  TORCH_CHECK(topk_w.scalar_type() == at::kFloat, "topk_w must be float32");
  TORCH_CHECK(topk_ids.size(0) == hidden.size(0) && topk_w.size(0) == hidden.size(0) &&
                  topk_w.size(1) == topk_ids.size(1),
              "moe_forward: token / top_k dimensions disagree");
  TORCH_CHECK(hidden.size(1) == moe->info(1), "hidden size ", hidden.size(1), " != handle H ",
              moe->info(1));
  TORCH_CHECK(topk_ids.device() == hidden.device() && topk_w.device() == hidden.device() &&
                  out.device() == hidden.device(),
              "all tensors must be on the same device");
  TORCH_CHECK(out.sizes() == hidden.sizes() && out.scalar_type() == hidden.scalar_type() &&
                  out.is_contiguous(),
              "out must be a contiguous tensor like hidden");
  at::Tensor x = contig(hidden), ids = contig(topk_ids), w = contig(topk_w);
  check_status(mi_moe_forward(moe->h, x.data_ptr(), out.data_ptr(), w.data_ptr<float>(),
                              ids.data_ptr<int32_t>(), x.size(0), ids.size(1), act_code(x),
                              stream_of(x)),
               "moe_forward");
}

// Int8-gemm/nanovllm_ops.cpp:219-236
at::Tensor moe_forward_hip(const at::Tensor& hidden, const at::Tensor& topk_ids,
                           const at::Tensor& topk_w,
                           const c10::intrusive_ptr<MoEInferHandle>& moe) {
  at::Tensor out = at::empty_like(hidden, hidden.options().memory_format(at::MemoryFormat::Contiguous));
  forward_into(hidden, topk_ids, topk_w, moe, out);
  return out;
}

at::Tensor moe_forward_cpu_reject(const at::Tensor&, const at::Tensor&, const at::Tensor&,
                                  const c10::intrusive_ptr<MoEInferHandle>&) {
  TORCH_CHECK(false, "nanovllm::moe_forward: this MI355X build runs on HIP tensors only "
              "(move hidden/topk_ids/topk_w to cuda)");
}

void moe_forward_out_hip(const at::Tensor& hidden, const at::Tensor& topk_ids,
                         const at::Tensor& topk_w, const c10::intrusive_ptr<MoEInferHandle>& moe,
                         at::Tensor out) {
  forward_into(hidden, topk_ids, topk_w, moe, out);
}

int logits_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kFloat) return MI_MOE_F32;
  if (t.scalar_type() == at::kBFloat16) return MI_MOE_BF16;
  TORCH_CHECK(t.scalar_type() == at::kHalf, "router logits must be float32, bfloat16 or float16");
  return MI_MOE_F16;
}

std::tuple<at::Tensor, at::Tensor> moe_topk_softmax_hip(const at::Tensor& logits, int64_t top_k,
                                                        bool renormalize) {
  TORCH_CHECK(logits.is_cuda() && logits.dim() == 2, "moe_topk_softmax: logits must be a [T,E] HIP tensor");
  at::Tensor x = contig(logits);
  const int64_t T = x.size(0), E = x.size(1);
  at::Tensor ids = at::empty({T, top_k}, x.options().dtype(at::kInt));
  at::Tensor w = at::empty({T, top_k}, x.options().dtype(at::kFloat));
  check_status(mi_moe_topk_softmax(x.data_ptr(), logits_code(x), T, E, top_k, renormalize ? 1 : 0,
                                   ids.data_ptr<int32_t>(), w.data_ptr<float>(), stream_of(x)),
               "moe_topk_softmax");
  return {ids, w};
}

std::tuple<at::Tensor, at::Tensor> moe_topk_softmax_cpu_reject(const at::Tensor&, int64_t, bool) {
  TORCH_CHECK(false, "nanovllm::moe_topk_softmax: this MI355X build runs on HIP tensors only");
}

at::Tensor moe_forward_logits_hip(const at::Tensor& hidden, const at::Tensor& router_logits, int64_t top_k,
                                  bool renormalize, const c10::intrusive_ptr<MoEInferHandle>& moe) {
  TORCH_CHECK(hidden.is_cuda() && router_logits.is_cuda() && hidden.device() == router_logits.device(),
              "moe_forward_logits: hidden and router_logits must be HIP tensors on one device");
  TORCH_CHECK(hidden.dim() == 2 && router_logits.dim() == 2 && router_logits.size(0) == hidden.size(0),
              "moe_forward_logits: expected hidden [T,H], router_logits [T,E]");
  TORCH_CHECK(router_logits.size(1) == moe->info(0), "router_logits has ", router_logits.size(1),
              " experts, handle has ", moe->info(0));
  TORCH_CHECK(hidden.size(1) == moe->info(1), "hidden size ", hidden.size(1), " != handle H ", moe->info(1));
  at::Tensor x = contig(hidden), g = contig(router_logits);
  at::Tensor out = at::empty_like(x);
  check_status(mi_moe_forward_logits(moe->h, x.data_ptr(), out.data_ptr(), g.data_ptr(), logits_code(g),
                                     x.size(0), top_k, renormalize ? 1 : 0, act_code(x), nullptr, nullptr,
                                     stream_of(x)),
               "moe_forward_logits");
  return out;
}

at::Tensor moe_forward_logits_cpu_reject(const at::Tensor&, const at::Tensor&, int64_t, bool,
                                         const c10::intrusive_ptr<MoEInferHandle>&) {
  TORCH_CHECK(false, "nanovllm::moe_forward_logits: this MI355X build runs on HIP tensors only");
}

int scale_code(const at::Tensor& d) {
  if (d.scalar_type() == at::kBFloat16) return MI_MOE_BF16;
  TORCH_CHECK(d.scalar_type() == at::kHalf, "scales must be float16 or bfloat16");
  return MI_MOE_F16;
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(nanovllm, m) {
  m.class_<MoEInferHandle>("MoEInfer")
      .def(torch::init<int64_t, int64_t, int64_t, int64_t>())
      // Int8-gemm/nanovllm_ops.cpp:354-365
      .def("quantize_and_store_expert",
           [](const c10::intrusive_ptr<MoEInferHandle>& self, int64_t expert_idx,
              const std::string& proj_name, const at::Tensor& w) {
             TORCH_CHECK(self->quant_type == 0,
                         "Q4_0 does not support online quantization. "
                         "Use store_quantized_repack() with pre-quantized weights.");
             int proj = proj_name == "gate_proj" ? 0 : proj_name == "up_proj" ? 1
                      : proj_name == "down_proj" ? 2 : -1;
             TORCH_CHECK(proj >= 0, "Unknown proj_name: ", proj_name);
             at::Tensor wc = contig(w);
             int wd = wc.scalar_type() == at::kFloat ? 2 : wc.scalar_type() == at::kBFloat16 ? 1
                    : wc.scalar_type() == at::kHalf ? 0 : -1;
             TORCH_CHECK(wd >= 0, "weight must be float32, float16 or bfloat16");
             const int64_t H = self->info(1), I = self->info(2);
             TORCH_CHECK(wc.dim() == 2, "weight must be 2D");
             if (proj < 2) {
               TORCH_CHECK(wc.size(0) == I && wc.size(1) == H, "gate/up weight must be [I,H]");
             } else {
               TORCH_CHECK(wc.size(0) == H && wc.size(1) == I, "down weight must be [H,I]");
             }
             check_status(mi_moe_quantize_and_store_expert(self->h, expert_idx, proj, wc.data_ptr(),
                                                           wd, wc.is_cuda() ? 1 : 0, stream_of(wc)),
                          "quantize_and_store_expert");
           })
      // Int8-gemm/nanovllm_ops.cpp:366-371
      .def("store_quantized_repack",
           [](const c10::intrusive_ptr<MoEInferHandle>& self, const at::Tensor& gate_up_qs,
              const at::Tensor& gate_up_d, const at::Tensor& down_qs, const at::Tensor& down_d) {
             TORCH_CHECK(self->quant_type == 0 || self->quant_type == 1,
                         "store_quantized_repack needs a Q8_0 or Q4_0 handle");
             TORCH_CHECK(gate_up_d.scalar_type() == down_d.scalar_type(),
                         "gate_up_d and down_proj_d must have the same dtype");
             const int64_t E = self->info(0), H = self->info(1), I = self->info(2);
             TORCH_CHECK(gate_up_qs.dim() == 3, "gate_up_qs must be [E,2I,H]");
             TORCH_CHECK(down_qs.dim() == 3, "down_proj_qs must be [E,H,I]");
             if (self->quant_type == 0) {
               TORCH_CHECK(gate_up_qs.scalar_type() == at::kChar && down_qs.scalar_type() == at::kChar,
                           "Q8_0 qs must be int8");
               TORCH_CHECK(gate_up_qs.size(0) == E && gate_up_qs.size(1) == 2 * I && gate_up_qs.size(2) == H &&
                               down_qs.size(0) == E && down_qs.size(1) == H && down_qs.size(2) == I,
                           "Q8_0 qs shapes must be [E,2I,H] and [E,H,I]");
             } else {
               TORCH_CHECK((gate_up_qs.scalar_type() == at::kInt || gate_up_qs.scalar_type() == at::kUInt32) &&
                               (down_qs.scalar_type() == at::kInt || down_qs.scalar_type() == at::kUInt32),
                           "Q4_0 qs must be int32 (uint32 storage)");
               TORCH_CHECK(gate_up_qs.size(0) == E && gate_up_qs.size(1) == 2 * I && gate_up_qs.size(2) == H / 8 &&
                               down_qs.size(0) == E && down_qs.size(1) == H && down_qs.size(2) == I / 8,
                           "Q4_0 qs shapes must be [E,2I,H/8] and [E,H,I/8]");
             }
             TORCH_CHECK(gate_up_d.numel() == E * 2 * I * (H / 32) && down_d.numel() == E * H * (I / 32),
                         "scale shapes must be [E,2I,H/32] and [E,H,I/32]");
             at::Tensor a = contig(gate_up_qs), b = contig(gate_up_d), c = contig(down_qs), d = contig(down_d);
             const bool dev = a.is_cuda();
             TORCH_CHECK(b.is_cuda() == dev && c.is_cuda() == dev && d.is_cuda() == dev,
                         "all weight tensors must be on one device");
             check_status(mi_moe_store_quantized(self->h, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                                 d.data_ptr(), scale_code(b), dev ? 1 : 0, stream_of(a)),
                          "store_quantized_repack");
           })
      // build-defined W4A16 (AWQ layout) loader; see include/mi_moe.h
      .def("store_awq_repack",
           [](const c10::intrusive_ptr<MoEInferHandle>& self, const at::Tensor& w13_qweight,
              const at::Tensor& w13_qzeros, const at::Tensor& w13_scales,
              const at::Tensor& w2_qweight, const at::Tensor& w2_qzeros,
              const at::Tensor& w2_scales, int64_t group_size) {
             TORCH_CHECK(self->quant_type == 2, "store_awq_repack needs a W4A16 handle (quant_type 2)");
             const int64_t E = self->info(0), H = self->info(1), I = self->info(2);
             TORCH_CHECK(group_size > 0 && H % group_size == 0 && I % group_size == 0, "bad group_size");
             const int64_t g = group_size;
             TORCH_CHECK(w13_qweight.sizes() == at::IntArrayRef({E, H, 2 * I / 8}) &&
                             w13_qzeros.sizes() == at::IntArrayRef({E, H / g, 2 * I / 8}) &&
                             w13_scales.sizes() == at::IntArrayRef({E, H / g, 2 * I}),
                         "w13 AWQ tensors must be [E,H,2I/8], [E,H/g,2I/8], [E,H/g,2I]");
             TORCH_CHECK(w2_qweight.sizes() == at::IntArrayRef({E, I, H / 8}) &&
                             w2_qzeros.sizes() == at::IntArrayRef({E, I / g, H / 8}) &&
                             w2_scales.sizes() == at::IntArrayRef({E, I / g, H}),
                         "w2 AWQ tensors must be [E,I,H/8], [E,I/g,H/8], [E,I/g,H]");
             TORCH_CHECK(w13_qweight.scalar_type() == at::kInt && w13_qzeros.scalar_type() == at::kInt &&
                             w2_qweight.scalar_type() == at::kInt && w2_qzeros.scalar_type() == at::kInt,
                         "qweight / qzeros must be int32");
             TORCH_CHECK(w13_scales.scalar_type() == w2_scales.scalar_type(), "scale dtypes differ");
             at::Tensor a = contig(w13_qweight), b = contig(w13_qzeros), c = contig(w13_scales),
                        d = contig(w2_qweight), e = contig(w2_qzeros), f = contig(w2_scales);
             const bool dev = a.is_cuda();
             TORCH_CHECK(b.is_cuda() == dev && c.is_cuda() == dev && d.is_cuda() == dev &&
                             e.is_cuda() == dev && f.is_cuda() == dev,
                         "all weight tensors must be on one device");
             check_status(mi_moe_store_awq(self->h, a.data_ptr<int32_t>(), b.data_ptr<int32_t>(),
                                           c.data_ptr(), d.data_ptr<int32_t>(), e.data_ptr<int32_t>(),
                                           f.data_ptr(), g, scale_code(c), dev ? 1 : 0, stream_of(a)),
                          "store_awq_repack");
           })
      .def("get_last_run_time_ms",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) {
             return mi_moe_get_last_run_time_ms(self->h);
           })
      .def("get_last_phase_times_ms",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) {
             double ms[2] = {0.0, 0.0};
             const int n = mi_moe_get_last_phase_times_ms(self->h, ms, 2);
             TORCH_CHECK(n > 0, "get_last_phase_times_ms: ", mi_moe_last_error());
             return std::vector<double>(ms, ms + n);
           })
      .def("set_timing",
           [](const c10::intrusive_ptr<MoEInferHandle>& self, bool enable) {
             check_status(mi_moe_set_timing(self->h, enable ? 1 : 0), "set_timing");
           })
      .def("get_quant_type",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) { return self->get_quant_type(); })
      .def("get_num_experts",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) { return self->info(0); })
      .def("get_hidden_size",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) { return self->info(1); })
      .def("get_intermediate_size",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) { return self->info(2); });

  m.def("moe_forward(Tensor hidden, Tensor topk_ids, Tensor topk_w, "
        "__torch__.torch.classes.nanovllm.MoEInfer moe) -> Tensor");
  m.def("moe_forward_out(Tensor hidden, Tensor topk_ids, Tensor topk_w, "
        "__torch__.torch.classes.nanovllm.MoEInfer moe, Tensor(a!) out) -> ()");
  m.def("moe_topk_softmax(Tensor logits, int top_k, bool renormalize=True) -> (Tensor, Tensor)");
  m.def("moe_forward_logits(Tensor hidden, Tensor router_logits, int top_k, bool renormalize, "
        "__torch__.torch.classes.nanovllm.MoEInfer moe) -> Tensor");
}

TORCH_LIBRARY_IMPL(nanovllm, CUDA, m) {
  m.impl("moe_forward", &moe_forward_hip);
  m.impl("moe_forward_out", &moe_forward_out_hip);
  m.impl("moe_topk_softmax", &moe_topk_softmax_hip);
  m.impl("moe_forward_logits", &moe_forward_logits_hip);
}

TORCH_LIBRARY_IMPL(nanovllm, CPU, m) {
  m.impl("moe_forward", &moe_forward_cpu_reject);
  m.impl("moe_topk_softmax", &moe_topk_softmax_cpu_reject);
  m.impl("moe_forward_logits", &moe_forward_logits_cpu_reject);
}
