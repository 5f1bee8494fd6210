// nanovllm_shim.cpp -- PyTorch-ROCm binding of libmimoe.so with the schema of
// the reference extension (Int8-gemm/nanovllm_ops.cpp:349-412):
//   torch.classes.nanovllm.MoEInfer(E, H, I, quant_type)
//   torch.ops.nanovllm.moe_forward(hidden, topk_ids, topk_w, moe) -> Tensor
// plus the build-defined W4A16 loader store_awq_repack, the out variant
// moe_forward_out, and the router step the reference runs in its Python
// harness (make_topk_from_logits_cpu, Int8-gemm/test/fused_moe_cpu.py:20-37)
// as moe_topk_softmax / moe_forward_logits.  Only this file sees torch types; it calls the C ABI of
// include/mi_moe.h: HIP tensors run the device kernels on the current HIP stream; CPU tensors run the
// host engine (the reference's CPU algorithm for Q8_0 / Q4_0; every expert on the host executor for
// W4A16), which needs weights stored from host tensors (kept by default when no HIP device is present,
// or with MIMOE_HOST_WEIGHTS=1; never with MIMOE_HOST_WEIGHTS=0).
#include <c10/hip/HIPStream.h>
#include <torch/custom_class.h>
#include <tuple>
#include <vector>
#include <torch/library.h>
#include <ATen/ATen.h>

#include <cstdlib>
#include <string>
#include <chrono>
#include <algorithm>
#include <cmath>

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

// The reference's CPU layout variables (Int8-gemm/moe_infer.cpp:25,
// Int8-gemm/numa_threadpool.h:498-504, README.md:179): -1 when unset.
int64_t env_int(const char* name) {
  const char* s = getenv(name);
  if (!s || !*s) return -1;
  char* end = nullptr;
  const long long v = strtoll(s, &end, 10);
  TORCH_CHECK(end && *end == '\0', name, "=", s, " is not an integer");
  return v;
}

// Host threads of the CPU path: MIMOE_CPU_THREADS, else OMP_NUM_THREADS, else
// every CPU of the affinity mask (0).
int host_threads() {
  for (const char* v : {"MIMOE_CPU_THREADS", "OMP_NUM_THREADS"}) {
    const char* s = getenv(v);
    if (s && atoi(s) > 0) return atoi(s);
  }
  return 0;
}

bool hip_device_present() {
  int n = 0;
  return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

struct MoEInferHandle : torch::CustomClassHolder {
  int64_t E, H, I, quant_type;
  mi_moe_handle* h = nullptr;      // device weights (when a HIP device is present)
  mi_moe_cpu* cpu = nullptr;       // host engine, Q8_0 / Q4_0
  mi_moe_hybrid* hcpu = nullptr;   // W4A16 with every expert on the host executor
  bool keep_host = false;          // weights stored from host tensors also fill the host path
  bool last_cpu = false;           // the last forward ran on the host
  double last_cpu_ms = -1.0;

  // Int8-gemm/nanovllm_ops.cpp:28-30 (quant_type: 0 Q8_0, 1 Q4_0; 2 W4A16)
  MoEInferHandle(int64_t E_, int64_t H_, int64_t I_, int64_t qt) : E(E_), H(H_), I(I_), quant_type(qt) {
    TORCH_CHECK(qt >= 0 && qt <= 2, "quant_type must be 0 (Q8_0), 1 (Q4_0) or 2 (W4A16)");
    const bool dev = hip_device_present();
    if (dev) check_status(mi_moe_create(E, H, I, (int)qt, &h), "MoEInfer");
    const char* kh = getenv("MIMOE_HOST_WEIGHTS");
    keep_host = kh ? atoi(kh) != 0 : !dev;
    if (!dev) TORCH_CHECK(keep_host, "MoEInfer: no HIP device and MIMOE_HOST_WEIGHTS=0: nowhere to keep the weights");
  }
  ~MoEInferHandle() override {
    if (h) mi_moe_destroy(h);
    if (cpu) mi_moe_cpu_destroy(cpu);
    if (hcpu) mi_moe_hybrid_destroy(hcpu);
  }
  std::string get_quant_type() const {
    return quant_type == 1 ? "Q4_0" : (quant_type == 2 ? "W4A16" : "Q8_0");
  }
  int64_t info(int which) const { return which == 0 ? E : (which == 1 ? H : I); }
  mi_moe_handle* dev() const {
    TORCH_CHECK(h != nullptr, "MoEInfer: no HIP device for this call");
    return h;
  }
  // NANOVLLM_TP_SIZE / NANOVLLM_TP_THREADS_PER_NODE, when set, give the
  // reference's layout: tp shards over NUMA nodes, that many threads per node
  // (the reference's default tp of 2 fails on one-node hosts, so unset means
  // one shard per NUMA node here); otherwise MIMOE_CPU_THREADS /
  // OMP_NUM_THREADS threads over whole nodes.
  mi_moe_cpu* host_engine() {
    if (!cpu) {
      const int64_t tp = env_int("NANOVLLM_TP_SIZE"), per = env_int("NANOVLLM_TP_THREADS_PER_NODE");
      if (tp >= 0 || per >= 0) {
        TORCH_CHECK(tp != 0 && tp < 0x10000, "tp_size must be >= 1 (NANOVLLM_TP_SIZE=", tp, ")");
        check_status(mi_moe_cpu_create_numa(E, H, I, (int)quant_type, tp > 0 ? (int)tp : 0,
                                            per > 0 ? (int)std::min<int64_t>(per, 1 << 20) : 0, &cpu),
                     "MoEInfer (host)");
      } else {
        check_status(mi_moe_cpu_create(E, H, I, (int)quant_type, host_threads(), 0, &cpu), "MoEInfer (host)");
      }
    }
    return cpu;
  }
  mi_moe_hybrid* host_w4() {
    if (!hcpu) {
      std::vector<uint8_t> all((size_t)E, 1);
      check_status(mi_moe_hybrid_create(E, H, I, MI_MOE_W4A16, all.data(), std::min(host_threads(), 16), &hcpu),
                   "MoEInfer (host)");
    }
    return hcpu;
  }
};

at::Tensor contig(const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

void check_forward_tensors(const at::Tensor& hidden, const at::Tensor& topk_ids, const at::Tensor& topk_w,
                           const c10::intrusive_ptr<MoEInferHandle>& moe, const at::Tensor& out) {
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
}

void forward_into(const at::Tensor& hidden, const at::Tensor& topk_ids, const at::Tensor& topk_w,
                  const c10::intrusive_ptr<MoEInferHandle>& moe, at::Tensor& out) {
  TORCH_CHECK(hidden.is_cuda(), "moe_forward: expected HIP tensors here");
  check_forward_tensors(hidden, topk_ids, topk_w, moe, out);
  at::Tensor x = contig(hidden), ids = contig(topk_ids), w = contig(topk_w);
  check_status(mi_moe_forward(moe->dev(), x.data_ptr(), out.data_ptr(), w.data_ptr<float>(),
                              ids.data_ptr<int32_t>(), x.size(0), ids.size(1), act_code(x),
                              stream_of(x)),
               "moe_forward");
  moe->last_cpu = false;
}

// The CPU key: the host engine (Q8_0 / Q4_0: the reference algorithm,
// Int8-gemm/nanovllm_ops.cpp:219-236 -> moe_infer.cpp:430-456) or, for W4A16,
// every expert on the host executor.
void forward_into_cpu(const at::Tensor& hidden, const at::Tensor& topk_ids, const at::Tensor& topk_w,
                      const c10::intrusive_ptr<MoEInferHandle>& moe, at::Tensor& out) {
  check_forward_tensors(hidden, topk_ids, topk_w, moe, out);
  at::Tensor x = contig(hidden), ids = contig(topk_ids), w = contig(topk_w);
  const int64_t T = x.size(0), K = ids.size(1);
  if (moe->quant_type == 2) {
    TORCH_CHECK(moe->hcpu != nullptr, "moe_forward (CPU): no host weights; store the weights from host tensors "
                "(with MIMOE_HOST_WEIGHTS=1 where a HIP device is present)");
    at::Tensor part = at::empty({T, moe->H}, x.options().dtype(at::kFloat));
    const auto t0 = std::chrono::steady_clock::now();
    check_status(mi_moe_hybrid_host_forward(moe->hcpu, x.data_ptr(), w.data_ptr<float>(), ids.data_ptr<int32_t>(),
                                            T, K, act_code(x), part.data_ptr<float>()),
                 "moe_forward (CPU)");
    out.copy_(part);   // fp32 -> the hidden dtype, round to nearest even
    moe->last_cpu_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  } else {
    TORCH_CHECK(moe->cpu != nullptr, "moe_forward (CPU): no host weights; store the weights from host tensors "
                "(with MIMOE_HOST_WEIGHTS=1 where a HIP device is present)");
    check_status(mi_moe_cpu_forward(moe->cpu, x.data_ptr(), out.data_ptr(), w.data_ptr<float>(),
                                    ids.data_ptr<int32_t>(), T, K, act_code(x)),
                 "moe_forward (CPU)");
    double ms = -1.0;
    check_status(mi_moe_cpu_get_info(moe->cpu, nullptr, nullptr, nullptr, nullptr, nullptr, &ms), "get_info");
    moe->last_cpu_ms = ms;
  }
  moe->last_cpu = true;
}

// Int8-gemm/nanovllm_ops.cpp:219-236
at::Tensor moe_forward_hip(const at::Tensor& hidden, const at::Tensor& topk_ids,
                           const at::Tensor& topk_w,
                           const c10::intrusive_ptr<MoEInferHandle>& moe) {
  at::Tensor out = at::empty_like(hidden, hidden.options().memory_format(at::MemoryFormat::Contiguous));
  forward_into(hidden, topk_ids, topk_w, moe, out);
  return out;
}

// Int8-gemm/nanovllm_ops.cpp:219-236 (CPU key, :410-412)
at::Tensor moe_forward_cpu(const at::Tensor& hidden, const at::Tensor& topk_ids, const at::Tensor& topk_w,
                           const c10::intrusive_ptr<MoEInferHandle>& moe) {
  at::Tensor out = at::empty_like(hidden, hidden.options().memory_format(at::MemoryFormat::Contiguous));
  forward_into_cpu(hidden, topk_ids, topk_w, moe, out);
  return out;
}

void moe_forward_out_cpu(const at::Tensor& hidden, const at::Tensor& topk_ids, const at::Tensor& topk_w,
                         const c10::intrusive_ptr<MoEInferHandle>& moe, at::Tensor out) {
  forward_into_cpu(hidden, topk_ids, topk_w, moe, out);
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

// Router top-k + softmax on host tensors, the semantics of the device kernel
// (make_topk_from_logits_cpu, Int8-gemm/test/fused_moe_cpu.py:20-37): the K
// largest logits in descending order, equal logits lower expert id first,
// softmax over the K values (renormalize) or the full softmax gathered.
std::tuple<at::Tensor, at::Tensor> moe_topk_softmax_cpu(const at::Tensor& logits, int64_t top_k, bool renormalize) {
  TORCH_CHECK(logits.dim() == 2, "moe_topk_softmax: logits must be [T,E]");
  at::Tensor x = contig(logits).to(at::kFloat);
  const int64_t T = x.size(0), E = x.size(1);
  TORCH_CHECK(top_k >= 1 && top_k <= E && top_k <= 64, "top_k=", top_k, " must be in [1, min(E, 64)]");
  at::Tensor ids = at::empty({T, top_k}, x.options().dtype(at::kInt));
  at::Tensor w = at::empty({T, top_k}, x.options().dtype(at::kFloat));
  const float* g = x.data_ptr<float>();
  int32_t* oi = ids.data_ptr<int32_t>();
  float* ow = w.data_ptr<float>();
  check_status(mi_moe_cpu_topk_softmax(g, T, E, top_k, renormalize ? 1 : 0, oi, ow), "moe_topk_softmax");
  return {ids, w};
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
  check_status(mi_moe_forward_logits(moe->dev(), x.data_ptr(), out.data_ptr(), g.data_ptr(), logits_code(g),
                                     x.size(0), top_k, renormalize ? 1 : 0, act_code(x), nullptr, nullptr,
                                     stream_of(x)),
               "moe_forward_logits");
  moe->last_cpu = false;
  return out;
}

at::Tensor moe_forward_logits_cpu(const at::Tensor& hidden, const at::Tensor& router_logits, int64_t top_k,
                                  bool renormalize, const c10::intrusive_ptr<MoEInferHandle>& moe) {
  TORCH_CHECK(hidden.dim() == 2 && router_logits.dim() == 2 && router_logits.size(0) == hidden.size(0),
              "moe_forward_logits: expected hidden [T,H], router_logits [T,E]");
  TORCH_CHECK(router_logits.size(1) == moe->info(0), "router_logits has ", router_logits.size(1),
              " experts, handle has ", moe->info(0));
  auto picks = moe_topk_softmax_cpu(router_logits, top_k, renormalize);
  return moe_forward_cpu(hidden, std::get<0>(picks), std::get<1>(picks), moe);
}

int scale_code(const at::Tensor& d) {
  if (d.scalar_type() == at::kBFloat16) return MI_MOE_BF16;
  TORCH_CHECK(d.scalar_type() == at::kHalf, "scales must be float16 or bfloat16");
  return MI_MOE_F16;
}

}  // namespace

// The graph-mode context of the reference's device op
// (MoEGraphContext, Int8-gemm/nanovllm_ops.cpp:160-201): built for a number
// of tokens, a top_k and an activation dtype (0 fp16, 1 bf16).  Here it
// grows the handle's device workspace to that size up front, so calls of at
// most num_tokens tokens at this top_k allocate nothing and can be captured
// into a HIP graph.  Any top_k >= 1 is accepted (the reference: 1, 8, 10).
struct MoEGraphContext : torch::CustomClassHolder {
  int64_t num_tokens, top_k, dtype;
  MoEGraphContext(const c10::intrusive_ptr<MoEInferHandle>& moe, int64_t T, int64_t K, int64_t dt)
      : num_tokens(T), top_k(K), dtype(dt) {
    TORCH_CHECK(T >= 0 && K >= 1, "MoEGraphContext: num_tokens >= 0 and top_k >= 1");
    TORCH_CHECK(dt == 0 || dt == 1, "MoEGraphContext: dtype must be 0 (float16) or 1 (bfloat16)");
    if (moe->h) check_status(mi_moe_reserve(moe->h, T, K, (void*)c10::hip::getCurrentHIPStream().stream()),
                             "MoEGraphContext");
  }
};

// The reference's callback report thread (NpuCallbackManager,
// Int8-gemm/nanovllm_ops.cpp:38-138) serves its host-callback op; the device
// op here needs none, so the class holds nothing (constructible, for callers
// that create one).
struct NpuCallbackManager : torch::CustomClassHolder {
  NpuCallbackManager(int64_t, int64_t) {}
};

// moe_forward_npu_graph_out (Int8-gemm/nanovllm_ops.cpp:308-342,406): the
// layer into `out` for the context's shape.
void moe_forward_graph_out_impl(const at::Tensor& hidden, const at::Tensor& topk_ids, const at::Tensor& topk_w,
                                const c10::intrusive_ptr<MoEInferHandle>& moe,
                                const c10::intrusive_ptr<MoEGraphContext>& ctx, at::Tensor out) {
  TORCH_CHECK(hidden.dim() == 2 && hidden.size(0) <= ctx->num_tokens,
              "moe_forward_npu_graph_out: more tokens than the MoEGraphContext was built for");
  TORCH_CHECK(topk_ids.dim() == 2 && topk_ids.size(1) == ctx->top_k,
              "moe_forward_npu_graph_out: top_k differs from the MoEGraphContext's");
  TORCH_CHECK((ctx->dtype == 1) == (hidden.scalar_type() == at::kBFloat16),
              "moe_forward_npu_graph_out: hidden dtype differs from the MoEGraphContext's");
  if (hidden.is_cuda()) {
    forward_into(hidden, topk_ids, topk_w, moe, out);
  } else {
    moe_forward_out_cpu(hidden, topk_ids, topk_w, moe, out);
  }
}

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
             if (self->h)
               check_status(mi_moe_quantize_and_store_expert(self->h, expert_idx, proj, wc.data_ptr(),
                                                             wd, wc.is_cuda() ? 1 : 0, stream_of(wc)),
                            "quantize_and_store_expert");
             if (!wc.is_cuda() && self->keep_host)
               check_status(mi_moe_cpu_quantize_and_store_expert(self->host_engine(), expert_idx, proj,
                                                                 wc.data_ptr(), wd),
                            "quantize_and_store_expert (host)");
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
             if (self->h)
               check_status(mi_moe_store_quantized(self->h, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                                   d.data_ptr(), scale_code(b), dev ? 1 : 0, stream_of(a)),
                            "store_quantized_repack");
             if (!dev && self->keep_host)
               check_status(mi_moe_cpu_store_quantized(self->host_engine(), a.data_ptr(), b.data_ptr(),
                                                       c.data_ptr(), d.data_ptr(), scale_code(b)),
                            "store_quantized_repack (host)");
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
             if (self->h)
               check_status(mi_moe_store_awq(self->h, a.data_ptr<int32_t>(), b.data_ptr<int32_t>(),
                                             c.data_ptr(), d.data_ptr<int32_t>(), e.data_ptr<int32_t>(),
                                             f.data_ptr(), g, scale_code(c), dev ? 1 : 0, stream_of(a)),
                            "store_awq_repack");
             if (!dev && self->keep_host)
               check_status(mi_moe_hybrid_store_awq(self->host_w4(), a.data_ptr<int32_t>(), b.data_ptr<int32_t>(),
                                                    c.data_ptr(), d.data_ptr<int32_t>(), e.data_ptr<int32_t>(),
                                                    f.data_ptr(), g, scale_code(c), 0, nullptr),
                            "store_awq_repack (host)");
           })
      .def("get_last_run_time_ms",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) {
             if (self->last_cpu || !self->h) return self->last_cpu_ms;
             return mi_moe_get_last_run_time_ms(self->h);
           })
      .def("get_last_phase_times_ms",
           [](const c10::intrusive_ptr<MoEInferHandle>& self) {
             double ms[2] = {0.0, 0.0};
             const int n = mi_moe_get_last_phase_times_ms(self->dev(), ms, 2);
             TORCH_CHECK(n > 0, "get_last_phase_times_ms: ", mi_moe_last_error());
             return std::vector<double>(ms, ms + n);
           })
      .def("set_timing",
           [](const c10::intrusive_ptr<MoEInferHandle>& self, bool enable) {
             if (self->h) check_status(mi_moe_set_timing(self->h, enable ? 1 : 0), "set_timing");
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
  // the reference's device-op names (Int8-gemm/nanovllm_ops.cpp:393-407): the
  // stream op is moe_forward, the graph op writes into out
  m.class_<NpuCallbackManager>("NpuCallbackManager").def(torch::init<int64_t, int64_t>());
  m.class_<MoEGraphContext>("MoEGraphContext")
      .def(torch::init<const c10::intrusive_ptr<MoEInferHandle>&, int64_t, int64_t, int64_t>());
  m.def("moe_forward_npu_stream(Tensor hidden, Tensor topk_ids, Tensor topk_w, "
        "__torch__.torch.classes.nanovllm.MoEInfer moe) -> Tensor");
  m.def("moe_forward_npu_graph_out(Tensor hidden, Tensor topk_ids, Tensor topk_w, "
        "__torch__.torch.classes.nanovllm.MoEInfer moe, __torch__.torch.classes.nanovllm.MoEGraphContext ctx, "
        "Tensor(a!) out) -> ()");
  m.def("moe_forward_logits(Tensor hidden, Tensor router_logits, int top_k, bool renormalize, "
        "__torch__.torch.classes.nanovllm.MoEInfer moe) -> Tensor");
}

TORCH_LIBRARY_IMPL(nanovllm, CUDA, m) {
  m.impl("moe_forward", &moe_forward_hip);
  m.impl("moe_forward_out", &moe_forward_out_hip);
  m.impl("moe_topk_softmax", &moe_topk_softmax_hip);
  m.impl("moe_forward_logits", &moe_forward_logits_hip);
  m.impl("moe_forward_npu_stream", &moe_forward_hip);
  m.impl("moe_forward_npu_graph_out", &moe_forward_graph_out_impl);
}

TORCH_LIBRARY_IMPL(nanovllm, CPU, m) {
  m.impl("moe_forward", &moe_forward_cpu);
  m.impl("moe_forward_out", &moe_forward_out_cpu);
  m.impl("moe_topk_softmax", &moe_topk_softmax_cpu);
  m.impl("moe_forward_logits", &moe_forward_logits_cpu);
  m.impl("moe_forward_npu_stream", &moe_forward_cpu);
  m.impl("moe_forward_npu_graph_out", &moe_forward_graph_out_impl);
}
