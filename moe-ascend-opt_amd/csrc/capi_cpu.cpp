// capi_cpu.cpp -- the mi_moe_cpu_* entry points of the C ABI (include/mi_moe.h):
// the host engine of cpu_moe.cpp behind the same status / last-error
// convention as the device entry points.  Host-only C++ (no HIP calls).
#include <cstdio>
#include <cstring>
#include <exception>
#include <new>
#include <vector>

#include "cpu_moe.hpp"
#include "mi_moe.h"

#define MI_API extern "C" __attribute__((visibility("default")))

namespace mimoe {
int api_fail(int code, const char* msg);   // records the thread's last error (capi.hip)
}

struct mi_moe_cpu {
  mimoe_cpu::Engine* eng = nullptr;
};

namespace {

int fail(int code, const char* msg) { return mimoe::api_fail(code, msg); }

int check(const mi_moe_cpu* c) {
  if (!c || !c->eng) return fail(MI_MOE_EINVAL, "null cpu handle");
  return MI_MOE_OK;
}

}  // namespace

namespace {
template <class Make>
int cpu_create(int64_t E, int64_t H, int64_t I, int quant_type, mi_moe_cpu** out, Make make) {
  if (!out) return fail(MI_MOE_EINVAL, "out is null");
  *out = nullptr;
  if (E <= 0 || H <= 0 || I <= 0) return fail(MI_MOE_EINVAL, "E, H, I must be positive");
  if (quant_type != MI_MOE_Q8_0 && quant_type != MI_MOE_Q4_0)
    return fail(MI_MOE_EUNSUPPORTED, "the CPU engine runs Q8_0 and Q4_0 (quant_type 0 / 1)");
  if (H % 32 != 0 || I % 32 != 0) return fail(MI_MOE_EINVAL, "hidden and intermediate sizes must be multiples of 32");
  mi_moe_cpu* c = new (std::nothrow) mi_moe_cpu();
  if (!c) return fail(MI_MOE_EINVAL, "out of host memory");
  try {
    c->eng = make();
  } catch (const std::exception& ex) {
    delete c;
    return fail(MI_MOE_EINVAL, ex.what());
  }
  if (!c->eng->shape_ok()) {
    char msg[160];
    snprintf(msg, sizeof(msg), "intermediate size %lld does not split into %d shards of a multiple of 32",
             (long long)I, c->eng->tp());
    delete c->eng;
    delete c;
    return fail(MI_MOE_EINVAL, msg);
  }
  *out = c;
  return MI_MOE_OK;
}
}  // namespace

MI_API int mi_moe_cpu_create(int64_t E, int64_t H, int64_t I, int quant_type, int num_threads, int tp,
                             mi_moe_cpu** out) {
  if (num_threads < 0 || tp < 0) return fail(MI_MOE_EINVAL, "num_threads and tp must be >= 0");
  return cpu_create(E, H, I, quant_type, out,
                    [&] { return new mimoe_cpu::Engine(E, H, I, quant_type, num_threads, tp); });
}

MI_API int mi_moe_cpu_create_numa(int64_t E, int64_t H, int64_t I, int quant_type, int tp, int threads_per_node,
                                  mi_moe_cpu** out) {
  if (tp < 0 || threads_per_node < 0) return fail(MI_MOE_EINVAL, "tp and threads_per_node must be >= 0");
  return cpu_create(E, H, I, quant_type, out, [&] {
    return new mimoe_cpu::Engine(E, H, I, quant_type, mimoe_cpu::Engine::NumaLayout{}, tp, threads_per_node);
  });
}

MI_API int mi_moe_cpu_destroy(mi_moe_cpu* c) {
  if (!c) return MI_MOE_OK;
  delete c->eng;
  delete c;
  return MI_MOE_OK;
}

MI_API int mi_moe_cpu_store_quantized(mi_moe_cpu* c, const void* gate_up_qs, const void* gate_up_d,
                                      const void* down_qs, const void* down_d, int scale_dtype) {
  int rc = check(c);
  if (rc) return rc;
  if (scale_dtype != MI_MOE_F16 && scale_dtype != MI_MOE_BF16)
    return fail(MI_MOE_EINVAL, "scales must be float16 or bfloat16");
  if (!gate_up_qs || !gate_up_d || !down_qs || !down_d) return fail(MI_MOE_EINVAL, "null weight pointer");
  try {
    c->eng->store(gate_up_qs, (const uint16_t*)gate_up_d, down_qs, (const uint16_t*)down_d, scale_dtype);
  } catch (const std::exception& ex) {
    return fail(MI_MOE_EINVAL, ex.what());
  }
  return MI_MOE_OK;
}

MI_API int mi_moe_cpu_quantize_and_store_expert(mi_moe_cpu* c, int64_t expert, int proj, const void* w,
                                                int w_dtype) {
  int rc = check(c);
  if (rc) return rc;
  if (c->eng->quant() != MI_MOE_Q8_0)
    return fail(MI_MOE_EINVAL, "Q4_0 does not support online quantization. "
                               "Use store_quantized_repack() with pre-quantized weights.");
  if (expert < 0 || expert >= c->eng->E()) return fail(MI_MOE_EINVAL, "expert index out of range");
  if (proj < 0 || proj > 2) return fail(MI_MOE_EINVAL, "Unknown proj (0 gate_proj, 1 up_proj, 2 down_proj)");
  if (w_dtype < 0 || w_dtype > 2) return fail(MI_MOE_EINVAL, "weight must be float32, float16 or bfloat16");
  if (!w) return fail(MI_MOE_EINVAL, "null weight pointer");
  const int64_t N = proj == 2 ? c->eng->H() : c->eng->I(), K = proj == 2 ? c->eng->I() : c->eng->H();
  try {
    std::vector<float> wf((size_t)(N * K));
    for (int64_t i = 0; i < N * K; ++i) {
      wf[(size_t)i] = w_dtype == MI_MOE_F32 ? ((const float*)w)[i]
                                            : mimoe_cpu::half_to_f32(((const uint16_t*)w)[i], w_dtype);
    }
    c->eng->quantize_and_store(expert, proj, wf.data());
  } catch (const std::exception& ex) {
    return fail(MI_MOE_EINVAL, ex.what());
  }
  return MI_MOE_OK;
}

MI_API int mi_moe_cpu_forward(mi_moe_cpu* c, const void* x, void* y, const float* topk_w, const int32_t* topk_ids,
                              int64_t T, int64_t K, int act_dtype) {
  int rc = check(c);
  if (rc) return rc;
  if (!c->eng->loaded()) return fail(MI_MOE_ENOTLOADED, "weights not stored");
  if (act_dtype != MI_MOE_F16 && act_dtype != MI_MOE_BF16) return fail(MI_MOE_EINVAL, "hidden dtype must be fp16 or bf16");
  if (T < 0 || K < 1 || K > 64) return fail(MI_MOE_EINVAL, "bad T / top_k");
  if (T == 0) return MI_MOE_OK;
  if (!x || !y || !topk_w || !topk_ids) return fail(MI_MOE_EINVAL, "null data pointer");
  try {
    c->eng->forward((const uint16_t*)x, (uint16_t*)y, topk_w, topk_ids, T, K, act_dtype);
  } catch (const std::bad_alloc&) {
    return fail(MI_MOE_EINVAL, "out of host memory");
  } catch (const std::exception& ex) {
    return fail(MI_MOE_EINVAL, ex.what());
  }
  return MI_MOE_OK;
}

MI_API int mi_moe_cpu_get_info(mi_moe_cpu* c, int* threads, int* tp, int* isa, int* affinity_cpus,
                               int* affinity_nodes, double* last_ms) {
  int rc = check(c);
  if (rc) return rc;
  if (threads) *threads = c->eng->threads();
  if (tp) *tp = c->eng->tp();
  if (isa) *isa = (int)c->eng->isa();
  if (affinity_cpus) *affinity_cpus = c->eng->topology().affinity_cpus;
  if (affinity_nodes) *affinity_nodes = c->eng->topology().affinity_nodes;
  if (last_ms) *last_ms = c->eng->last_ms();
  return MI_MOE_OK;
}

MI_API int mi_moe_cpu_set_isa(mi_moe_cpu* c, int isa) {
  int rc = check(c);
  if (rc) return rc;
  if (isa < 0 || isa > 3 || !mimoe_cpu::isa_supported((mimoe_cpu::Isa)isa))
    return fail(MI_MOE_EUNSUPPORTED, "instruction set not available on this host");
  c->eng->set_isa((mimoe_cpu::Isa)isa);
  return MI_MOE_OK;
}

MI_API int mi_moe_cpu_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t K, int renormalize,
                                   int32_t* topk_ids, float* topk_w) {
  if (T < 0 || E < 1 || E > 512 || K < 1 || K > E || K > 64)
    return fail(MI_MOE_EINVAL, "bad T / E / top_k (E <= 512, 1 <= top_k <= min(E, 64))");
  if (T == 0) return MI_MOE_OK;
  if (!logits || !topk_ids || !topk_w) return fail(MI_MOE_EINVAL, "null pointer");
  mimoe_cpu::topk_softmax(logits, T, E, K, renormalize, topk_ids, topk_w);
  return MI_MOE_OK;
}

MI_API const char* mi_moe_cpu_isa_name(int isa) {
  return isa >= 0 && isa <= 3 ? mimoe_cpu::isa_name((mimoe_cpu::Isa)isa) : "unknown";
}
