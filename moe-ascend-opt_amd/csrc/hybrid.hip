// hybrid.hip -- the hybrid CPU-offload executor (mi_moe_hybrid_* in
// include/mi_moe.h).  Hot experts live compacted in a device handle; cold
// experts keep their weights in host memory and run on host threads: Q8_0 /
// Q4_0 on the host engine of the reference CPU algorithm (cpu_moe.cpp, VNNI /
// AVX2 int8 dots, bit-equal to the oracle), W4A16 on the host executor
// (host_experts.cpp, wire-format bytes).
//
// One forward on the caller's stream S, with a side stream D owned by the
// handle (both at the default priority):
//   S: event "in" ............ remap ids (cold -> -1, hot -> slot) -> device
//      forward of the hot experts into y ............ wait "part" -> y += part
//   D: wait "in" -> copy x, ids, topk_w to pinned host buffers -> host
//      callback: cold experts on the host pool, fp32 partial into pinned host
//      memory -> event "part"
// so the host experts overlap the device kernels; the add kernel reads the
// partial from the pinned buffer (no copy command).  The reference's NPU op
// does the whole layer in such a callback (moe_forward_npu_stream,
// Int8-gemm/nanovllm_ops.cpp:244-305); the per-expert split is its roadmap
// (README.md:124-134: hot experts resident in device memory, cold ones on the
// CPU).  The final y is round(round(y_hot) + y_cold): the device part is
// rounded to the activation dtype before the add.
#include <hip/hip_runtime.h>
#include <sched.h>

#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <vector>

#include "cpu_moe.hpp"
#include "host_experts.hpp"
#include "mi_moe.h"
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"

#define MI_API extern "C" __attribute__((visibility("default")))

namespace mimoe {
namespace {

int hfail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return api_fail(code, buf);
}

#define HCHK(expr)                                                                      \
  do {                                                                                  \
    hipError_t _e = (expr);                                                             \
    if (_e != hipSuccess)                                                               \
      return hfail(MI_MOE_EHIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), \
                   __FILE__, __LINE__);                                                 \
  } while (0)

struct DBuf {
  void* p = nullptr;
  size_t bytes = 0;
  hipError_t alloc(size_t b) {
    release();
    hipError_t e = hipMalloc(&p, b ? b : 256);
    if (e == hipSuccess) bytes = b; else p = nullptr;
    return e;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  void retire(std::vector<void*>& keep) {   // freed later by the owner
    if (p) keep.push_back(p);
    p = nullptr;
    bytes = 0;
  }
};

struct PinBuf {
  void* p = nullptr;
  size_t bytes = 0;
  hipError_t alloc(size_t b) {
    release();
    hipError_t e = hipHostMalloc(&p, b ? b : 256, hipHostMallocDefault);
    if (e == hipSuccess) bytes = b; else p = nullptr;
    return e;
  }
  void release() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    bytes = 0;
  }
  void retire(std::vector<void*>& keep) {   // freed later by the owner
    if (p) keep.push_back(p);
    p = nullptr;
    bytes = 0;
  }
};

__global__ void remap_ids_kernel(const int32_t* __restrict__ ids, const int32_t* __restrict__ slot, int n, int E,
                                 int32_t* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const int e = ids[i];
    out[i] = (unsigned)e < (unsigned)E ? slot[e] : -1;
  }
}

// y = round(y + part) (has_dev) or round(part): 4 values per thread (H % 32 == 0);
// part is pinned host memory written by the host callback before event "part".
template <int ACT>
__global__ void add_partial_kernel(uint16_t* __restrict__ y, const float* __restrict__ part, int64_t n4,
                                   int has_dev) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const f32x4_t p = reinterpret_cast<const f32x4_t*>(part)[i];
    u32x2_t v = has_dev ? reinterpret_cast<const u32x2_t*>(y)[i] : u32x2_t{0, 0};
    const float a0 = to_f32<ACT>(v.x & 0xffffu) + p.x, a1 = to_f32<ACT>(v.x >> 16) + p.y;
    const float a2 = to_f32<ACT>(v.y & 0xffffu) + p.z, a3 = to_f32<ACT>(v.y >> 16) + p.w;
    v.x = from_f32<ACT>(a0) | ((uint32_t)from_f32<ACT>(a1) << 16);
    v.y = from_f32<ACT>(a2) | ((uint32_t)from_f32<ACT>(a3) << 16);
    reinterpret_cast<u32x2_t*>(y)[i] = v;
  }
}

// The call's inputs into the pinned host buffers the host callback reads:
// hidden rows (nx16 16-byte words), ids and weights (n each).  Vector stores
// straight into host memory, so the side stream carries no copy commands.
__global__ void stage_inputs_kernel(const u32x4_t* __restrict__ x, int64_t nx16, const int32_t* __restrict__ ids,
                                    const float* __restrict__ w, int64_t n, u32x4_t* __restrict__ xh,
                                    int32_t* __restrict__ idsh, float* __restrict__ wh) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nx16; i += stride) xh[i] = x[i];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    idsh[i] = ids[i];
    wh[i] = w[i];
  }
}

// One CPU of the affinity mask is left to the runtime and the caller (which
// waits on the stream): with every CPU in the pool the host pass ran slower
// (W4A16 bs 8 on 16 CPUs: 0.24-0.27 ms with 16 threads, 0.20-0.21 with 15).
int default_threads() {
  cpu_set_t set;
  int n = 0;
  if (sched_getaffinity(0, sizeof(set), &set) == 0) n = CPU_COUNT(&set);
  if (n <= 0) {
    const unsigned hc = std::thread::hardware_concurrency();
    n = hc ? (int)hc : 1;
  }
  n = n > 1 ? n - 1 : 1;
  return n < 16 ? n : 16;
}

}  // namespace
}  // namespace mimoe

using namespace mimoe;

// Arguments of one host callback, with the staging buffers of its call (a
// graph replays the staging kernel on the buffers it captured, so the
// callback must read those, not the handle's current ones).  An eager call's
// context is freed by its callback; a captured call's context belongs to the
// graph (a HIP user object it retains: freed when the graph and its
// instances are), or, if that cannot be set up, to the handle (graph_ctx).
struct CallCtx {
  struct mi_moe_hybrid* hh;
  int64_t T, K;
  int act;
  std::chrono::steady_clock::time_point enqueued;
  bool eager;
  const uint16_t* x_h;
  const int32_t* ids_h;
  const float* w_h;
  float* part_h;
};

void delete_call_ctx(void* p) { delete static_cast<CallCtx*>(p); }

struct mi_moe_hybrid {
  int64_t E = 0, H = 0, I = 0;
  int quant = 0;
  int device = 0;
  bool loaded = false;
  mi_moe_handle* dev = nullptr;      // hot experts in slot order (null if all are cold)
  int64_t Eg = 0;
  std::vector<int32_t> slot_of;      // [E]: device slot, or -1 for a cold expert
  mimoe_host::ColdSet cold;
  std::unique_ptr<mimoe_host::Pool> pool;            // W4A16 host executor
  std::unique_ptr<mimoe_cpu::Engine> qeng;           // Q8_0 / Q4_0: the cold experts on the host engine
  std::vector<int32_t> qids;                         // host pass: ids mapped to cold experts (-1 otherwise)
  std::mutex host_mu;                // host forwards run one at a time
  DBuf slot_dev, ids_dev;
  PinBuf x_h, ids_h, w_h, part_h;
  int64_t cap_T = 0, cap_n = 0;
  hipStream_t side = nullptr;
  hipEvent_t ev_in = nullptr, ev_part = nullptr;
  std::atomic<double> last_host_ms{-1.0};
  std::atomic<double> last_queue_ms{-1.0};   // forward call -> start of its host callback
  std::atomic<int64_t> last_pairs{0};
  std::atomic<int> host_error{0};    // a host callback failed (reported by the next call)
  std::vector<std::unique_ptr<CallCtx>> graph_ctx;   // captured callbacks' arguments not owned by a graph
  // staging that was live during a capture is not freed when it grows but
  // kept until destroy (captured graphs hold its addresses)
  bool captured = false;
  std::vector<void*> retired_dev, retired_pin;
};

namespace {

void run_host(mi_moe_hybrid* hh, const uint16_t* x, int act, const int32_t* ids, const float* w, int64_t T,
              int64_t K, float* part) {
  std::lock_guard<std::mutex> lk(hh->host_mu);
  const auto t0 = std::chrono::steady_clock::now();
  int64_t np = 0;
  if (hh->quant == 2) {
    np = mimoe_host::forward(hh->cold, *hh->pool, x, act, ids, w, T, K, part);
  } else if (!hh->qeng) {   // no cold expert
    std::memset(part, 0, sizeof(float) * (size_t)(T * hh->H));
  } else {
    hh->qids.resize((size_t)(T * K));
    for (int64_t i = 0; i < T * K; ++i) {
      const int32_t e = ids[i];
      const int32_t c = (e >= 0 && e < hh->E) ? hh->cold.cold_of[(size_t)e] : -1;
      hh->qids[(size_t)i] = c;
      np += c >= 0;
    }
    hh->qeng->forward(x, nullptr, w, hh->qids.data(), T, K, act, part);
  }
  const auto t1 = std::chrono::steady_clock::now();
  hh->last_pairs.store(np);
  hh->last_host_ms.store(std::chrono::duration<double, std::milli>(t1 - t0).count());
}

// Stream host callback: no HIP calls in here.
void host_callback(void* arg) {
  CallCtx* ctx = static_cast<CallCtx*>(arg);
  std::unique_ptr<CallCtx> own(ctx->eager ? ctx : nullptr);
  mi_moe_hybrid* hh = ctx->hh;
  if (ctx->eager)
    hh->last_queue_ms.store(
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - ctx->enqueued).count());
  try {
    run_host(hh, ctx->x_h, ctx->act, ctx->ids_h, ctx->w_h, ctx->T, ctx->K, ctx->part_h);
  } catch (...) {   // poison the partial: the call's y must not look valid
    float* part = ctx->part_h;
    const float qnan = __builtin_nanf("");
    for (int64_t i = 0; i < ctx->T * hh->H; ++i) part[i] = qnan;
    hh->host_error.store(1);
  }
}

int check_h(const mi_moe_hybrid* hh) {
  if (!hh) return hfail(MI_MOE_EINVAL, "null hybrid handle");
  if (hh->device < 0) return hfail(MI_MOE_EHIP, "the handle was made without a HIP device");
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != hh->device)
    return hfail(MI_MOE_EINVAL, "current HIP device %d differs from the handle's device %d", cur, hh->device);
  return MI_MOE_OK;
}

int grow(mi_moe_hybrid* hh, int64_t T, int64_t n, hipStream_t st) {
  if (T <= hh->cap_T && n <= hh->cap_n) return MI_MOE_OK;
  int64_t capT = hh->cap_T ? hh->cap_T : 16, capn = hh->cap_n ? hh->cap_n : 128;
  while (capT < T) capT *= 2;
  while (capn < n) capn *= 2;
  HCHK(hipStreamSynchronize(st));   // queued work may still use the buffers
  HCHK(hipStreamSynchronize(hh->side));
  if (hh->captured) {   // and captured graphs
    for (PinBuf* b : {&hh->x_h, &hh->part_h, &hh->ids_h, &hh->w_h}) b->retire(hh->retired_pin);
    hh->ids_dev.retire(hh->retired_dev);
  }
  HCHK(hh->x_h.alloc((size_t)capT * hh->H * 2));
  HCHK(hh->part_h.alloc((size_t)capT * hh->H * sizeof(float)));
  HCHK(hh->ids_h.alloc((size_t)capn * sizeof(int32_t)));
  HCHK(hh->w_h.alloc((size_t)capn * sizeof(float)));
  HCHK(hh->ids_dev.alloc((size_t)capn * sizeof(int32_t)));
  hh->cap_T = capT;
  hh->cap_n = capn;
  return MI_MOE_OK;
}

// Split caller arrays [E, ...] (host or device memory) into the compacted hot
// arrays (device, slot order) and the cold experts' host copies.
int split_arrays(mi_moe_hybrid* hh, const void* const* src, int narr, int src_on_device, hipStream_t st,
                 std::vector<DBuf>& hot) {
  hot.resize((size_t)narr);
  bool copies = false;   // HIP copies issued (synchronized below)
  for (int a = 0; a < narr; ++a) {
    const size_t eb = mimoe_host::expert_bytes(hh->quant, hh->H, hh->I, a);
    if (!src[a]) return hfail(MI_MOE_EINVAL, "null weight pointer");
    if (hh->Eg > 0) HCHK(hot[a].alloc((size_t)hh->Eg * eb));
    hh->cold.arr[a].resize((size_t)hh->cold.Ec * eb);
    for (int64_t e = 0; e < hh->E; ++e) {
      const char* s = static_cast<const char*>(src[a]) + (size_t)e * eb;
      const int32_t sl = hh->slot_of[e], c = hh->cold.cold_of[e];
      if (sl >= 0) {
        HCHK(hipMemcpyAsync(static_cast<char*>(hot[a].p) + (size_t)sl * eb, s, eb,
                            src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
        copies = true;
      } else if (src_on_device) {
        HCHK(hipMemcpyAsync(hh->cold.arr[a].data() + (size_t)c * eb, s, eb, hipMemcpyDeviceToHost, st));
        copies = true;
      } else {
        std::memcpy(hh->cold.arr[a].data() + (size_t)c * eb, s, eb);
      }
    }
  }
  if (copies) HCHK(hipStreamSynchronize(st));
  return MI_MOE_OK;
}

// Store-time checks: a device is needed for device experts or device sources.
int check_store(const mi_moe_hybrid* hh, int src_on_device) {
  if (!hh) return hfail(MI_MOE_EINVAL, "null hybrid handle");
  if (hh->Eg == 0 && !src_on_device && hh->device < 0) return MI_MOE_OK;
  return check_h(hh);
}

}  // namespace

MI_API int mi_moe_hybrid_create(int64_t E, int64_t H, int64_t I, int quant_type, const uint8_t* host_mask,
                                int num_threads, mi_moe_hybrid** out) {
  if (!out) return hfail(MI_MOE_EINVAL, "out is null");
  *out = nullptr;
  if (!host_mask) return hfail(MI_MOE_EINVAL, "host_mask is null");
  if (num_threads < 0 || num_threads > 256) return hfail(MI_MOE_EINVAL, "num_threads must be in [0, 256]");
  int rc = check_dims(E, H, I, quant_type);   // the device handle's shape rules
  if (rc) return rc;
  mi_moe_hybrid* hh = new (std::nothrow) mi_moe_hybrid();
  if (!hh) return hfail(MI_MOE_EINVAL, "out of host memory");
  hh->E = E; hh->H = H; hh->I = I; hh->quant = quant_type;
  hh->slot_of.assign((size_t)E, -1);
  hh->cold.quant = quant_type;
  hh->cold.E = E; hh->cold.H = H; hh->cold.I = I;
  hh->cold.cold_of.assign((size_t)E, -1);
  for (int64_t e = 0; e < E; ++e) {
    if (host_mask[e]) hh->cold.cold_of[e] = (int32_t)hh->cold.Ec++;
    else hh->slot_of[e] = (int32_t)hh->Eg++;
  }
  auto bail = [&](int code) {
    mi_moe_hybrid_destroy(hh);
    return code;
  };
  // Without a HIP device only an all-host handle can be made; it serves
  // mi_moe_hybrid_host_forward (weights stored from host memory).
  if (hipGetDevice(&hh->device) != hipSuccess) {
    (void)hipGetLastError();
    hh->device = -1;
    if (hh->Eg > 0) return bail(hfail(MI_MOE_EHIP, "no HIP device for the %lld device experts", (long long)hh->Eg));
  }
  if (hh->Eg > 0) {
    rc = mi_moe_create(hh->Eg, H, I, quant_type, &hh->dev);
    if (rc) return bail(rc);
    if (hh->slot_dev.alloc((size_t)E * sizeof(int32_t)) != hipSuccess ||
        hipMemcpy(hh->slot_dev.p, hh->slot_of.data(), (size_t)E * sizeof(int32_t), hipMemcpyHostToDevice) != hipSuccess)
      return bail(hfail(MI_MOE_EHIP, "slot table upload failed"));
  }
  if (hh->device >= 0 &&
      (hipStreamCreateWithFlags(&hh->side, hipStreamNonBlocking) != hipSuccess ||
       hipEventCreateWithFlags(&hh->ev_in, hipEventDisableTiming) != hipSuccess ||
       hipEventCreateWithFlags(&hh->ev_part, hipEventDisableTiming) != hipSuccess))
    return bail(hfail(MI_MOE_EHIP, "stream / event creation failed"));
  try {
    const int nt = num_threads ? num_threads : default_threads();
    if (quant_type == MI_MOE_W4A16) hh->pool.reset(new mimoe_host::Pool(nt));
    else if (hh->cold.Ec > 0) {
      hh->qeng.reset(new mimoe_cpu::Engine(hh->cold.Ec, H, I, quant_type, nt, 1));
      hh->qeng->set_split_max(nt);   // few cold experts per call: every host thread on them
    }
  } catch (...) {
    return bail(hfail(MI_MOE_EINVAL, "host thread pool creation failed"));
  }
  *out = hh;
  return MI_MOE_OK;
}

MI_API int mi_moe_hybrid_destroy(mi_moe_hybrid* hh) {
  if (!hh) return MI_MOE_OK;
  if (hh->side) (void)hipStreamSynchronize(hh->side);
  if (hh->device >= 0) (void)hipDeviceSynchronize();
  if (hh->dev) mi_moe_destroy(hh->dev);
  hh->slot_dev.release(); hh->ids_dev.release();
  hh->x_h.release(); hh->ids_h.release(); hh->w_h.release(); hh->part_h.release();
  for (void* p : hh->retired_dev) (void)hipFree(p);
  for (void* p : hh->retired_pin) (void)hipHostFree(p);
  if (hh->ev_in) (void)hipEventDestroy(hh->ev_in);
  if (hh->ev_part) (void)hipEventDestroy(hh->ev_part);
  if (hh->side) (void)hipStreamDestroy(hh->side);
  delete hh;
  return MI_MOE_OK;
}

MI_API int mi_moe_hybrid_store_quantized(mi_moe_hybrid* hh, const void* gate_up_qs, const void* gate_up_d,
                                         const void* down_qs, const void* down_d, int scale_dtype,
                                         int src_on_device, void* stream) {
  int rc = check_store(hh, src_on_device);
  if (rc) return rc;
  if (hh->quant != MI_MOE_Q8_0 && hh->quant != MI_MOE_Q4_0)
    return hfail(MI_MOE_EINVAL, "store_quantized needs a Q8_0 or Q4_0 handle");
  if (scale_dtype != MI_MOE_F16 && scale_dtype != MI_MOE_BF16)
    return hfail(MI_MOE_EINVAL, "gate_up_d must be float16 or bfloat16");
  hipStream_t st = (hipStream_t)stream;
  const void* src[4] = {gate_up_qs, gate_up_d, down_qs, down_d};
  std::vector<DBuf> hot;
  rc = split_arrays(hh, src, 4, src_on_device, st, hot);
  if (rc) return rc;
  if (hh->dev) {
    rc = mi_moe_store_quantized(hh->dev, hot[0].p, hot[1].p, hot[2].p, hot[3].p, scale_dtype, 1, stream);
    if (rc) return rc;
  }
  if (hh->qeng) {   // the engine keeps its own packed copy; the wire bytes are not needed after
    try {
      hh->qeng->store(hh->cold.arr[0].data(), (const uint16_t*)hh->cold.arr[1].data(), hh->cold.arr[2].data(),
                      (const uint16_t*)hh->cold.arr[3].data(), scale_dtype);
    } catch (...) {
      return hfail(MI_MOE_EINVAL, "out of host memory");
    }
    for (auto& v : hh->cold.arr) std::vector<uint8_t>().swap(v);
  }
  hh->cold.scale_dtype = scale_dtype;
  hh->loaded = true;
  return MI_MOE_OK;
}

MI_API int mi_moe_hybrid_store_awq(mi_moe_hybrid* hh, const int32_t* w13_qweight, const int32_t* w13_qzeros,
                                   const void* w13_scales, const int32_t* w2_qweight, const int32_t* w2_qzeros,
                                   const void* w2_scales, int64_t group, int scale_dtype, int src_on_device,
                                   void* stream) {
  int rc = check_store(hh, src_on_device);
  if (rc) return rc;
  if (hh->quant != MI_MOE_W4A16) return hfail(MI_MOE_EINVAL, "store_awq needs a W4A16 handle (quant_type 2)");
  if (group != 128) return hfail(MI_MOE_EUNSUPPORTED, "W4A16 group size %lld unsupported (128 only)", (long long)group);
  if (scale_dtype != MI_MOE_F16 && scale_dtype != MI_MOE_BF16)
    return hfail(MI_MOE_EINVAL, "scale dtype must be fp16 or bf16");
  hipStream_t st = (hipStream_t)stream;
  const void* src[6] = {w13_qweight, w13_qzeros, w13_scales, w2_qweight, w2_qzeros, w2_scales};
  std::vector<DBuf> hot;
  rc = split_arrays(hh, src, 6, src_on_device, st, hot);
  if (rc) return rc;
  if (hh->dev) {
    rc = mi_moe_store_awq(hh->dev, (const int32_t*)hot[0].p, (const int32_t*)hot[1].p, hot[2].p,
                          (const int32_t*)hot[3].p, (const int32_t*)hot[4].p, hot[5].p, group, scale_dtype, 1,
                          stream);
    if (rc) return rc;
  }
  hh->cold.scale_dtype = scale_dtype;
  try {
    mimoe_host::prepare_host_layouts(hh->cold);
  } catch (...) {
    return hfail(MI_MOE_EINVAL, "out of host memory");
  }
  hh->loaded = true;
  return MI_MOE_OK;
}

MI_API int mi_moe_hybrid_forward(mi_moe_hybrid* hh, const void* x, void* y, const float* topk_w,
                                 const int32_t* topk_ids, int64_t T, int64_t K, int act_dtype, void* stream) {
  int rc = check_h(hh);
  if (rc) return rc;
  if (!hh->loaded) return hfail(MI_MOE_ENOTLOADED, "weights not stored");
  if (hh->host_error.exchange(0)) return hfail(MI_MOE_EDEVICE, "a previous host expert pass failed (out of host memory)");
  if (act_dtype != MI_MOE_F16 && act_dtype != MI_MOE_BF16) return hfail(MI_MOE_EINVAL, "hidden dtype must be fp16 or bf16");
  if (T < 0 || K < 1 || K > 64) return hfail(MI_MOE_EINVAL, "bad T=%lld / top_k=%lld", (long long)T, (long long)K);
  if (T == 0) return MI_MOE_OK;
  if (T * K > ((int64_t)1 << 24)) return hfail(MI_MOE_EINVAL, "T*top_k too large");
  if (!x || !y || !topk_w || !topk_ids) return hfail(MI_MOE_EINVAL, "null data pointer");
  if (((uintptr_t)x & 15u) || ((uintptr_t)y & 15u)) return hfail(MI_MOE_EINVAL, "hidden/out must be 16-byte aligned");
  if (hh->cold.Ec == 0) return mi_moe_forward(hh->dev, x, y, topk_w, topk_ids, T, K, act_dtype, stream);
  hipStream_t st = (hipStream_t)stream;
  const int64_t n = T * K, H = hh->H;
  // Under graph capture nothing may synchronize or allocate: the staging
  // buffers (and the device handle's workspace) must already hold this call,
  // i.e. a call of at least this size was made before the capture.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HCHK(hipStreamIsCapturing(st, &cap));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  if (capturing && (T > hh->cap_T || n > hh->cap_n))
    return hfail(MI_MOE_EINVAL, "hybrid call of T=%lld, %lld pairs under graph capture needs larger staging buffers: "
                 "make one call of this size before capturing", (long long)T, (long long)n);
  rc = grow(hh, T, n, st);
  if (rc) return rc;
  // inputs to the host buffers on the caller's stream (after the previous
  // call's add kernel, so after its host pass), then the side stream: cold
  // experts in a host callback, the partial back to the device.  Copy
  // commands on the side stream were measured to hold the caller's thread
  // until the previous callback had run; a kernel does not.
  const int64_t nx16 = T * H * 2 / 16;
  const int64_t nmax = nx16 > n ? nx16 : n;
  const int sgrid = (int)((nmax + 255) / 256 < 1024 ? (nmax + 255) / 256 : 1024);
  hipLaunchKernelGGL(stage_inputs_kernel, dim3(sgrid), dim3(256), 0, st, (const u32x4_t*)x, nx16, topk_ids, topk_w, n,
                     (u32x4_t*)hh->x_h.p, (int32_t*)hh->ids_h.p, (float*)hh->w_h.p);
  HCHK(hipGetLastError());
  HCHK(hipEventRecord(hh->ev_in, st));
  HCHK(hipStreamWaitEvent(hh->side, hh->ev_in, 0));
  const CallCtx proto{hh, T, K, act_dtype, std::chrono::steady_clock::now(), !capturing,
                      (const uint16_t*)hh->x_h.p, (const int32_t*)hh->ids_h.p, (const float*)hh->w_h.p,
                      (float*)hh->part_h.p};
  CallCtx* ctx = new (std::nothrow) CallCtx(proto);
  if (!ctx) return hfail(MI_MOE_EINVAL, "out of host memory");
  if (capturing) {
    hh->captured = true;
    // the graph being captured owns the context (a user object it retains);
    // failing that, the handle keeps it
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipGraph_t graph = nullptr;
    hipUserObject_t obj = nullptr;
    bool owned = false;
    if (hipStreamGetCaptureInfo_v2(st, &cs, nullptr, &graph, nullptr, nullptr) == hipSuccess && graph &&
        hipUserObjectCreate(&obj, ctx, delete_call_ctx, 1, hipUserObjectNoDestructorSync) == hipSuccess) {
      owned = hipGraphRetainUserObject(graph, obj, 1, hipGraphUserObjectMove) == hipSuccess;
      if (!owned) {
        (void)hipUserObjectRelease(obj, 1);   // deletes ctx
        ctx = new (std::nothrow) CallCtx(proto);
        if (!ctx) return hfail(MI_MOE_EINVAL, "out of host memory");
      }
    }
    (void)hipGetLastError();
    if (!owned) hh->graph_ctx.emplace_back(ctx);
  }
  hipError_t e = hipLaunchHostFunc(hh->side, host_callback, ctx);
  if (e != hipSuccess) {
    if (!capturing) delete ctx;   // a captured call's context stays with its owner
    return hfail(MI_MOE_EHIP, "hipLaunchHostFunc failed: %s", hipGetErrorString(e));
  }
  HCHK(hipEventRecord(hh->ev_part, hh->side));
  // caller stream: the hot experts on the device
  if (hh->dev) {
    const int blocks = (int)((n + 255) / 256);
    hipLaunchKernelGGL(remap_ids_kernel, dim3(blocks), dim3(256), 0, st, topk_ids, (const int32_t*)hh->slot_dev.p,
                       (int)n, (int)hh->E, (int32_t*)hh->ids_dev.p);
    HCHK(hipGetLastError());
    rc = mi_moe_forward(hh->dev, x, y, topk_w, (const int32_t*)hh->ids_dev.p, T, K, act_dtype, stream);
    if (rc) return rc;
  }
  HCHK(hipStreamWaitEvent(st, hh->ev_part, 0));
  const int64_t n4 = T * H / 4;
  const int grid = (int)((n4 + 255) / 256 < 2048 ? (n4 + 255) / 256 : 2048);
  if (act_dtype == MI_MOE_BF16)
    hipLaunchKernelGGL(add_partial_kernel<1>, dim3(grid), dim3(256), 0, st, (uint16_t*)y,
                       (const float*)hh->part_h.p, n4, hh->dev ? 1 : 0);
  else
    hipLaunchKernelGGL(add_partial_kernel<0>, dim3(grid), dim3(256), 0, st, (uint16_t*)y,
                       (const float*)hh->part_h.p, n4, hh->dev ? 1 : 0);
  HCHK(hipGetLastError());
  return MI_MOE_OK;
}

MI_API int mi_moe_hybrid_host_forward(mi_moe_hybrid* hh, const void* x_host, const float* topk_w_host,
                                      const int32_t* topk_ids_host, int64_t T, int64_t K, int act_dtype,
                                      float* y_part_host) {
  if (!hh) return hfail(MI_MOE_EINVAL, "null hybrid handle");
  if (!hh->loaded) return hfail(MI_MOE_ENOTLOADED, "weights not stored");
  if (act_dtype != MI_MOE_F16 && act_dtype != MI_MOE_BF16) return hfail(MI_MOE_EINVAL, "hidden dtype must be fp16 or bf16");
  if (T < 0 || K < 1 || K > 64) return hfail(MI_MOE_EINVAL, "bad T=%lld / top_k=%lld", (long long)T, (long long)K);
  if (T == 0) return MI_MOE_OK;
  if (!x_host || !topk_w_host || !topk_ids_host || !y_part_host) return hfail(MI_MOE_EINVAL, "null data pointer");
  try {
    run_host(hh, (const uint16_t*)x_host, act_dtype, topk_ids_host, topk_w_host, T, K, y_part_host);
  } catch (...) {
    return hfail(MI_MOE_EINVAL, "out of host memory");
  }
  return MI_MOE_OK;
}

MI_API int mi_moe_hybrid_get_stats(mi_moe_hybrid* hh, int64_t* device_experts, int64_t* host_experts,
                                   int64_t* host_weight_bytes, double* last_host_ms, int64_t* last_host_pairs,
                                   double* last_queue_ms) {
  if (!hh) return hfail(MI_MOE_EINVAL, "null hybrid handle");
  if (device_experts) *device_experts = hh->Eg;
  if (host_experts) *host_experts = hh->cold.Ec;
  if (host_weight_bytes) {   // wire-format bytes of the cold experts once stored
    int64_t b = 0;
    for (int a = 0; hh->loaded && a < mimoe_host::num_arrays(hh->quant); ++a)
      b += hh->cold.Ec * (int64_t)mimoe_host::expert_bytes(hh->quant, hh->H, hh->I, a);
    *host_weight_bytes = b;
  }
  if (last_host_ms) *last_host_ms = hh->last_host_ms.load();
  if (last_host_pairs) *last_host_pairs = hh->last_pairs.load();
  if (last_queue_ms) *last_queue_ms = hh->last_queue_ms.load();
  return MI_MOE_OK;
}
