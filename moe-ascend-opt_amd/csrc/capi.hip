// capi.hip -- the C ABI of libmimoe.so (include/mi_moe.h): handle lifetime,
// weight ingestion (wire layout -> device tile layout), the fused forward,
// and the standalone routing / quantization entry points.
//
// Host-side counterpart of MoEInfer (Int8-gemm/moe_infer.{h,cpp}) and the op
// body of moe_forward (Int8-gemm/nanovllm_ops.cpp:219-236).  No exceptions
// cross the ABI: every entry point returns a status and records a message
// readable with mi_moe_last_error().
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "mi_moe.h"
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"
#include "mi_moe_sched.hpp"

#define MI_API extern "C" __attribute__((visibility("default")))

namespace mimoe {
constexpr size_t kXAllBytes = 16384; // hidden rows phase 1 copies whole on the decode path
constexpr int kDecodeCols = 4;       // phase-1 pass width on the decode path

// kernels / launchers defined in the other translation units
hipError_t launch_route_global(const int32_t*, int, int, int, const RouteGlobal&, hipStream_t, int, int);
hipError_t launch_combine(const float*, const float*, const int32_t*, void*, int, int, int, int, int,
                          hipStream_t, bool);
hipError_t launch_awq_repack_all(const int32_t*, const int32_t*, const uint16_t*, const int32_t*,
                                 const int32_t*, const uint16_t*, void*, unsigned char*, void*,
                                 unsigned char*, int, int, int, hipStream_t);
hipError_t launch_quant_act(const void*, int, int64_t, int64_t, int8_t*, float*, hipStream_t);
W4Plan w4a16_plan(int, int);
hipError_t launch_w4a16(const W4Args&, const W4Plan&, int, int, int, hipStream_t, hipEvent_t);
hipError_t launch_w4a16_gemm(const W4Args&, int, int, hipStream_t, hipEvent_t);
W4FusedPlan w4a16_fused_plan(int, int, int, int, int, int, int);
hipError_t launch_w4a16_fused(const W4Args&, const W4FusedPlan&, int, hipStream_t);
hipError_t launch_qint(const QArgs&, int, int, int, int, int, bool, hipStream_t);
size_t q_fused_lds(int, int, int, int, int);
hipError_t launch_q_fused(const QArgs&, int, int, int, hipStream_t);
hipError_t launch_qint_gemm(const QArgs&, int, int, int, hipStream_t);
hipError_t launch_quant_route(const void*, int, int64_t, int64_t, int8_t*, float*, const int32_t*, int, int, int,
                              const RouteGlobal&, hipStream_t, int);
hipError_t launch_topk_softmax(const void*, int, int, int, int, int, int32_t*, float*, hipStream_t);
hipError_t launch_q_repack(int, const void*, const uint16_t*, void*, uint16_t*, int, int, int, int,
                           int, hipStream_t);
hipError_t launch_q8_online_quant(const void*, int, int, int, int, int, int, void*, uint16_t*,
                                  hipStream_t);
hipError_t launch_q_block_dots(int, const void*, const int8_t*, int32_t*, int, int, int, int, int,
                               int, int, hipStream_t);
hipError_t launch_q_mfma_block_check(int, int, const void*, const uint16_t*, const int8_t*, int32_t*, float*,
                                     int, int, int, int, int, int, int, hipStream_t);
}  // namespace mimoe

using namespace mimoe;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIPCHK(expr)                                                                   \
  do {                                                                                 \
    hipError_t _e = (expr);                                                            \
    if (_e != hipSuccess)                                                              \
      return fail(MI_MOE_EHIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), \
                  __FILE__, __LINE__);                                                 \
  } while (0)

struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  // hand the allocation over to `keep` (freed later) instead of freeing it
  void retire(std::vector<void*>& keep) {
    if (p) keep.push_back(p);
    p = nullptr;
    bytes = 0;
  }
  hipError_t alloc(size_t b) {
    release();
    if (b == 0) b = 256;
    hipError_t e = hipMalloc(&p, b);
    if (e == hipSuccess) bytes = b;
    return e;
  }
};

// Scoped temporary device copy of a caller buffer (host or device source).
struct Staged {
  const void* ptr = nullptr;
  DevBuf own;
  hipError_t stage(const void* src, size_t bytes, int on_device, hipStream_t st) {
    if (on_device) { ptr = src; return hipSuccess; }
    hipError_t e = own.alloc(bytes);
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(own.p, src, bytes, hipMemcpyHostToDevice, st);
    ptr = own.p;
    return e;
  }
  ~Staged() { own.release(); }
};

}  // namespace

struct mi_moe_handle {
  int64_t E = 0, H = 0, I = 0;
  int quant = 0;
  int scale_dtype = 0;
  int group = 128;
  int device = 0;
  int num_cu = 0;
  bool loaded = false;
  bool timing = false;   // HIP events around each forward only when asked (mi_moe_set_timing)
  bool timed_once = false;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  hipEvent_t evmid = nullptr;   // between the gate_up and down launches (W4A16)
  bool mid_recorded = false;
  // weights (device layout)
  DevBuf w13, w13_s, w13_z, w2, w2_s, w2_z;
  DevBuf tact;   // tagged_act_bytes(I): act hand-over units of the one-launch decode kernel
  // workspace
  int64_t cap_T = 0, cap_n = 0;
  DevBuf act, eout, act_d, r_counts, r_starts, r_active, r_tok, r_scat, r_U, r_tiles, r_ntiles;
  DevBuf xq, xd;   // Q8_0 activations of the grouped-GEMM path
  DevBuf r_chunk;  // per-chunk expert counts of the multi-workgroup routing
  DevBuf r_rids, r_rw;   // router top-k ids / weights of mi_moe_forward_logits
  int64_t cap_r = 0;     // capacity of r_rids / r_rw in (t, k) entries
  // A call captured into a HIP graph bakes the workspace addresses into the
  // graph: workspace that was live during a capture is not freed when it
  // grows but kept here until mi_moe_destroy, so such graphs stay valid.
  bool captured = false;   // a forward on this handle has been captured
  std::vector<void*> retired;
};

namespace {

int check_handle(const mi_moe_handle* h) {
  if (!h) return fail(MI_MOE_EINVAL, "null handle");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(MI_MOE_EHIP, "hipGetDevice failed");
  if (dev != h->device)
    return fail(MI_MOE_EINVAL, "current HIP device %d differs from the handle's device %d", dev,
                h->device);
  return MI_MOE_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int ensure_workspace(mi_moe_handle* h, int64_t T, int64_t n, hipStream_t st) {
  if (h->r_U.p == nullptr) {
    HIPCHK(h->r_counts.alloc((size_t)h->E * sizeof(int32_t)));
    HIPCHK(h->r_starts.alloc((size_t)(h->E + 1) * sizeof(int32_t)));
    HIPCHK(h->r_active.alloc((size_t)h->E * sizeof(int32_t)));
    HIPCHK(h->r_U.alloc(sizeof(int32_t)));
    HIPCHK(h->r_ntiles.alloc(sizeof(int32_t)));
  }
  if (T <= h->cap_T && n <= h->cap_n) return MI_MOE_OK;
  int64_t capT = h->cap_T ? h->cap_T : 16;
  while (capT < T) capT *= 2;
  int64_t capn = h->cap_n ? h->cap_n : 128;
  while (capn < n) capn *= 2;
  // buffers may be in use by queued work on this stream, or by captured graphs
  HIPCHK(hipStreamSynchronize(st));
  if (h->captured) {
    for (DevBuf* b : {&h->act, &h->act_d, &h->eout, &h->r_tok, &h->r_scat, &h->r_tiles, &h->r_chunk, &h->xq, &h->xd})
      b->retire(h->retired);
  }
  HIPCHK(h->act.alloc((size_t)capn * h->I * 2));
  HIPCHK(h->act_d.alloc((size_t)capn * (h->I / 32) * sizeof(float)));
  HIPCHK(h->eout.alloc((size_t)capn * h->H * sizeof(float)));
  HIPCHK(h->r_tok.alloc((size_t)capn * sizeof(int32_t)));
  HIPCHK(h->r_scat.alloc((size_t)capn * sizeof(int32_t)));
  HIPCHK(h->r_tiles.alloc((size_t)gemm_tiles_max(capn, (int)h->E) * 4 * sizeof(int32_t)));
  HIPCHK(h->r_chunk.alloc((size_t)route_chunks((int)capn) * h->E * sizeof(int32_t)));
  if (h->quant != MI_MOE_W4A16) {
    HIPCHK(h->xq.alloc((size_t)capT * h->H));
    HIPCHK(h->xd.alloc((size_t)capT * (h->H / 32) * sizeof(float)));
  }
  h->cap_T = capT;
  h->cap_n = capn;
  return MI_MOE_OK;
}

RouteGlobal route_view(mi_moe_handle* h) {
  RouteGlobal rg;
  rg.counts = (int32_t*)h->r_counts.p;
  rg.starts = (int32_t*)h->r_starts.p;
  rg.active = (int32_t*)h->r_active.p;
  rg.tok = (int32_t*)h->r_tok.p;
  rg.scat = (int32_t*)h->r_scat.p;
  rg.U = (int32_t*)h->r_U.p;
  rg.tiles = (int32_t*)h->r_tiles.p;
  rg.ntiles = (int32_t*)h->r_ntiles.p;
  rg.chunk = (int32_t*)h->r_chunk.p;
  return rg;
}

// Device workspace of one forward call: the handle's grown buffers
// (mi_moe_forward) or slices of the no-alloc scratch (mi_moe_forward_noalloc).
struct Work {
  void* act = nullptr;      // [n, I] act dtype (W4A16) or int8 (Q8_0 / Q4_0)
  float* act_d = nullptr;   // [n, I/32] intermediate Q8_0 scales
  float* eout = nullptr;    // [n, H] per-pair outputs (paths with a separate combine)
  int8_t* xq = nullptr;     // [T, H] Q8_0 activations (int8 grouped GEMMs)
  float* xd = nullptr;      // [T, H/32]
  unsigned long long* tact = nullptr; // tagged act units of the one-launch decode kernel
  RouteGlobal rg{};
};

// ---------------------------------------------------------------- no-alloc scratch
// The workspace of mi_moe_forward_noalloc: one array per GPU, held from the
// code object's load until the process ends.  Host code never names it
// directly: its device address comes from hipGetSymbolAddress, once per
// device at mi_moe_create (with that device current), and is kept in
// g_scratch_ptr.  Every no-alloc call on a GPU uses the same array.
constexpr size_t kNoAllocScratchBytes = (size_t)MI_MOE_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// mi_moe_route's per-device routing arrays (grown on demand, kept until the
// process ends; calls on one process serialize on the mutex).
std::mutex g_route_mu;
DevBuf g_route_buf[kMaxDevices];

int init_scratch(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return MI_MOE_OK;   // the no-alloc entry point then reports it
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev]) return MI_MOE_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return fail(MI_MOE_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
  // the one-launch decode units at the head start zeroed (no dispatch has tag 0)
  const hipError_t ez = hipMemset(p, 0, tagged_act_bytes(kTagActMaxI));
  if (ez != hipSuccess)
    return fail(MI_MOE_EHIP, "clearing the no-alloc scratch head failed on device %d: %s", dev, hipGetErrorString(ez));
  g_scratch_ptr[dev] = p;
  return MI_MOE_OK;
}

void* scratch_of(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return g_scratch_ptr[dev];
}

// Slices of one call's workspace laid out from base (256-byte aligned);
// returns the bytes taken.  With base == nullptr it only measures.
size_t carve_work(unsigned char* base, const mi_moe_handle* h, int64_t T, int64_t n, bool need_eout, Work& w) {
  size_t off = tagged_act_bytes(kTagActMaxI);   // the head holds the one-launch decode units
  w.tact = base ? (unsigned long long*)base : nullptr;
  auto take = [&](size_t bytes) -> void* {
    void* p = base ? base + off : nullptr;
    off += (bytes + 255) & ~(size_t)255;
    return p;
  };
  const int64_t E = h->E, H = h->H, I = h->I;
  w.rg.counts = (int32_t*)take((size_t)E * 4);
  w.rg.starts = (int32_t*)take((size_t)(E + 1) * 4);
  w.rg.active = (int32_t*)take((size_t)E * 4);
  w.rg.U = (int32_t*)take(4);
  w.rg.ntiles = (int32_t*)take(4);
  w.rg.tok = (int32_t*)take((size_t)n * 4);
  w.rg.scat = (int32_t*)take((size_t)n * 4);
  w.rg.tiles = (int32_t*)take((size_t)gemm_tiles_max(n, (int)E) * 16);
  w.rg.chunk = (int32_t*)take((size_t)route_chunks((int)n) * E * 4);
  w.act = take((size_t)n * I * 2);
  w.act_d = (float*)take((size_t)n * (I / 32) * 4);
  w.eout = need_eout ? (float*)take((size_t)n * H * 4) : nullptr;
  if (h->quant != MI_MOE_W4A16) {
    w.xq = (int8_t*)take((size_t)T * H);
    w.xd = (float*)take((size_t)T * (H / 32) * 4);
  }
  return off;
}

// The call's workspace: the handle's buffers (grown on demand; growth
// synchronizes the stream) or, for the no-alloc entry point, the scratch.
int get_work(mi_moe_handle* h, int64_t T, int64_t n, bool need_eout, bool noalloc, hipStream_t st, Work& w) {
  if (!noalloc) {
    const int rc = ensure_workspace(h, T, n, st);
    if (rc) return rc;
    w.act = h->act.p;
    w.act_d = (float*)h->act_d.p;
    w.eout = (float*)h->eout.p;
    w.xq = (int8_t*)h->xq.p;
    w.xd = (float*)h->xd.p;
    w.tact = (unsigned long long*)h->tact.p;
    w.rg = route_view(h);
    return MI_MOE_OK;
  }
  unsigned char* base = (unsigned char*)scratch_of(h->device);
  if (!base) return fail(MI_MOE_EHIP, "no-alloc scratch unavailable on device %d", h->device);
  const size_t need = carve_work(nullptr, h, T, n, need_eout, w);
  if (need > kNoAllocScratchBytes)
    return fail(MI_MOE_EINVAL, "this call (T=%lld, %lld routed pairs) needs %zu bytes of workspace; "
                "mi_moe_forward_noalloc holds at most %zu (use mi_moe_forward)", (long long)T, (long long)n,
                need, kNoAllocScratchBytes);
  carve_work(base, h, T, n, need_eout, w);
  return MI_MOE_OK;
}

void fill_sched(mi_moe_handle* h, SchedArgs& c, const void* x, void* y, const float* tw,
                const int32_t* ids, int64_t T, int64_t K, const Work& w) {
  c.x = (const uint16_t*)x;
  c.y = (uint16_t*)y;
  c.tw = tw;
  c.ids = ids;
  c.T = (int)T; c.K = (int)K; c.E = (int)h->E; c.H = (int)h->H; c.I = (int)h->I;
  c.n = (int)(T * K);
  c.route_global = c.n > kRouteLdsMax;
  c.rg = w.rg;
  c.eout = w.eout;
}

int forward_w4a16(mi_moe_handle* h, const void* x, void* y, const float* tw, const int32_t* ids,
                  int64_t T, int64_t K, int act, bool noalloc, hipStream_t st) {
  const int64_t n = T * K;
  // decode path: T*K <= 64 pairs, at most kDownMaxK experts per token (a
  // wave each in the down kernel), and both kernels' LDS fits; otherwise the
  // sorted path (mi_moe_create checked that it fits)
  const size_t lmax = device_max_lds();
  const bool decode = n <= 64 && K <= kDownMaxK && w4_decode_fits((int)h->H, (int)h->I, (int)K, lmax);
  Work w;
  int rc = get_work(h, T, n, !decode, noalloc, st, w);
  if (rc) return rc;
  W4Args a;
  std::memset(&a, 0, sizeof(a));
  fill_sched(h, a.c, x, y, tw, ids, T, K, w);
  a.w13 = h->w13.p; a.w13_m = (const unsigned char*)h->w13_s.p;
  a.w2 = h->w2.p; a.w2_m = (const unsigned char*)h->w2_s.p;
  a.act = (uint16_t*)w.act;
  a.sdt = h->scale_dtype;
  a.tact = w.tact;
  hipEvent_t mid = h->timing && !noalloc ? h->evmid : nullptr;
  if (decode) {
    // phase 1 copies the hidden rows of every token when they are few
    const int nw1 = w4_p1_waves(n, (int)h->H);
    a.x_all = (size_t)T * h->H * 2 <= kXAllBytes && w4_p1_lds_bytes((int)h->H, (int)T, 1, nw1) <= lmax;
    // an expert rarely gets more than a few of the T tokens; a narrow pass
    // keeps the LDS small (occupancy), extra columns take another pass
    a.p1_cols = (int)(T < kDecodeCols ? T : kDecodeCols);
    while (!a.x_all && a.p1_cols > 1 && w4_p1_lds_bytes((int)h->H, a.p1_cols, 1, nw1) > lmax) --a.p1_cols;
    // one launch (gate_up hands act to down inside it) for top-k <= 8
    const W4FusedPlan fp = w4a16_fused_plan((int)T, (int)K, (int)h->H, (int)h->I, a.x_all, a.p1_cols, h->num_cu);
    if (fp.ok && a.tact) {
      HIPCHK(launch_w4a16_fused(a, fp, act, st));
      return MI_MOE_OK;
    }
    const W4Plan plan = w4a16_plan((int)h->H, (int)h->I);
    HIPCHK(launch_w4a16(a, plan, act, (int)(n * (h->I / 16)), (int)(T * (h->H / 16)), st, mid));
    if (!noalloc) h->mid_recorded = mid != nullptr;   // a no-alloc call leaves the timed call's record
    return MI_MOE_OK;
  }
  // sorted path: routing with row tiles, the two grouped GEMMs, the combine
  HIPCHK(launch_route_global(ids, (int)n, (int)K, (int)h->E, a.c.rg, st, 0, 1));
  HIPCHK(launch_w4a16_gemm(a, act, (int)gemm_tiles_max(n, (int)h->E), st, mid));
  if (!noalloc) h->mid_recorded = mid != nullptr;
  HIPCHK(launch_combine(a.c.eout, tw, ids, y, (int)T, (int)K, (int)h->E, (int)h->H, act, st, true));
  return MI_MOE_OK;
}

int q_alloc_weights(mi_moe_handle* h) {
  const int64_t E = h->E, H = h->H, I = h->I;
  const int64_t bb = h->quant == MI_MOE_Q8_0 ? 2048 : 1024;  // bytes per (tile, block)
  HIPCHK(h->w13.alloc((size_t)E * (I / 32) * (H / 32) * bb));
  HIPCHK(h->w13_s.alloc((size_t)E * (I / 32) * (H / 32) * 64 * 2));
  HIPCHK(h->w2.alloc((size_t)E * (H / 64) * (I / 32) * bb));
  HIPCHK(h->w2_s.alloc((size_t)E * (H / 64) * (I / 32) * 64 * 2));
  HIPCHK(hipMemset(h->w13.p, 0, h->w13.bytes));
  HIPCHK(hipMemset(h->w13_s.p, 0, h->w13_s.bytes));
  HIPCHK(hipMemset(h->w2.p, 0, h->w2.bytes));
  HIPCHK(hipMemset(h->w2_s.p, 0, h->w2_s.bytes));
  return MI_MOE_OK;
}

int forward_q(mi_moe_handle* h, const void* x, void* y, const float* tw, const int32_t* ids,
              int64_t T, int64_t K, int act, bool noalloc, hipStream_t st) {
  const int64_t n = T * K;
  // decode sizes: the lane-per-row kernels, with the down projection and the
  // combine token-major in one launch (no eout round trip) where it fits;
  // above q_lpr_max_pairs routed pairs, or where the lane-per-row LDS does not
  // fit, the int8 grouped GEMMs (mi_moe_create checked that one of the two
  // serves every call)
  const size_t lmax = device_max_lds();
  const int iE = (int)h->E, iH = (int)h->H, iI = (int)h->I, in = (int)n, iK = (int)K;
  const bool small = n <= q_lpr_max_pairs(h->quant);
  const bool token_down = small && K <= kDownMaxK && q_lpr_fits(iH, iI, iE, in, iK, true, lmax);
  const bool lpr_small = small && (token_down || q_lpr_fits(iH, iI, iE, in, iK, false, lmax));
  const bool gemm = q_gemm_ok(iH, iI) && !lpr_small;
  if (!gemm && !q_lpr_fits(iH, iI, iE, in, iK, token_down, lmax))
    return fail(MI_MOE_EUNSUPPORTED, "Q8_0/Q4_0 call of %lld routed pairs does not fit the device's LDS", (long long)n);
  Work w;
  int rc = get_work(h, T, n, gemm || !token_down, noalloc, st, w);
  if (rc) return rc;
  QArgs a;
  std::memset(&a, 0, sizeof(a));
  fill_sched(h, a.c, x, y, tw, ids, T, K, w);
  a.w13 = h->w13.p; a.w13_d = (const uint16_t*)h->w13_s.p;
  a.w2 = h->w2.p; a.w2_d = (const uint16_t*)h->w2_s.p;
  a.act_q = (int8_t*)w.act;
  a.act_d = w.act_d;
  a.tact = w.tact;
  if (gemm) {
    // sorted path: Q8_0 activations once per token, routing with row tiles,
    // the two int8 grouped GEMMs, the combine
    a.xq = w.xq;
    a.xd = w.xd;
    HIPCHK(launch_quant_route(x, act, T, h->H, w.xq, w.xd, ids, (int)n, (int)K, (int)h->E, a.c.rg, st, 0));
    HIPCHK(launch_qint_gemm(a, h->quant, h->scale_dtype, (int)gemm_tiles_max(n, (int)h->E), st));
    HIPCHK(launch_combine(a.c.eout, tw, ids, y, (int)T, (int)K, (int)h->E, (int)h->H, act, st, false));
    return MI_MOE_OK;
  }
  // the smallest calls in one launch (gate_up hands the intermediate to down inside it)
  if (token_down && a.tact && q_fused_lds(in, iK, iH, iI, iE)) {
    HIPCHK(launch_q_fused(a, h->quant, act, h->scale_dtype, st));
    return MI_MOE_OK;
  }
  if (a.c.route_global) HIPCHK(launch_route_global(ids, (int)n, (int)K, (int)h->E, a.c.rg, st, 0, 0));
  const int64_t umax = n < h->E ? n : h->E;
  const int64_t grid1 = (n <= kQBallotMaxPairs ? n : umax) * (h->I / 32), grid2 = umax * (h->H / 64);
  HIPCHK(launch_qint(a, h->quant, act, h->scale_dtype, (int)grid1, (int)grid2, token_down, st));
  if (!token_down) HIPCHK(launch_combine(a.c.eout, tw, ids, y, (int)T, (int)K, (int)h->E, (int)h->H, act, st, false));
  return MI_MOE_OK;
}

// Argument checks shared by mi_moe_forward and mi_moe_forward_noalloc.
int check_forward_args(mi_moe_handle* h, const void* x, void* y, const float* topk_w, const int32_t* topk_ids,
                       int64_t T, int64_t K, int act_dtype) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (!h->loaded) return fail(MI_MOE_ENOTLOADED, "weights not stored");
  if (act_dtype != MI_MOE_F16 && act_dtype != MI_MOE_BF16)
    return fail(MI_MOE_EINVAL, "hidden dtype must be fp16 or bf16");
  if (T < 0 || K < 1 || K > 64) return fail(MI_MOE_EINVAL, "bad T=%lld / top_k=%lld", (long long)T, (long long)K);
  if (T == 0) return MI_MOE_OK;
  if ((int64_t)T * K > (int64_t)1 << 24) return fail(MI_MOE_EINVAL, "T*top_k too large");
  if (!x || !y || !topk_w || !topk_ids) return fail(MI_MOE_EINVAL, "null data pointer");
  if (!aligned16(x) || !aligned16(y)) return fail(MI_MOE_EINVAL, "hidden/out must be 16-byte aligned");
  return MI_MOE_OK;
}

}  // namespace

// ====================================================================== ABI
MI_API const char* mi_moe_last_error(void) { return g_err.c_str(); }

MI_API int mi_moe_version(void) { return 100; }

namespace mimoe {
int api_fail(int code, const char* msg) {
  g_err = msg;
  return code;
}

int check_dims(int64_t E, int64_t H, int64_t I, int quant_type) {
  if (E <= 0 || H <= 0 || I <= 0) return fail(MI_MOE_EINVAL, "E, H, I must be positive");
  if (quant_type < 0 || quant_type > 2) return fail(MI_MOE_EINVAL, "quant_type must be 0, 1 or 2");
  if (H % 32 != 0) return fail(MI_MOE_EINVAL, "hidden_size must be multiple of 32");
  if (I % 32 != 0) return fail(MI_MOE_EINVAL, "intermediate_size must be multiple of 32");
  if (quant_type != MI_MOE_W4A16 && H % 64 != 0)
    return fail(MI_MOE_EINVAL, "hidden_size must be multiple of 64");
  if (quant_type == MI_MOE_W4A16 && (H % 512 != 0 || I % 128 != 0))
    return fail(MI_MOE_EINVAL, "W4A16 needs hidden_size %% 512 == 0 and intermediate_size %% 128 == 0");
  if (E > 512) return fail(MI_MOE_EUNSUPPORTED, "at most 512 experts");
  // one path must serve calls of every size: the W4A16 grouped GEMMs, or for
  // Q8_0 / Q4_0 the int8 grouped GEMMs or else the lane-per-row kernels at
  // the largest in-LDS routing
  const size_t lmax = device_max_lds();
  if (quant_type == MI_MOE_W4A16 && !w4_sorted_fits((int)H, (int)I, lmax))
    return fail(MI_MOE_EUNSUPPORTED, "W4A16 H=%lld I=%lld: the grouped GEMMs need %zu and %zu bytes of LDS, "
                "the device allows %zu", (long long)H, (long long)I, w4_gemm13_lds_bytes((int)H),
                w4_gemm2_lds_bytes((int)I), lmax);
  if (quant_type != MI_MOE_W4A16 && !q_gemm_ok((int)H, (int)I) &&
      !q_lpr_fits((int)H, (int)I, (int)E, kRouteLdsMax, 1, false, lmax))
    return fail(MI_MOE_EUNSUPPORTED, "Q8_0/Q4_0 H=%lld I=%lld: not multiples of 128 and too large for the "
                "lane-per-row kernels' LDS", (long long)H, (long long)I);
  return MI_MOE_OK;
}

size_t device_max_lds() {
  static std::atomic<int> cache[64];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kMaxLds;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return (size_t)v;
  int lds = 0;
  if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
      lds < (int)kMaxLds)
    lds = (int)kMaxLds;
  cache[dev].store(lds, std::memory_order_relaxed);
  return (size_t)lds;
}
}  // namespace mimoe

MI_API int mi_moe_create(int64_t E, int64_t H, int64_t I, int quant_type, mi_moe_handle** out) {
  if (!out) return fail(MI_MOE_EINVAL, "out is null");
  *out = nullptr;
  const int rc = check_dims(E, H, I, quant_type);
  if (rc) return rc;
  mi_moe_handle* h = new (std::nothrow) mi_moe_handle();
  if (!h) return fail(MI_MOE_EINVAL, "out of host memory");
  h->E = E; h->H = H; h->I = I; h->quant = quant_type;
  if (hipGetDevice(&h->device) != hipSuccess ||
      hipDeviceGetAttribute(&h->num_cu, hipDeviceAttributeMultiprocessorCount, h->device) != hipSuccess ||
      hipEventCreate(&h->ev0) != hipSuccess || hipEventCreate(&h->ev1) != hipSuccess ||
      hipEventCreate(&h->evmid) != hipSuccess) {
    delete h;
    return fail(MI_MOE_EHIP, "HIP device query / event creation failed");
  }
  // the one-launch decode units (zeroed: no dispatch has tag 0)
  if (I <= kTagActMaxI &&
      (h->tact.alloc(tagged_act_bytes((int)I)) != hipSuccess ||
       hipMemset(h->tact.p, 0, tagged_act_bytes((int)I)) != hipSuccess)) {
    mi_moe_destroy(h);
    return fail(MI_MOE_EHIP, "allocating the decode hand-over buffer failed");
  }
  // the no-alloc entry point's scratch address on this device (once per device)
  if (init_scratch(h->device) != MI_MOE_OK) {
    const std::string msg = g_err;
    mi_moe_destroy(h);
    return fail(MI_MOE_EHIP, "%s", msg.c_str());
  }
  *out = h;
  return MI_MOE_OK;
}

MI_API int mi_moe_destroy(mi_moe_handle* h) {
  if (!h) return MI_MOE_OK;
  (void)hipDeviceSynchronize();
  DevBuf* bufs[] = {&h->w13, &h->w13_s, &h->w13_z, &h->w2, &h->w2_s, &h->w2_z,
                    &h->act, &h->eout, &h->act_d, &h->r_counts, &h->r_starts,
                    &h->r_active, &h->r_tok, &h->r_scat, &h->r_U, &h->r_tiles, &h->r_ntiles,
                    &h->xq, &h->xd, &h->r_chunk, &h->r_rids, &h->r_rw, &h->tact};
  for (DevBuf* b : bufs) b->release();
  for (void* p : h->retired) (void)hipFree(p);
  if (h->ev0) (void)hipEventDestroy(h->ev0);
  if (h->ev1) (void)hipEventDestroy(h->ev1);
  if (h->evmid) (void)hipEventDestroy(h->evmid);
  delete h;
  return MI_MOE_OK;
}

MI_API int mi_moe_get_info(const mi_moe_handle* h, int64_t* E, int64_t* H, int64_t* I, int* quant,
                           int* scale_dtype) {
  if (!h) return fail(MI_MOE_EINVAL, "null handle");
  if (E) *E = h->E;
  if (H) *H = h->H;
  if (I) *I = h->I;
  if (quant) *quant = h->quant;
  if (scale_dtype) *scale_dtype = h->scale_dtype;
  return MI_MOE_OK;
}

MI_API int mi_moe_reserve(mi_moe_handle* h, int64_t T, int64_t K, void* stream) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (T < 0 || K < 1 || K > 64) return fail(MI_MOE_EINVAL, "bad T=%lld / top_k=%lld", (long long)T, (long long)K);
  if (T * K > ((int64_t)1 << 24)) return fail(MI_MOE_EINVAL, "T*top_k too large");
  return ensure_workspace(h, T, T * K, (hipStream_t)stream);
}

MI_API int mi_moe_set_timing(mi_moe_handle* h, int enable) {
  if (!h) return fail(MI_MOE_EINVAL, "null handle");
  h->timing = enable != 0;
  return MI_MOE_OK;
}

MI_API double mi_moe_get_last_run_time_ms(mi_moe_handle* h) {
  if (!h || !h->timing || !h->timed_once) return -1.0;
  if (hipEventSynchronize(h->ev1) != hipSuccess) return -1.0;
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, h->ev0, h->ev1) != hipSuccess) return -1.0;
  return (double)ms;
}

MI_API int mi_moe_store_awq(mi_moe_handle* h, const int32_t* w13_q, const int32_t* w13_z,
                            const void* w13_s, const int32_t* w2_q, const int32_t* w2_z,
                            const void* w2_s, int64_t group, int scale_dtype, int src_on_device,
                            void* stream) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (h->quant != MI_MOE_W4A16) return fail(MI_MOE_EINVAL, "store_awq needs a W4A16 handle (quant_type 2)");
  if (group != 128) return fail(MI_MOE_EUNSUPPORTED, "W4A16 group size %lld unsupported (128 only)", (long long)group);
  if (scale_dtype != MI_MOE_F16 && scale_dtype != MI_MOE_BF16) return fail(MI_MOE_EINVAL, "scale dtype must be fp16 or bf16");
  if (!w13_q || !w13_z || !w13_s || !w2_q || !w2_z || !w2_s) return fail(MI_MOE_EINVAL, "null weight pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t E = h->E, H = h->H, I = h->I, N13 = 2 * I;
  const size_t q13 = (size_t)E * H * (N13 / 8) * 4, z13 = (size_t)E * (H / 128) * (N13 / 8) * 4,
               s13 = (size_t)E * (H / 128) * N13 * 2;
  const size_t q2 = (size_t)E * I * (H / 8) * 4, z2 = (size_t)E * (I / 128) * (H / 8) * 4,
               s2 = (size_t)E * (I / 128) * H * 2;
  Staged a, b, c, d, e, f;
  HIPCHK(a.stage(w13_q, q13, src_on_device, st));
  HIPCHK(b.stage(w13_z, z13, src_on_device, st));
  HIPCHK(c.stage(w13_s, s13, src_on_device, st));
  HIPCHK(d.stage(w2_q, q2, src_on_device, st));
  HIPCHK(e.stage(w2_z, z2, src_on_device, st));
  HIPCHK(f.stage(w2_s, s2, src_on_device, st));
  const int64_t NT13 = 2 * (I / 16), G1 = H / 128, CH = I / 32, MQ = H / 64, G2 = I / 128;
  HIPCHK(h->w13.alloc((size_t)E * NT13 * G1 * 1024));
  HIPCHK(h->w13_s.alloc((size_t)E * (I / 16) * 80 * G1));    // metadata blocks
  HIPCHK(h->w2.alloc((size_t)E * CH * MQ * 1024));
  HIPCHK(h->w2_s.alloc((size_t)E * MQ * 4 * w2_meta_sec_bytes((int)G2)));   // metadata sections
  HIPCHK(launch_awq_repack_all((const int32_t*)a.ptr, (const int32_t*)b.ptr, (const uint16_t*)c.ptr,
                               (const int32_t*)d.ptr, (const int32_t*)e.ptr, (const uint16_t*)f.ptr,
                               h->w13.p, (unsigned char*)h->w13_s.p, h->w2.p, (unsigned char*)h->w2_s.p,
                               (int)E, (int)H, (int)I, st));
  HIPCHK(hipStreamSynchronize(st));
  h->scale_dtype = scale_dtype;
  h->group = (int)group;
  h->loaded = true;
  return MI_MOE_OK;
}

MI_API int mi_moe_store_quantized(mi_moe_handle* h, const void* gate_up_qs, const void* gate_up_d,
                                  const void* down_qs, const void* down_d, int scale_dtype,
                                  int src_on_device, void* stream) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (h->quant != MI_MOE_Q8_0 && h->quant != MI_MOE_Q4_0)
    return fail(MI_MOE_EINVAL, "store_quantized needs a Q8_0 or Q4_0 handle");
  if (scale_dtype != MI_MOE_F16 && scale_dtype != MI_MOE_BF16)
    return fail(MI_MOE_EINVAL, "gate_up_d must be float16 or bfloat16");
  if (!gate_up_qs || !gate_up_d || !down_qs || !down_d) return fail(MI_MOE_EINVAL, "null weight pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t E = h->E, H = h->H, I = h->I;
  const size_t qdiv = h->quant == MI_MOE_Q4_0 ? 2 : 1;
  Staged a, b, c, d;
  HIPCHK(a.stage(gate_up_qs, (size_t)E * 2 * I * H / qdiv, src_on_device, st));
  HIPCHK(b.stage(gate_up_d, (size_t)E * 2 * I * (H / 32) * 2, src_on_device, st));
  HIPCHK(c.stage(down_qs, (size_t)E * H * I / qdiv, src_on_device, st));
  HIPCHK(d.stage(down_d, (size_t)E * H * (I / 32) * 2, src_on_device, st));
  if (!h->w13.p) { rc = q_alloc_weights(h); if (rc) return rc; }
  HIPCHK(launch_q_repack(h->quant, a.ptr, (const uint16_t*)b.ptr, h->w13.p, (uint16_t*)h->w13_s.p,
                         (int)E, (int)(2 * I), (int)H, 0, (int)I, st));
  HIPCHK(launch_q_repack(h->quant, c.ptr, (const uint16_t*)d.ptr, h->w2.p, (uint16_t*)h->w2_s.p,
                         (int)E, (int)H, (int)I, 1, (int)I, st));
  HIPCHK(hipStreamSynchronize(st));
  h->scale_dtype = scale_dtype;
  h->loaded = true;
  return MI_MOE_OK;
}

MI_API int mi_moe_quantize_and_store_expert(mi_moe_handle* h, int64_t expert, int proj,
                                            const void* w, int w_dtype, int src_on_device,
                                            void* stream) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (h->quant != MI_MOE_Q8_0)
    return fail(MI_MOE_EINVAL, "Q4_0 does not support online quantization. "
                               "Use store_quantized_repack() with pre-quantized weights.");
  if (expert < 0 || expert >= h->E) return fail(MI_MOE_EINVAL, "expert index out of range");
  if (proj < 0 || proj > 2) return fail(MI_MOE_EINVAL, "Unknown proj (0 gate_proj, 1 up_proj, 2 down_proj)");
  if (w_dtype < 0 || w_dtype > 2) return fail(MI_MOE_EINVAL, "weight must be float32, float16 or bfloat16");
  if (!w) return fail(MI_MOE_EINVAL, "null weight pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t N = proj == 2 ? h->H : h->I, K = proj == 2 ? h->I : h->H;
  const size_t esz = w_dtype == 2 ? 4 : 2;
  Staged a;
  HIPCHK(a.stage(w, (size_t)N * K * esz, src_on_device, st));
  if (!h->w13.p) { rc = q_alloc_weights(h); if (rc) return rc; }
  void* wdst = proj == 2 ? h->w2.p : h->w13.p;
  uint16_t* ddst = (uint16_t*)(proj == 2 ? h->w2_s.p : h->w13_s.p);
  HIPCHK(launch_q8_online_quant(a.ptr, w_dtype, (int)N, (int)K, (int)expert, proj, (int)h->I, wdst,
                                ddst, st));
  HIPCHK(hipStreamSynchronize(st));
  h->scale_dtype = MI_MOE_F16;  // quantize_weight_only stores fp16 scales
  h->loaded = true;
  return MI_MOE_OK;
}

MI_API int mi_moe_block_dots(mi_moe_handle* h, int64_t expert, int proj, const int8_t* a_qs,
                             int64_t M, int32_t* isum, void* stream) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (h->quant != MI_MOE_Q8_0 && h->quant != MI_MOE_Q4_0)
    return fail(MI_MOE_EINVAL, "block dots need a Q8_0 or Q4_0 handle");
  if (!h->loaded) return fail(MI_MOE_ENOTLOADED, "weights not stored");
  if (expert < 0 || expert >= h->E || (proj != 0 && proj != 1) || M < 0)
    return fail(MI_MOE_EINVAL, "bad expert / proj / M");
  if (M == 0) return MI_MOE_OK;
  if (!a_qs || !isum) return fail(MI_MOE_EINVAL, "null pointer");
  const int64_t N = proj == 0 ? 2 * h->I : h->H, K = proj == 0 ? h->H : h->I;
  const int tiles = proj == 0 ? (int)(h->I / 32) : (int)(h->H / 64);
  HIPCHK(launch_q_block_dots(h->quant, proj == 0 ? h->w13.p : h->w2.p, a_qs, isum, (int)M, (int)N,
                             (int)K, (int)expert, proj, (int)h->I, tiles, (hipStream_t)stream));
  return MI_MOE_OK;
}

MI_API int mi_moe_block_dots_mfma(mi_moe_handle* h, int64_t expert, int proj, const int8_t* a_qs,
                                  int64_t M, int32_t* acc, float* prod, void* stream) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (h->quant != MI_MOE_Q8_0 && h->quant != MI_MOE_Q4_0)
    return fail(MI_MOE_EINVAL, "block dots need a Q8_0 or Q4_0 handle");
  if (!h->loaded) return fail(MI_MOE_ENOTLOADED, "weights not stored");
  if (h->H % 128 != 0 || h->I % 128 != 0)
    return fail(MI_MOE_EUNSUPPORTED, "the int8-MFMA grouped GEMMs need H %% 128 == 0 and I %% 128 == 0");
  if (expert < 0 || expert >= h->E || (proj != 0 && proj != 1) || M < 0)
    return fail(MI_MOE_EINVAL, "bad expert / proj / M");
  if (M == 0) return MI_MOE_OK;
  if (M > 65535 * 16) return fail(MI_MOE_EINVAL, "M too large");
  if (!a_qs || !acc || !prod) return fail(MI_MOE_EINVAL, "null pointer");
  if (((uintptr_t)a_qs & 7u) != 0) return fail(MI_MOE_EINVAL, "a_qs must be 8-byte aligned");
  const int64_t N = proj == 0 ? 2 * h->I : h->H, K = proj == 0 ? h->H : h->I;
  const int tiles = proj == 0 ? (int)(h->I / 32) : (int)(h->H / 64);
  HIPCHK(launch_q_mfma_block_check(h->quant, h->scale_dtype, proj == 0 ? h->w13.p : h->w2.p,
                                   (const uint16_t*)(proj == 0 ? h->w13_s.p : h->w2_s.p), a_qs, acc, prod,
                                   (int)M, (int)N, (int)K, (int)expert, proj, (int)h->I, tiles,
                                   (hipStream_t)stream));
  return MI_MOE_OK;
}

MI_API int mi_moe_forward(mi_moe_handle* h, const void* x, void* y, const float* topk_w,
                          const int32_t* topk_ids, int64_t T, int64_t K, int act_dtype,
                          void* stream) {
  int rc = check_forward_args(h, x, y, topk_w, topk_ids, T, K, act_dtype);
  if (rc || T == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) h->captured = true;
  if (h->timing) HIPCHK(hipEventRecord(h->ev0, st));
  h->mid_recorded = false;
  if (h->quant == MI_MOE_W4A16) rc = forward_w4a16(h, x, y, topk_w, topk_ids, T, K, act_dtype, false, st);
  else rc = forward_q(h, x, y, topk_w, topk_ids, T, K, act_dtype, false, st);
  if (rc) return rc;
  if (h->timing) {
    HIPCHK(hipEventRecord(h->ev1, st));
    h->timed_once = true;
  }
  return MI_MOE_OK;
}

MI_API int mi_moe_forward_noalloc(mi_moe_handle* h, const void* x, void* y, const float* topk_w,
                                  const int32_t* topk_ids, int64_t T, int64_t K, int act_dtype,
                                  void* stream) {
  int rc = check_forward_args(h, x, y, topk_w, topk_ids, T, K, act_dtype);
  if (rc || T == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (h->quant == MI_MOE_W4A16) return forward_w4a16(h, x, y, topk_w, topk_ids, T, K, act_dtype, true, st);
  return forward_q(h, x, y, topk_w, topk_ids, T, K, act_dtype, true, st);
}

MI_API int mi_moe_topk_softmax(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K,
                               int renormalize, int32_t* topk_ids, float* topk_w, void* stream) {
  if (logits_dtype != MI_MOE_F16 && logits_dtype != MI_MOE_BF16 && logits_dtype != MI_MOE_F32)
    return fail(MI_MOE_EINVAL, "logits dtype must be fp16, bf16 or fp32");
  if (T < 0 || E < 1 || E > 512) return fail(MI_MOE_EINVAL, "bad T=%lld / E=%lld (E <= 512)", (long long)T, (long long)E);
  if (K < 1 || K > E || K > 64) return fail(MI_MOE_EINVAL, "top_k=%lld must be in [1, min(E, 64)]", (long long)K);
  if (T > ((int64_t)1 << 24)) return fail(MI_MOE_EINVAL, "T too large");
  if (T == 0) return MI_MOE_OK;
  if (!logits || !topk_ids || !topk_w) return fail(MI_MOE_EINVAL, "null pointer");
  HIPCHK(launch_topk_softmax(logits, logits_dtype, (int)T, (int)E, (int)K, renormalize ? 1 : 0, topk_ids, topk_w,
                             (hipStream_t)stream));
  return MI_MOE_OK;
}

MI_API int mi_moe_forward_logits(mi_moe_handle* h, const void* x, void* y, const void* router_logits,
                                 int logits_dtype, int64_t T, int64_t K, int renormalize, int act_dtype,
                                 int32_t* topk_ids_out, float* topk_w_out, void* stream) {
  int rc = check_handle(h);
  if (rc) return rc;
  if (T < 0 || K < 1 || K > 64) return fail(MI_MOE_EINVAL, "bad T=%lld / top_k=%lld", (long long)T, (long long)K);
  if (T == 0) return MI_MOE_OK;
  if ((topk_ids_out == nullptr) != (topk_w_out == nullptr))
    return fail(MI_MOE_EINVAL, "topk_ids_out and topk_w_out must both be given or both be null");
  hipStream_t st = (hipStream_t)stream;
  int32_t* ids = topk_ids_out;
  float* w = topk_w_out;
  if (!ids) {
    const int64_t need = T * K;
    if (need > h->cap_r) {
      int64_t cap = h->cap_r ? h->cap_r : 1024;
      while (cap < need) cap *= 2;
      HIPCHK(hipStreamSynchronize(st));   // the buffers may be in use by queued work
      if (h->captured) {                  // or by captured graphs
        h->r_rids.retire(h->retired);
        h->r_rw.retire(h->retired);
      }
      HIPCHK(h->r_rids.alloc((size_t)cap * sizeof(int32_t)));
      HIPCHK(h->r_rw.alloc((size_t)cap * sizeof(float)));
      h->cap_r = cap;
    }
    ids = (int32_t*)h->r_rids.p;
    w = (float*)h->r_rw.p;
  }
  rc = mi_moe_topk_softmax(router_logits, logits_dtype, T, h->E, K, renormalize, ids, w, stream);
  if (rc) return rc;
  return mi_moe_forward(h, x, y, w, ids, T, K, act_dtype, stream);
}

MI_API int mi_moe_get_last_phase_times_ms(mi_moe_handle* h, double* ms, int max_phases) {
  if (!h || !ms || max_phases < 1) return fail(MI_MOE_EINVAL, "null handle / buffer");
  if (!h->timing || !h->timed_once) return fail(MI_MOE_EINVAL, "timing off or no timed call");
  HIPCHK(hipEventSynchronize(h->ev1));
  float t = 0.0f;
  if (!h->mid_recorded || max_phases < 2) {
    HIPCHK(hipEventElapsedTime(&t, h->ev0, h->ev1));
    ms[0] = t;
    return 1;
  }
  HIPCHK(hipEventElapsedTime(&t, h->ev0, h->evmid));
  ms[0] = t;
  HIPCHK(hipEventElapsedTime(&t, h->evmid, h->ev1));
  ms[1] = t;
  return 2;
}

MI_API int mi_moe_quantize_act_q8_0(const void* x, int act_dtype, int64_t T, int64_t H,
                                    int8_t* x_qs, float* x_d, void* stream) {
  if (act_dtype != MI_MOE_F16 && act_dtype != MI_MOE_BF16) return fail(MI_MOE_EINVAL, "dtype must be fp16 or bf16");
  if (T < 0 || H <= 0 || H % 32) return fail(MI_MOE_EINVAL, "H must be a positive multiple of 32");
  if (T == 0) return MI_MOE_OK;
  if (!x || !x_qs || !x_d) return fail(MI_MOE_EINVAL, "null pointer");
  if (!aligned16(x) || !aligned16(x_qs)) return fail(MI_MOE_EINVAL, "x and x_qs must be 16-byte aligned");
  HIPCHK(launch_quant_act(x, act_dtype, T, H, x_qs, x_d, (hipStream_t)stream));
  return MI_MOE_OK;
}

MI_API int mi_moe_route(const int32_t* ids, int64_t T, int64_t K, int64_t E, int32_t* counts,
                        int32_t* starts, int32_t* token_map, int32_t* scatter, void* stream) {
  if (T < 0 || K < 1 || E < 1) return fail(MI_MOE_EINVAL, "bad T/K/E");
  if (E > 512) return fail(MI_MOE_EUNSUPPORTED, "at most 512 experts");
  if (T * K > ((int64_t)1 << 24)) return fail(MI_MOE_EINVAL, "T*K too large");
  if (!counts || !starts) return fail(MI_MOE_EINVAL, "null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (T == 0) {  // nothing routed: empty histogram
    HIPCHK(hipMemsetAsync(counts, 0, (size_t)E * sizeof(int32_t), st));
    HIPCHK(hipMemsetAsync(starts, 0, (size_t)(E + 1) * sizeof(int32_t), st));
    HIPCHK(hipStreamSynchronize(st));
    return MI_MOE_OK;
  }
  if (!ids || !token_map || !scatter) return fail(MI_MOE_EINVAL, "null pointer");
  // the routing kernels' own arrays (active experts, their count, per-chunk
  // histograms) live in a per-device buffer that grows to the largest call
  // and is reused; the call holds it until its stream has finished
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(MI_MOE_EUNSUPPORTED, "device index %d out of range", dev);
  const size_t a_bytes = ((size_t)E * sizeof(int32_t) + 255) & ~(size_t)255;
  const size_t need = a_bytes + 256 + (size_t)route_chunks((int)(T * K)) * E * sizeof(int32_t);
  std::lock_guard<std::mutex> lock(g_route_mu);
  DevBuf& buf = g_route_buf[dev];
  if (buf.bytes < need) HIPCHK(buf.alloc(need));
  unsigned char* base = (unsigned char*)buf.p;
  RouteGlobal rg{counts, starts, (int32_t*)base, token_map, scatter, (int32_t*)(base + a_bytes), nullptr, nullptr,
                 (int32_t*)(base + a_bytes + 256)};
  HIPCHK(launch_route_global(ids, (int)(T * K), (int)K, (int)E, rg, st, 1, 0));
  HIPCHK(hipStreamSynchronize(st));
  return MI_MOE_OK;
}
