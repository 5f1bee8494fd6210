// mi_moe_sched.hpp -- work decomposition shared by every fused MoE path.
//
// A layer call is two launches on the caller's stream (plus a routing kernel
// when T*K exceeds the in-LDS routing limit):
//   phase 1 (one workgroup per (expert, slice of I)):  gate_up GEMV/GEMM,
//       SiLU*mul, optional Q8_0 re-quantization -> act[pos][slice]
//   phase 2 (one workgroup per (expert, 64-row block of H)): down projection
//       -> eout[pos][64hb..64hb+63]; then arrivals are counted per
//       (token, hb) and the last arriving expert of a token sums eout over k
//       in order and casts (Stage C1 + C2 of Int8-gemm/q8_gemm.cpp:593-641,
//       tp = 1).  Nothing waits: the count decides who combines.
// The kernel boundary between the phases is the only dependency.  Every
// workgroup routes the (t,k) pairs itself -- the stable counting sort of
// preprocess_moe_routing (Int8-gemm/moe_common.cpp:146-216) -- in LDS for
// small T*K, or reads the arrays the routing kernel wrote.  Workgroups whose
// item index is past the active experts exit at once.
#pragma once
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"

namespace mimoe {

struct RouteView {
  const int* starts;
  const int* active;
  const int* tok;
  const int* scat;
  int U;
};

__device__ __forceinline__ int nvalid_of(const RouteView& rv, int t, int K) {
  int c = 0;
  for (int k = 0; k < K; ++k) c += rv.scat[t * K + k] >= 0;
  return c;
}

__host__ __device__ inline size_t route_lds_ints(int E, int n) { return (size_t)3 * E + 1 + 2 * (size_t)n; }

// Route (LDS or global) -> RouteView.  route_lds_buf holds route_lds_ints(E,n)
// ints when !c.route_global.
__device__ inline RouteView sched_route(const SchedArgs& c, int* route_lds_buf, int* s_U) {
  RouteView rv;
  if (!c.route_global) {
    int* counts = route_lds_buf;
    int* starts = counts + c.E;
    int* active = starts + c.E + 1;
    int* tok = active + c.E;
    int* scat = tok + c.n;
    route_lds(c.ids, c.n, c.K, c.E, counts, starts, active, tok, scat, s_U);
    rv.starts = starts; rv.active = active; rv.tok = tok; rv.scat = scat; rv.U = *s_U;
  } else {
    rv.starts = c.rg.starts; rv.active = c.rg.active; rv.tok = c.rg.tok; rv.scat = c.rg.scat;
    rv.U = *c.rg.U;
  }
  return rv;
}

// Tokens without any valid expert id get y = 0 (Int8-gemm/q8_gemm.cpp:
// 329-332 and 599-611).  Called by one workgroup of phase 1.
template <int ACT>
__device__ void zero_unrouted(const SchedArgs& c, const RouteView& rv) {
  const int tid = threadIdx.x;
  for (int t = tid >> 6; t < c.T; t += kBlock / kWave)
    if (nvalid_of(rv, t, c.K) == 0)
      for (int h = tid & 63; h < c.H; h += kWave) c.y[(size_t)t * c.H + h] = 0;
}

// Phase-2 epilogue: eout rows [p0, p0+cnt) x cols [64hb, 64hb+64) are
// written by this workgroup.  Count arrivals; the last expert of a token
// combines y[t, 64hb..] = cast(sum_k w[t,k] * eout[scatter[t,k]]) in k order
// and re-arms the counter for the next call.
template <int ACT>
__device__ void combine_hb(const SchedArgs& c, const RouteView& rv, int p0, int cnt, int hb,
                           int* s_list, int* s_nlist) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int NI2 = c.H >> 6;
  fence_release();
  __syncthreads();
  for (int c0 = 0; c0 < cnt; c0 += kBlock) {
    if (tid == 0) *s_nlist = 0;
    __syncthreads();
    const int ci = c0 + tid;
    if (ci < cnt) {
      const int t = rv.tok[p0 + ci];
      const uint32_t old = __hip_atomic_fetch_add(c.cnt2 + (size_t)t * NI2 + hb, 1u,
                                                  __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      if ((int)old + 1 == nvalid_of(rv, t, c.K)) s_list[atomicAdd(s_nlist, 1)] = t;
    }
    __syncthreads();
    const int nl = *s_nlist;
    if (nl > 0) {
      fence_acquire();
      for (int li = wave; li < nl; li += kBlock / kWave) {
        const int t = s_list[li];
        const int h = 64 * hb + lane;
        float acc = 0.0f;
        for (int k = 0; k < c.K; ++k) {
          const int pos = rv.scat[t * c.K + k];
          if (pos < 0) continue;
          const float prod = c.tw[t * c.K + k] * c.eout[(size_t)pos * c.H + h];
          acc = acc + prod;
        }
        c.y[(size_t)t * c.H + h] = from_f32<ACT>(acc);
        if (lane == 0) c.cnt2[(size_t)t * NI2 + hb] = 0u;
      }
    }
    __syncthreads();
  }
}

}  // namespace mimoe
