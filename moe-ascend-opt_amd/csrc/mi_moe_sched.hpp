// mi_moe_sched.hpp -- routing view of the Q8_0 / Q4_0 multi-launch path.
//
// Phase 1 (one workgroup per (expert, slice of I)) computes gate_up +
// SiLU*mul (+ the intermediate Q8_0) into act[i] for every routed pair
// i = t*K+k of the expert; phase 2 (one workgroup per (expert, 64-row block of
// H)) computes the down projection into eout[i]; a combine kernel sums eout
// over k in order and casts (Stage C1 + C2 of Int8-gemm/q8_gemm.cpp:593-641,
// tp = 1).  Kernel boundaries are the only dependencies.  Every workgroup
// routes the pairs itself -- the stable counting sort of
// preprocess_moe_routing (Int8-gemm/moe_common.cpp:146-216) -- in LDS for
// small T*K, or reads the arrays the routing kernel wrote.  Workgroups whose
// item index is past the active experts exit at once.
#pragma once
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"

namespace mimoe {

struct RouteView {
  const int* starts;   // [E+1]
  const int* active;   // [U] ascending expert ids
  const int* pair;     // [n] pair index t*K+k per expert-sorted position
  int U;
};

// Route (LDS or global) -> RouteView.  route_lds_buf holds route_lds_ints(E,n)
// ints when !c.route_global.
__device__ inline RouteView sched_route(const SchedArgs& c, int* route_lds_buf, int* s_U) {
  RouteView rv;
  if (!c.route_global) {
    int* counts = route_lds_buf;
    int* starts = counts + c.E;
    int* active = starts + c.E + 1;
    int* pair = active + c.E;
    int* scat = pair + c.n;
    route_lds(c.ids, c.n, c.K, c.E, counts, starts, active, pair, scat, s_U);
    rv.starts = starts; rv.active = active; rv.pair = pair; rv.U = *s_U;
  } else {
    rv.starts = c.rg.starts; rv.active = c.rg.active; rv.pair = c.rg.tok;
    rv.U = *c.rg.U;
  }
  return rv;
}

__device__ __forceinline__ uint64_t lanemask_lt(int lane) {
  return lane ? (~0ull >> (64 - lane)) : 0ull;
}

// Routing for T*K <= 64 without a sort: every wave reads all ids at once.
// Work item pi (a pair index) serves its expert iff pi is the expert's first
// pair; column j of the expert is its j-th pair in ascending pair order, the
// order the stable counting sort of preprocess_moe_routing
// (Int8-gemm/moe_common.cpp:146-216) gives.  Lane l of `colpair` holds the
// pair index of column l.  Whole-wave routine.
struct BallotCols {
  int e, cnt, colpair;
  uint64_t vmask;      // bit i: pair i has a valid expert id
  bool serve;
};
__device__ __forceinline__ BallotCols ballot_cols(const SchedArgs& c, int pi, int lane) {
  BallotCols b;
  const int myid = lane < c.n ? c.ids[lane] : -1;
  const bool myvalid = lane < c.n && (unsigned)myid < (unsigned)c.E;
  b.vmask = __ballot(myvalid);
  b.e = __shfl(myid, pi);
  const uint64_t match = __ballot(myvalid && myid == b.e);
  b.serve = (unsigned)b.e < (unsigned)c.E && (__ffsll((long long)match) - 1) == pi;
  b.cnt = __popcll(match);
  const bool inm = (match >> lane) & 1;
  const uint64_t lt = lanemask_lt(lane);
  const int dst = inm ? __popcll(match & lt) : b.cnt + __popcll(~match & lt);
  b.colpair = __builtin_amdgcn_ds_permute(dst << 2, lane);   // full permutation
  return b;
}

// The same routing for up to 64 * NH pairs (lane l holds ids l, l + 64, ...):
// work item pi serves its expert iff it is the expert's first pair; the
// expert's pairs in ascending order (its columns) go to cols[0, cnt) in LDS,
// written by wave 0 (the caller barriers before reading them).  Every wave
// computes the same values.  Whole-workgroup routine.
template <int NH>
__device__ __forceinline__ bool ballot_route_n(const SchedArgs& c, int pi, int tid, int* cols, int& e_out,
                                               int& cnt_out) {
  const int lane = tid & 63;
  int id[NH];
  bool ok[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {   // all loads issued before any is used
    const int i = 64 * h + lane;
    id[h] = i < c.n ? c.ids[i] : -1;
  }
  int e = -1;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    ok[h] = 64 * h + lane < c.n && (unsigned)id[h] < (unsigned)c.E;
    const int v = __shfl(id[h], pi & 63);
    if ((pi >> 6) == h) e = v;
  }
  uint64_t m[NH];
  int cnt = 0, first = -1;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    m[h] = __ballot(ok[h] && id[h] == e);
    if (first < 0 && m[h]) first = 64 * h + __ffsll((long long)m[h]) - 1;
    cnt += __popcll(m[h]);
  }
  const bool serve = (unsigned)e < (unsigned)c.E && first == pi;
  if (serve && tid < kWave) {
    const uint64_t lt = lanemask_lt(lane);
    int off = 0;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      if ((m[h] >> lane) & 1) cols[off + __popcll(m[h] & lt)] = 64 * h + lane;
      off += __popcll(m[h]);
    }
  }
  e_out = e;
  cnt_out = cnt;
  return serve;
}

}  // namespace mimoe
