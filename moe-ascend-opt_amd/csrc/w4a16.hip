// w4a16.hip -- W4A16 (AWQ-style int4 weights, 16-bit activations) fused MoE
// layer for gfx950: dispatch -> gate_up -> SiLU*mul -> down -> weighted
// combine -> cast, the dataflow of moe_forward_ptr_impl
// (Int8-gemm/q8_gemm.cpp:276-646) applied to the W4A16 format of the absent
// NPU grouped_gemv (README.md:19-30).
//
// MFMA form.  v_mfma_f32_16x16x32_{bf16,f16} with A = activations (16 token
// columns of one expert x 32 k) and B = dequantized weights (32 k x 16 output
// rows).  Lane l holds A row (token column) l%16 and B column (weight row)
// l%16 for k = 8*(l/16)..+7 of the step; D lane l holds weight row l%16 for
// token columns 4*(l/16)..+3.  Dequantization: (w >> 4p) & 0x000F000F | magic
// gives the 16-bit pair (offset + q_2p, offset + q_2p+1) exactly (offset 128
// with bf16 magic 0x4300, 1024 with fp16 magic 0x6400).  Offset and zero point
// are removed per group with the column sums X of the activations (an MFMA
// against an all-ones B):  y[t,n] += s[n,g] * (G[t,n] - (offset+z[n,g]) X[t,g]).
//
// Memory plan.  Every workgroup reads one contiguous block of weights, which
// its waves stream into registers with 16-byte loads; the small operands (the
// block's scales and zeros, and the activation rows of its columns) are
// copied into LDS with direct-to-LDS loads issued in the same burst, so a
// workgroup waits for memory once.
//
// Device layouts (built by the load-time repack from the AWQ wire format):
//   w13 tiles [e][j (I/16)][gate,up][g (H/128)][64 lanes][16 B]: a tile is
//     16 rows x 128 k; lane 16q+r holds row r, k = 128g+32q+8i+(0..7) in word
//     i, element 2p at bits 4p and 2p+1 at bits 4p+16.
//   w13 metadata, one block of 80*G1 bytes per (e, j): scales u32 [r 16][g]
//     (gate scale bits | up scale bits << 16), then zeros u8 [r][g]
//     (gate zero | up zero << 4).
//   w2 chunks [e][m (H/64)][c (I/32)][64 lanes][16 B]: lane 16q+r word jj
//     holds row h = 64m+16jj+r, k = 32c+8q+(0..7) (same pair packing).
//   w2 metadata, one block of 160*G2 bytes per (e, m) (G2 = I/128): scales
//     u16 [g2][r][jj], then zeros u16 [g2][r] (nibble jj).
//
// Paths (chosen on the host); rows of act/eout are indexed by pair i = t*K+k:
//   decode (T*K <= 64): two launches.  Work items are pairs (an item serves
//     its expert iff it is the expert's first pair; the others exit at once).
//     Phase 1: gate_up + SiLU*mul -> act.  Phase 2: down -> eout, then the
//     combine, elected per (token, 64-row block) by an arrival counter.
//   general: routing (in LDS up to 1024 pairs, else a routing kernel), phase 1,
//     phase 2 -> eout, and a combine kernel.
#pragma clang fp contract(off)
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"
#include "mi_moe_sched.hpp"

namespace mimoe {

template <int ACT>
__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (ACT == 1)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <int ACT>
struct W4Consts {
  static constexpr uint32_t magic = ACT == 1 ? 0x43004300u : 0x64006400u;
  static constexpr float offset = ACT == 1 ? 128.0f : 1024.0f;
  static constexpr uint32_t one2 = ACT == 1 ? 0x3f803f80u : 0x3c003c00u;
};

template <int ACT>
__device__ __forceinline__ u32x4_t deq4(uint32_t w) {
  constexpr uint32_t M = W4Consts<ACT>::magic;
  u32x4_t a;
  a.x = (w & 0x000f000fu) | M;
  a.y = ((w >> 4) & 0x000f000fu) | M;
  a.z = ((w >> 8) & 0x000f000fu) | M;
  a.w = ((w >> 12) & 0x000f000fu) | M;
  return a;
}

template <int ACT>
__device__ __forceinline__ u32x4_t ones4() {
  const uint32_t o = W4Consts<ACT>::one2;
  return u32x4_t{o, o, o, o};
}

__device__ __forceinline__ u32x4_t ldg16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ u32x4_t lds16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ u32x4_t zero4() { return u32x4_t{0, 0, 0, 0}; }

__device__ __forceinline__ uint64_t lanemask_lt(int lane) {
  return lane ? (~0ull >> (64 - lane)) : 0ull;
}
__device__ __forceinline__ uint64_t bits_range(int lo, int count) {
  const uint64_t m = count >= 64 ? ~0ull : ((1ull << count) - 1);
  return m << lo;
}

// scale bits -> fp32 (sdt: 1 bf16, 0 fp16; uniform)
__device__ __forceinline__ float scale_f32(uint32_t bits, int sdt) {
  return sdt ? bf16_to_f32(bits) : f16_to_f32(bits);
}

// acc[t] += s * (G[t] - c * X[t]) for the lane's 4 token columns
__device__ __forceinline__ void fold(f32x4_t& acc, const f32x4_t G, const f32x4_t X, float s,
                                     float c) {
  acc.x = __builtin_fmaf(s, __builtin_fmaf(-c, X.x, G.x), acc.x);
  acc.y = __builtin_fmaf(s, __builtin_fmaf(-c, X.y, G.y), acc.y);
  acc.z = __builtin_fmaf(s, __builtin_fmaf(-c, X.z, G.z), acc.z);
  acc.w = __builtin_fmaf(s, __builtin_fmaf(-c, X.w, G.w), acc.w);
}

// Copy nitems 16-byte items into LDS (contiguous from dst, 16-byte aligned)
// with direct-to-LDS loads (global_load_lds_dwordx4): wave instruction s moves
// items 64s..64s+63, lane l landing at dst + 1024s + 16l; instructions are
// dealt round-robin to the 4 waves.  src(k) is evaluated by every lane of a
// participating wave (it may shuffle).  The caller waits for vmcnt and
// barriers before reading the copy.
template <class Src>
__device__ __forceinline__ void stage_lds(unsigned char* dst, int nitems, int wave, int lane,
                                          Src src) {
  for (int s = wave; s * 64 < nitems; s += 4) {   // uniform per wave
    const int k = s * 64 + lane;
    const void* p = src(k < nitems ? k : nitems - 1);
    if (k < nitems) __builtin_amdgcn_global_load_lds(p, dst + s * 1024, 16, 0, 0);
  }
}

__device__ __forceinline__ void wait_all_and_sync() {
  __builtin_amdgcn_s_waitcnt(0);   // vmcnt = expcnt = lgkmcnt = 0 (direct-to-LDS copies landed)
  __syncthreads();
}

// ================================================================ routing
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

// Expert and columns of a work item: ballot routing (BALLOT) or the sorted
// routing arrays.
template <int BALLOT>
struct Cols {
  int e = 0, cnt = 0, colpair = 0;
  const int* pairs = nullptr;
  uint64_t vmask = 0;
  // pair index of column col; every lane of the wave must call it (BALLOT)
  __device__ __forceinline__ int pair(int col, bool valid) const {
    if constexpr (BALLOT) {
      const int p = __shfl(colpair, col & 63);
      return valid ? p : 0;
    } else {
      return valid ? pairs[col] : 0;
    }
  }
};

// Returns false when the item has nothing to do.
template <int BALLOT>
__device__ __forceinline__ bool get_cols(const SchedArgs& c, int item, int lane, void* route_lds,
                                         int* s_U, Cols<BALLOT>& out) {
  if constexpr (BALLOT) {
    const BallotCols b = ballot_cols(c, item, lane);
    out.e = b.e; out.cnt = b.cnt; out.colpair = b.colpair; out.vmask = b.vmask;
    return b.serve;
  } else {
    const RouteView rv = sched_route(c, reinterpret_cast<int*>(route_lds), s_U);
    if (item >= rv.U) return false;
    out.e = rv.active[item];
    const int p0 = rv.starts[out.e];
    out.cnt = rv.starts[out.e + 1] - p0;
    out.pairs = rv.pair + p0;
    return true;
  }
}

// ================================================================ phase 1
// Workgroup (item, 16-row slice j): gate/up rows j*16.. of the item's expert
// over all H (the 4 waves split the H groups), every routed pair of the expert
// in passes of p1_cols columns; SiLU*mul into act[pair].  Each wave keeps the
// weights of NB groups in flight together (NB from the host: min(8, H/512)
// rounded down to an instantiated size); loads past the wave's last group
// repeat its last group, so the load sequence has no branches.
// LDS: red [wave][gate,up][64][4] f32 | metadata 80*G1 B | x rows [p1_cols][H] | routing.
template <int ACT, int BALLOT, int NB>
__global__ __launch_bounds__(kBlock) void w4a16_phase1_kernel(W4Args a) {
  const SchedArgs& c = a.c;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_U;
  const int H = c.H, G1 = H >> 7, NI1 = c.I >> 4, P = a.p1_cols;
  float* red = reinterpret_cast<float*>(smem);
  unsigned char* meta = smem + kP1RedBytes;
  uint16_t* xs = reinterpret_cast<uint16_t*>(meta + 80 * G1);
  unsigned char* route = reinterpret_cast<unsigned char*>(xs) + (size_t)P * H * 2;
  const int item = blockIdx.x / NI1, j = blockIdx.x - item * NI1;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  Cols<BALLOT> cl;
  if (!get_cols<BALLOT>(c, item, lane, route, &s_U, cl)) return;  // uniform
  const int e = cl.e, cnt = cl.cnt;
  const size_t blk = (size_t)e * NI1 + j;
  const unsigned char* msrc = a.w13_m + blk * 80 * G1;
  stage_lds(meta, 5 * G1, wave, lane, [&](int k) { return (const void*)(msrc + 16 * k); });
  const int g0 = G1 * wave / 4, ng = G1 * (wave + 1) / 4 - g0;   // equal for all waves (G1 % 4 == 0)
  const char* wg = (const char*)a.w13 + (blk * 2 * G1 + g0) * 1024 + lane * 16;
  const char* wu = wg + (size_t)G1 * 1024;
  const uint32_t* msc = reinterpret_cast<const uint32_t*>(meta) + r * G1;
  const unsigned char* mz = meta + 64 * G1 + r * G1;
  const int HI = H >> 3;
  constexpr float off = W4Consts<ACT>::offset;
  for (int cb0 = 0; cb0 < cnt; cb0 += P) {
    const int ncol = min(P, cnt - cb0);
    stage_lds(reinterpret_cast<unsigned char*>(xs), ncol * HI, wave, lane, [&](int k) {
      const int cc = k / HI;
      const int t = cl.pair(cb0 + cc, true) / c.K;
      return (const void*)(c.x + (size_t)t * H + 8 * (k - cc * HI));
    });
    f32x4_t accg = {0, 0, 0, 0}, accu = {0, 0, 0, 0};
    for (int gb = 0; gb < ng; gb += NB) {
      u32x4_t wgv[NB], wuv[NB];
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        const size_t go = (size_t)min(gb + gi, ng - 1) * 1024;
        wgv[gi] = ldg16(wg + go);
        wuv[gi] = ldg16(wu + go);
      }
      if (gb == 0) wait_all_and_sync();   // metadata and x rows are in LDS
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        if (gb + gi >= ng) break;
        const int g = g0 + gb + gi;
        u32x4_t A[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) A[i] = r < ncol ? lds16(xs + r * H + 128 * g + 32 * q + 8 * i) : zero4();
        f32x4_t X = {0, 0, 0, 0}, Gg = {0, 0, 0, 0}, Gu = {0, 0, 0, 0};
        const uint32_t wgw[4] = {wgv[gi].x, wgv[gi].y, wgv[gi].z, wgv[gi].w};
        const uint32_t wuw[4] = {wuv[gi].x, wuv[gi].y, wuv[gi].z, wuv[gi].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          X = mfma16<ACT>(A[i], ones4<ACT>(), X);
          Gg = mfma16<ACT>(A[i], deq4<ACT>(wgw[i]), Gg);
          Gu = mfma16<ACT>(A[i], deq4<ACT>(wuw[i]), Gu);
        }
        const uint32_t sc = msc[g];
        const uint32_t zz = mz[g];
        fold(accg, Gg, X, scale_f32(sc & 0xffffu, a.sdt), off + (float)(zz & 0xfu));
        fold(accu, Gu, X, scale_f32(sc >> 16, a.sdt), off + (float)(zz >> 4));
      }
    }
    *reinterpret_cast<f32x4_t*>(red + ((wave * 2 + 0) * 64 + lane) * 4) = accg;
    *reinterpret_cast<f32x4_t*>(red + ((wave * 2 + 1) * 64 + lane) * 4) = accu;
    __syncthreads();
    if (tid < 64) {
      f32x4_t g = *reinterpret_cast<const f32x4_t*>(red + ((0 * 2 + 0) * 64 + tid) * 4);
      f32x4_t u = *reinterpret_cast<const f32x4_t*>(red + ((0 * 2 + 1) * 64 + tid) * 4);
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        g += *reinterpret_cast<const f32x4_t*>(red + ((w * 2 + 0) * 64 + tid) * 4);
        u += *reinterpret_cast<const f32x4_t*>(red + ((w * 2 + 1) * 64 + tid) * 4);
      }
      const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int col = cb0 + 4 * (tid >> 4) + v;
        const int p = cl.pair(col, col < cnt);
        if (col < cnt) a.act[(size_t)p * c.I + 16 * j + (tid & 15)] = from_f32<ACT>(silu_mul(gv[v], uv[v]));
      }
    }
    __syncthreads();   // red and xs are reused by the next pass
  }
}

// ================================================================ phase 2
// Workgroup (item, quad m = rows 64m..64m+63): down over all I (the waves
// split the 32-k chunks), for every routed pair of the item's expert in
// passes of p2_cols columns.
//   BALLOT = 0: eout[pair][64m..] (a combine kernel follows).
//   BALLOT = 1: eout rows are written with atomic exchanges; after them each
//     column adds one arrival to the counter of (token, m).  The workgroup
//     that completes a counter (all valid pairs of the token arrived) reads
//     the token's K rows back with atomic reads, forms
//     y = cast(sum_k w[t,k] * eout[t*K+k]) in k order -- Stage C1 + C2 of
//     Int8-gemm/q8_gemm.cpp:593-641 -- and puts the counter back to zero.
//     Data crosses workgroups only through atomic read-modify-writes.
// Each wave keeps the weights of NB chunks in flight together (NB from the
// host: min(12, I/128) rounded down to an instantiated size; loads past the
// wave's last chunk repeat it).
// LDS: red [wave][jj][64][4] f32 | metadata 160*G2 B | act rows [p2_cols][I] | routing.
template <int ACT, int BALLOT, int NB>
__global__ __launch_bounds__(kBlock) void w4a16_phase2_kernel(W4Args a) {
  const SchedArgs& c = a.c;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_U;
  __shared__ int s_done[64];
  __shared__ int s_nd;
  const int H = c.H, I = c.I, MQ = H >> 6, CH = I >> 5, G2 = I >> 7, P = a.p2_cols;
  float* red = reinterpret_cast<float*>(smem);
  unsigned char* meta = smem + kP2RedBytes;
  uint16_t* as = reinterpret_cast<uint16_t*>(meta + 160 * G2);
  unsigned char* route = reinterpret_cast<unsigned char*>(as) + (size_t)P * I * 2;
  const int item = blockIdx.x / MQ, m = blockIdx.x - item * MQ;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  Cols<BALLOT> cl;
  const bool serve = get_cols<BALLOT>(c, item, lane, route, &s_U, cl);
  if constexpr (BALLOT) {
    // a token whose ids are all invalid gets y = 0 (Int8-gemm/q8_gemm.cpp:329-332, 599-611)
    if (item % c.K == 0 && tid < 64) {
      const int t = item / c.K;
      if ((cl.vmask & bits_range(t * c.K, c.K)) == 0) c.y[(size_t)t * H + 64 * m + tid] = 0;
    }
  }
  if (!serve) return;  // uniform
  const int e = cl.e, cnt = cl.cnt;
  const size_t blk = (size_t)e * MQ + m;
  const unsigned char* msrc = a.w2_m + blk * 160 * G2;
  stage_lds(meta, 10 * G2, wave, lane, [&](int k) { return (const void*)(msrc + 16 * k); });
  const int c0 = CH * wave / 4, nc = CH * (wave + 1) / 4 - c0;   // equal for all waves (CH % 4 == 0)
  const char* wb = (const char*)a.w2 + (blk * CH + c0) * 1024 + lane * 16;
  const int II = I >> 3;
  constexpr float off = W4Consts<ACT>::offset;
  for (int cb0 = 0; cb0 < cnt; cb0 += P) {
    const int ncol = min(P, cnt - cb0);
    stage_lds(reinterpret_cast<unsigned char*>(as), ncol * II, wave, lane, [&](int k) {
      const int cc = k / II;
      const int p = cl.pair(cb0 + cc, true);
      return (const void*)(a.act + (size_t)p * I + 8 * (k - cc * II));
    });
    f32x4_t acc[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) acc[jj] = f32x4_t{0, 0, 0, 0};
    for (int cb = 0; cb < nc; cb += NB) {
      u32x4_t wv[NB];
#pragma unroll
      for (int ci = 0; ci < NB; ++ci) wv[ci] = ldg16(wb + (size_t)min(cb + ci, nc - 1) * 1024);
      if (cb == 0) wait_all_and_sync();   // metadata and act rows are in LDS
#pragma unroll
      for (int ci = 0; ci < NB; ++ci) {
        if (cb + ci >= nc) break;
        const int ch = c0 + cb + ci, g2 = ch >> 2;
        const u32x4_t A = r < ncol ? lds16(as + r * I + 32 * ch + 8 * q) : zero4();
        const f32x4_t X = mfma16<ACT>(A, ones4<ACT>(), f32x4_t{0, 0, 0, 0});
        const u32x2_t sv = *reinterpret_cast<const u32x2_t*>(meta + 8 * (g2 * 16 + r));
        const uint32_t zv = *reinterpret_cast<const uint16_t*>(meta + 128 * G2 + 2 * (g2 * 16 + r));
        const uint32_t ww[4] = {wv[ci].x, wv[ci].y, wv[ci].z, wv[ci].w};
        const uint32_t sb[4] = {sv.x & 0xffffu, sv.x >> 16, sv.y & 0xffffu, sv.y >> 16};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const f32x4_t G = mfma16<ACT>(A, deq4<ACT>(ww[jj]), f32x4_t{0, 0, 0, 0});
          fold(acc[jj], G, X, scale_f32(sb[jj], a.sdt), off + (float)((zv >> (4 * jj)) & 0xfu));
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      *reinterpret_cast<f32x4_t*>(red + ((wave * 4 + jj) * 64 + lane) * 4) = acc[jj];
    __syncthreads();
    {
      const int jj = tid >> 6, ln = tid & 63;
      f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(red + ((0 * 4 + jj) * 64 + ln) * 4);
#pragma unroll
      for (int w = 1; w < 4; ++w) v4 += *reinterpret_cast<const f32x4_t*>(red + ((w * 4 + jj) * 64 + ln) * 4);
      const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int col = cb0 + 4 * (ln >> 4) + v;
        const int p = cl.pair(col, col < cnt);
        if (col < cnt) {
          float* dst = c.eout + (size_t)p * H + 64 * m + 16 * jj + (ln & 15);
          if constexpr (BALLOT)
            __hip_atomic_exchange(reinterpret_cast<uint32_t*>(dst), __float_as_uint(vv[v]),
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            *dst = vv[v];
        }
      }
    }
    __syncthreads();   // red and as are reused by the next pass
  }
  if constexpr (BALLOT) {
    __builtin_amdgcn_s_waitcnt(0);   // this workgroup's exchanges are performed
    if (tid == 0) s_nd = 0;
    __syncthreads();
    if (tid < cnt) {                 // wave 0: lane == column
      const int t = cl.colpair / c.K;
      const int nv = __popcll(cl.vmask & bits_range(t * c.K, c.K));
      const uint32_t old = __hip_atomic_fetch_add(c.arrive + (size_t)t * MQ + m, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      if ((int)old + 1 == nv) s_done[atomicAdd(&s_nd, 1)] = t;
    }
    __syncthreads();
    const int nd = s_nd;
    for (int li = 0; li < nd; ++li) {
      const int t = s_done[li];
      if (tid < 64) {
        const int h = 64 * m + tid;
        float acc = 0.0f;
        for (int k = 0; k < c.K; ++k) {
          const int i = t * c.K + k;
          if ((unsigned)c.ids[i] >= (unsigned)c.E) continue;
          const uint32_t bits = __hip_atomic_fetch_or(reinterpret_cast<uint32_t*>(c.eout + (size_t)i * H + h),
                                                      0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const float prod = c.tw[i] * __uint_as_float(bits);
          acc = acc + prod;
        }
        c.y[(size_t)t * H + h] = from_f32<ACT>(acc);
      }
      if (tid == 0)
        __hip_atomic_exchange(c.arrive + (size_t)t * MQ + m, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ================================================================ repack
// AWQ wire (qweight [E][K][N/8], nibble slot {0,4,1,5,2,6,3,7}[n%8]) -> tiles.
__device__ __forceinline__ int awq_slot(int col) {
  return ((col & 1) << 2) | ((col >> 1) & 3);
}
__device__ __forceinline__ uint32_t awq_nib(const int32_t* base, int ncols, int k, int n) {
  return ((uint32_t)base[(size_t)k * (ncols / 8) + (n >> 3)] >> (4 * awq_slot(n & 7))) & 0xfu;
}

// w13: one thread per device u32 word; tile ti = 2j + which covers rows
// which*I + 16j .. +15 of the 2I outputs.
__global__ void awq_repack_w13(const int32_t* __restrict__ src, uint32_t* __restrict__ dst, int E,
                               int H, int I) {
  const int G = H >> 7, NT = 2 * (I >> 4), N = 2 * I;
  const size_t total = (size_t)E * NT * G * 256;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int wi = idx & 3, lane = (idx >> 2) & 63;
    size_t t = idx >> 8;
    const int g = t % G; t /= G;
    const int ti = t % NT;
    const int e = (int)(t / NT);
    const int n = (ti & 1) * I + 16 * (ti >> 1) + (lane & 15);
    const int k0 = 128 * g + 32 * (lane >> 4) + 8 * wi;
    const int32_t* base = src + (size_t)e * H * (N / 8);
    uint32_t word = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) word |= awq_nib(base, N, k0 + 2 * p + hh, n) << (4 * p + 16 * hh);
    dst[idx] = word;
  }
}

// w13 metadata blocks: one thread per (e, j, r, g).
__global__ void awq_repack_w13_meta(const uint16_t* __restrict__ scales, const int32_t* __restrict__ qzeros,
                                    unsigned char* __restrict__ m_dst, int E, int H, int I) {
  const int G = H >> 7, NI1 = I >> 4, N = 2 * I;
  const size_t total = (size_t)E * NI1 * 16 * G;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int g = idx % G;
    size_t t = idx / G;
    const int r = t % 16; t /= 16;
    const int j = t % NI1;
    const int e = (int)(t / NI1);
    const int ng = 16 * j + r, nu = I + 16 * j + r;
    unsigned char* blk = m_dst + ((size_t)e * NI1 + j) * 80 * G;
    const uint32_t sg = scales[((size_t)e * G + g) * N + ng], su = scales[((size_t)e * G + g) * N + nu];
    reinterpret_cast<uint32_t*>(blk)[r * G + g] = sg | (su << 16);
    const int32_t* zb = qzeros + (size_t)e * G * (N / 8);
    blk[64 * G + r * G + g] = (unsigned char)(awq_nib(zb, N, g, ng) | (awq_nib(zb, N, g, nu) << 4));
  }
}

// w2: one thread per device u32 word: (e, quad m, chunk c, lane, word jj).
__global__ void awq_repack_w2(const int32_t* __restrict__ src, uint32_t* __restrict__ dst, int E,
                              int H, int I) {
  const int CH = I >> 5, MQ = H >> 6;
  const size_t total = (size_t)E * MQ * CH * 256;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int jj = idx & 3, lane = (idx >> 2) & 63;
    size_t t = idx >> 8;
    const int cc = t % CH; t /= CH;
    const int m = t % MQ;
    const int e = (int)(t / MQ);
    const int h = 64 * m + 16 * jj + (lane & 15);
    const int k0 = 32 * cc + 8 * (lane >> 4);
    const int32_t* base = src + (size_t)e * I * (H / 8);
    uint32_t word = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) word |= awq_nib(base, H, k0 + 2 * p + hh, h) << (4 * p + 16 * hh);
    dst[idx] = word;
  }
}

// w2 metadata blocks: one thread per (e, m, g2, r).
__global__ void awq_repack_w2_meta(const uint16_t* __restrict__ scales, const int32_t* __restrict__ qzeros,
                                   unsigned char* __restrict__ m_dst, int E, int H, int I) {
  const int G2 = I >> 7, MQ = H >> 6;
  const size_t total = (size_t)E * MQ * G2 * 16;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int r = idx & 15;
    size_t t = idx >> 4;
    const int g2 = t % G2; t /= G2;
    const int m = t % MQ;
    const int e = (int)(t / MQ);
    unsigned char* blk = m_dst + ((size_t)e * MQ + m) * 160 * G2;
    uint32_t zq = 0;
    for (int jj = 0; jj < 4; ++jj) {
      const int h = 64 * m + 16 * jj + r;
      reinterpret_cast<uint16_t*>(blk)[(g2 * 16 + r) * 4 + jj] = scales[((size_t)e * G2 + g2) * H + h];
      zq |= awq_nib(qzeros + (size_t)e * G2 * (H / 8), H, g2, h) << (4 * jj);
    }
    reinterpret_cast<uint16_t*>(blk + 128 * G2)[g2 * 16 + r] = (uint16_t)zq;
  }
}

static int grid_for(size_t total) {
  size_t g = (total + 255) / 256;
  return (int)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

hipError_t launch_awq_repack_all(const int32_t* w13q, const int32_t* w13z, const uint16_t* w13s,
                                 const int32_t* w2q, const int32_t* w2z, const uint16_t* w2s,
                                 void* d13, unsigned char* d13m, void* d2, unsigned char* d2m, int E,
                                 int H, int I, hipStream_t st) {
  const int G = H >> 7, NT = 2 * (I >> 4), CH = I >> 5, MQ = H >> 6, G2 = I >> 7;
  hipLaunchKernelGGL(awq_repack_w13, dim3(grid_for((size_t)E * NT * G * 256)), dim3(256), 0, st,
                     w13q, (uint32_t*)d13, E, H, I);
  hipLaunchKernelGGL(awq_repack_w13_meta, dim3(grid_for((size_t)E * (I >> 4) * 16 * G)), dim3(256), 0,
                     st, w13s, w13z, d13m, E, H, I);
  hipLaunchKernelGGL(awq_repack_w2, dim3(grid_for((size_t)E * CH * MQ * 256)), dim3(256), 0, st,
                     w2q, (uint32_t*)d2, E, H, I);
  hipLaunchKernelGGL(awq_repack_w2_meta, dim3(grid_for((size_t)E * G2 * MQ * 16)), dim3(256), 0, st,
                     w2s, w2z, d2m, E, H, I);
  return hipGetLastError();
}

// ================================================================ launchers
// Instantiated batch sizes (weights per wave in flight together).
constexpr int kP1Batches[] = {1, 2, 4, 6, 8};
constexpr int kP2Batches[] = {1, 2, 4, 6, 8, 12};

static int pick_batch(const int* sizes, int count, int need) {
  int b = sizes[0];
  for (int i = 0; i < count; ++i)
    if (sizes[i] <= need) b = sizes[i];
  return b;
}

template <int ACT, int BALLOT, int NB>
static void launch_p1(const W4Args& a, int grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((w4a16_phase1_kernel<ACT, BALLOT, NB>), dim3(grid), dim3(kBlock), lds, st, a);
}
template <int ACT, int BALLOT, int NB>
static void launch_p2(const W4Args& a, int grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((w4a16_phase2_kernel<ACT, BALLOT, NB>), dim3(grid), dim3(kBlock), lds, st, a);
}

template <int ACT, int BALLOT>
static hipError_t launch_w4_t(const W4Args& a, int grid1, int grid2, hipStream_t st) {
  const size_t route = (BALLOT || a.c.route_global) ? 0 : route_lds_ints(a.c.E, a.c.n) * sizeof(int);
  const size_t lds1 = w4_p1_lds_bytes(a.c.H, a.p1_cols) + route;
  const size_t lds2 = w4_p2_lds_bytes(a.c.I, a.p2_cols) + route;
  switch (pick_batch(kP1Batches, 5, a.c.H / 512)) {
    case 1: launch_p1<ACT, BALLOT, 1>(a, grid1, lds1, st); break;
    case 2: launch_p1<ACT, BALLOT, 2>(a, grid1, lds1, st); break;
    case 4: launch_p1<ACT, BALLOT, 4>(a, grid1, lds1, st); break;
    case 6: launch_p1<ACT, BALLOT, 6>(a, grid1, lds1, st); break;
    default: launch_p1<ACT, BALLOT, 8>(a, grid1, lds1, st); break;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  switch (pick_batch(kP2Batches, 6, a.c.I / 128)) {
    case 1: launch_p2<ACT, BALLOT, 1>(a, grid2, lds2, st); break;
    case 2: launch_p2<ACT, BALLOT, 2>(a, grid2, lds2, st); break;
    case 4: launch_p2<ACT, BALLOT, 4>(a, grid2, lds2, st); break;
    case 6: launch_p2<ACT, BALLOT, 6>(a, grid2, lds2, st); break;
    case 8: launch_p2<ACT, BALLOT, 8>(a, grid2, lds2, st); break;
    default: launch_p2<ACT, BALLOT, 12>(a, grid2, lds2, st); break;
  }
  return hipGetLastError();
}

// ballot = 1 (T*K <= 64): grid1 = T*K * I/16, grid2 = T*K * H/64, phase 2
// combines and writes y.  ballot = 0: grid1 = U * I/16, grid2 = U * H/64 with
// U = min(T*K, E) and sorted routing; the caller launches the combine.
hipError_t launch_w4a16(const W4Args& a, int act, int ballot, int grid1, int grid2, hipStream_t st) {
  if (act == 1) return ballot ? launch_w4_t<1, 1>(a, grid1, grid2, st) : launch_w4_t<1, 0>(a, grid1, grid2, st);
  return ballot ? launch_w4_t<0, 1>(a, grid1, grid2, st) : launch_w4_t<0, 0>(a, grid1, grid2, st);
}

}  // namespace mimoe
