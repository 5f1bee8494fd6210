// w4a16_fused.hip -- the W4A16 decode layer in one launch (gfx950):
// dispatch -> gate_up -> SiLU*mul -> down -> k-order combine -> cast, the
// dataflow of moe_forward_ptr_impl (Int8-gemm/q8_gemm.cpp:276-646) for the
// W4A16 format of the absent NPU grouped_gemv (README.md:19-30), which fuses
// Gate_Proj + Up_Proj -> SiLU -> Down_Proj in one kernel.
//
// Grid (1D): workgroups [0, n1) are gate_up items, [n1, n1 + n2) down items.
//  * gate_up item (pair i, slice block js): serves its expert iff i is the
//    expert's first pair (wave ballots over all ids, the column order of the
//    reference's stable counting sort, moe_common.cpp:146-216).  S groups of
//    NW waves each take one 16-row slice of I; the NW waves of a group split
//    K (H).  gate and up rows are dequantized in registers right after their
//    16-byte loads and multiplied on the MFMA (A = activation columns,
//    B = weights), SiLU*mul in fp32, act[pair] rounded to the activation dtype.
//  * down item (token t, 16-row tile of H): wave k < K takes routed expert
//    k: its w2 tile over all I against act[t*K+k]; y = cast(sum_k w * out_k)
//    in k order (Int8-gemm/q8_gemm.cpp:593-641), no atomics.
//
// Hand-over inside the launch: no atomics, no flags, nothing to clear between
// calls, no L2 write-back or invalidate.  act values travel in 8-byte units
// (tag << 32 | two 16-bit values) written with agent-scope coherent stores
// (global_store ... sc1: written through, never left dirty in one XCD's L2);
// the tag identifies the dispatch (the queue's address mixed with the AQL
// packet index, which only grows on a queue), so a unit is valid for this call
// iff it carries this dispatch's tag, and a producer never waits for its
// stores.  A down wave issues its w2 tile and metadata loads first, then
// reads its whole act row with sc1 loads, checks every tag and unpacks it
// into LDS, reading it again until every unit is there.  The waits end: the dispatcher
// starts workgroups in index order and every down workgroup comes after all
// gate_up workgroups it reads from, so they are resident or finished when it
// starts, and gate_up workgroups wait on nothing.  The wait is still bounded
// (kSpinMax polls); a wave that gives up makes its token's tile NaN and sets
// the timeout word, so a failure is loud, never silent.
#pragma clang fp contract(off)
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"
#include "mi_moe_sched.hpp"
#include "w4a16_device.hpp"
#include "handover.hpp"

namespace mimoe {

constexpr int kFusedWaves = kW4FusedWaves;
constexpr int kUnitBatch = 6;       // act units per lane loaded together by a down wave (I = 768: all)
// From this many gate_up items per resident-workgroup slot on, the gate_up
// workgroups fill the slots and each takes several items (pipelined); below
// it, one workgroup per item.  Same-box graph replays: at 3 items per slot
// (bs 8) the pipelined form is 0.7 us faster per layer, at 1.5 (bs 4) 0.2 us
// slower, and with half or three quarters of the slots slower at every size.
constexpr long kPipelinedItemsPerSlot = 2;

// ---------------------------------------------------------------- gate_up role
// One item per workgroup (the grid holds every item): item (pair, block js of
// S slices).  LDS: red [S][NW][gate,up][64][4] f32 | metadata [S][80*G1] |
// hidden rows (the pipelined role's layout, its second reduction buffer unused).
template <int ACT, int SDT, int NB, int NW, int S>
__device__ __forceinline__ void fused_gate_up_one(const SchedArgs& c, const W4Args& a, const char* w13,
                                              const unsigned char* w13_m, int item, int js,
                                              unsigned char* smem) {
  const int H = c.H, G1 = H >> 7, NI1 = c.I >> 4, P = a.p1_cols, HI = H >> 3;
  float* red = reinterpret_cast<float*>(smem);
  unsigned char* meta = smem + 2 * S * p1_red_bytes(NW);
  uint16_t* xs = reinterpret_cast<uint16_t*>(meta + S * 80 * G1);
  const int j0 = js * S;
  // wave index, slice group and expert are uniform: SGPRs (weight addresses
  // are a scalar base plus the lane's 16-byte offset)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int sg = wave / NW, wi = wave - sg * NW;
  const int q = lane >> 4, r = lane & 15;
  const unsigned lane16 = 16u * (unsigned)lane;
  if (a.x_all)   // uniform; x is [T][H] contiguous
    stage_lds(reinterpret_cast<unsigned char*>(xs), c.T * HI, wave, kFusedWaves, lane,
              [&](int k) { return (const void*)(c.x + 8 * (size_t)k); });
  const BallotCols cl = ballot_cols(c, item, lane);
  if (!cl.serve) {   // uniform
    __builtin_amdgcn_s_waitcnt(0);   // no copy into LDS outlives the workgroup
    return;
  }
  auto pair_of = [&](int col) { return __shfl(cl.colpair, col & 63); };
  const float rk = 1.0f / (float)c.K;
  auto tok_of = [&](int pair) { return div_small(pair, rk); };
  const int e = __builtin_amdgcn_readfirstlane(cl.e), cnt = __builtin_amdgcn_readfirstlane(cl.cnt);
  const size_t blk = (size_t)e * NI1 + j0;   // S consecutive slices: contiguous weights and metadata
  const unsigned char* msrc = w13_m + blk * 80 * G1;
  stage_lds(meta, S * 5 * G1, wave, kFusedWaves, lane, [&](int k) { return (const void*)(msrc + 16 * k); });
  const int g0 = G1 * wi / NW, ng = G1 * (wi + 1) / NW - g0;   // equal for all waves (G1 % NW == 0)
  const char* wg = w13 + ((blk + sg) * 2 * G1 + g0) * 1024;     // gate: + g KB, up: + (G1 + g) KB
  const unsigned char* ms = meta + sg * 80 * G1;
  float* rsw = red + sg * (p1_red_bytes(NW) / 4);
  const unsigned tag = dispatch_tag32();
  constexpr float off = W4Consts<ACT>::offset;
  for (int cb0 = 0; cb0 < cnt; cb0 += P) {
    const int ncol = min(P, cnt - cb0);
    int xr;   // LDS row of this lane's column
    if (a.x_all) {
      xr = tok_of(pair_of(cb0 + min(r, ncol - 1)));
    } else {
      // the pass's hidden rows: row cc at xs + cc * H, in 1 KB chunks (H % 512 == 0)
      for (int cc = 0; cc < ncol; ++cc) {   // uniform
        const char* src = reinterpret_cast<const char*>(c.x + (size_t)tok_of(pair_of(cb0 + cc)) * H) + 16 * lane;
        unsigned char* dst = reinterpret_cast<unsigned char*>(xs + (size_t)cc * H);
        for (int ch = wave; ch < (HI >> 6); ch += kFusedWaves)
          __builtin_amdgcn_global_load_lds(src + 1024 * ch, dst + 1024 * ch, 16, 0, 0);
      }
      xr = min(r, ncol - 1);
    }
    const uint16_t* xrow = xs + xr * H + 32 * q;
    f32x4_t accg = {0, 0, 0, 0}, accu = {0, 0, 0, 0};
    issue_order_fence();
    for (int gb = 0; gb < ng; gb += NB) {
      u32x4_t wgv[NB], wuv[NB];
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        const char* p = wg + (size_t)(gb + gi) * 1024;
        wgv[gi] = ldg16(p + lane16);
        wuv[gi] = ldg16(p + (size_t)G1 * 1024 + lane16);
      }
      if (gb == 0) wait_copies_and_sync<2 * NB>();   // metadata and x rows are in LDS
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        const int g = g0 + gb + gi;
        u32x4_t A[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) A[i] = lds16(xrow + 128 * g + 8 * i);
        f32x4_t X = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) X = mfma16<ACT>(A[i], ones4<ACT>(), X);
        f32x4_t Gg = {0, 0, 0, 0}, Gu = {0, 0, 0, 0};
        const uint32_t wgw[4] = {wgv[gi].x, wgv[gi].y, wgv[gi].z, wgv[gi].w};
        const uint32_t wuw[4] = {wuv[gi].x, wuv[gi].y, wuv[gi].z, wuv[gi].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          Gg = mfma16<ACT>(A[i], deq4<ACT>(wgw[i]), Gg);
          Gu = mfma16<ACT>(A[i], deq4<ACT>(wuw[i]), Gu);
        }
        const uint32_t sc = reinterpret_cast<const uint32_t*>(ms)[r * G1 + g];
        const uint32_t zz = ms[64 * G1 + r * G1 + g];
        fold(accg, Gg, X, scale_of<SDT>(sc & 0xffffu), off + (float)(zz & 0xfu));
        fold(accu, Gu, X, scale_of<SDT>(sc >> 16), off + (float)(zz >> 4));
      }
    }
    *reinterpret_cast<f32x4_t*>(rsw + ((wi * 2 + 0) * 64 + lane) * 4) = accg;
    *reinterpret_cast<f32x4_t*>(rsw + ((wi * 2 + 1) * 64 + lane) * 4) = accu;
    __syncthreads();
    if (tid < 64 * S) {   // wave s sums slice s: lane ln holds row ln & 15 of columns 4(ln >> 4)..+3
      const int s = tid >> 6, ln = tid & 63;
      const float* rs = red + s * (p1_red_bytes(NW) / 4);
      f32x4_t g = *reinterpret_cast<const f32x4_t*>(rs + ((0 * 2 + 0) * 64 + ln) * 4);
      f32x4_t u = *reinterpret_cast<const f32x4_t*>(rs + ((0 * 2 + 1) * 64 + ln) * 4);
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        g += *reinterpret_cast<const f32x4_t*>(rs + ((w * 2 + 0) * 64 + ln) * 4);
        u += *reinterpret_cast<const f32x4_t*>(rs + ((w * 2 + 1) * 64 + ln) * 4);
      }
      const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int col = cb0 + 4 * (ln >> 4) + v;
        const int p = pair_of(col);
        // rows r and r^1 are lanes ln and ln^1: one tagged unit per row pair;
        // the 8 units of a (pair, slice) are one 64-byte line
        const uint32_t bits = from_f32<ACT>(silu_mul_fast(gv[v], uv[v]));
        const uint32_t other = (uint32_t)__shfl_xor((int)bits, 1);
        // only the pass's ncol columns hold its results (the other MFMA
        // columns repeat its last one): a unit is stored once, final
        if (4 * (ln >> 4) + v < ncol && (ln & 1) == 0)
          store_agent(a.tact + (size_t)p * (c.I >> 1) + 8 * (j0 + s) + ((ln & 15) >> 1),
                      ((unsigned long long)tag << 32) | bits | (other << 16));
      }
    }
    __syncthreads();   // red and xs are reused by the next pass
  }
}

// Pipelined gate_up role (at least kPipelinedItemsPerSlot items per slot):
// workgroup g takes the items g, g + NG, g + 2 NG, ... (item = pair x block of
// S slices); an item serves its expert iff its pair is the expert's first
// pair.  The ids are read once per workgroup and every item's routing
// (ballots over them) needs no memory access, so an item that does not serve
// costs nothing.  Units (an item's passes of P token columns) are software
// pipelined: a unit's metadata / hidden-row copies and first weight batch are
// issued, then the previous unit's epilogue (cross-wave sums, SiLU*mul, act
// stores) runs from the other reduction buffer while they arrive.
// LDS: red [2][S][NW][gate,up][64][4] f32 | metadata [S][80*G1] | hidden rows.
template <int ACT, int SDT, int NB, int NW, int S>
__device__ __forceinline__ void fused_gate_up(const SchedArgs& c, const W4Args& a, const char* w13,
                                              const unsigned char* w13_m, int g, int NG, int njs,
                                              unsigned char* smem) {
  const int H = c.H, G1 = H >> 7, NI1 = c.I >> 4, HI = H >> 3;
  // token columns per pass: all 16 MFMA columns when every hidden row is in LDS
  const int P = a.x_all ? 16 : a.p1_cols;
  const int RB = p1_red_bytes(NW) / 4;   // floats of one slice's reduction buffer
  float* red = reinterpret_cast<float*>(smem);
  unsigned char* meta = smem + 2 * S * p1_red_bytes(NW);
  uint16_t* xs = reinterpret_cast<uint16_t*>(meta + S * 80 * G1);
  // wave index and slice group are uniform: SGPRs (weight addresses are a
  // scalar base plus the lane's 16-byte offset)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int sg = wave / NW, wi = wave - sg * NW;
  const int q = lane >> 4, r = lane & 15;
  const unsigned lane16 = 16u * (unsigned)lane;
  if (a.x_all)   // uniform; x is [T][H] contiguous
    stage_lds(reinterpret_cast<unsigned char*>(xs), c.T * HI, wave, kFusedWaves, lane,
              [&](int k) { return (const void*)(c.x + 8 * (size_t)k); });
  // the routing's inputs, read once: lane l holds pair l's expert id
  const int myid = lane < c.n ? c.ids[lane] : -1;
  const bool myvalid = lane < c.n && (unsigned)myid < (unsigned)c.E;
  const float rk = 1.0f / (float)c.K;
  auto tok_of = [&](int pair) { return div_small(pair, rk); };
  const unsigned tag = dispatch_tag32();
  const int g0 = G1 * wi / NW, ng = G1 * (wi + 1) / NW - g0;   // equal for all waves (G1 % NW == 0)
  const unsigned char* ms = meta + sg * 80 * G1;
  constexpr float off = W4Consts<ACT>::offset;
  // the previous unit, whose epilogue is pending
  bool pend = false;
  int p_buf = 0, p_ncol = 0, p_j0 = 0, p_cb0 = 0, p_colpair = 0;
  auto epilogue = [&]() {
    if (tid < 64 * S) {   // wave s sums slice s: lane ln holds row ln & 15 of columns 4(ln >> 4)..+3
      const int s = tid >> 6, ln = tid & 63;
      const float* rs = red + (p_buf * S + s) * RB;
      f32x4_t gs = *reinterpret_cast<const f32x4_t*>(rs + ((0 * 2 + 0) * 64 + ln) * 4);
      f32x4_t us = *reinterpret_cast<const f32x4_t*>(rs + ((0 * 2 + 1) * 64 + ln) * 4);
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        gs += *reinterpret_cast<const f32x4_t*>(rs + ((w * 2 + 0) * 64 + ln) * 4);
        us += *reinterpret_cast<const f32x4_t*>(rs + ((w * 2 + 1) * 64 + ln) * 4);
      }
      const float gv[4] = {gs.x, gs.y, gs.z, gs.w}, uv[4] = {us.x, us.y, us.z, us.w};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int col = p_cb0 + 4 * (ln >> 4) + v;
        const int pr = __shfl(p_colpair, col & 63);
        // rows r and r^1 are lanes ln and ln^1: one tagged unit per row pair;
        // the 8 units of a (pair, slice) are one 64-byte line
        const uint32_t bits = from_f32<ACT>(silu_mul_fast(gv[v], uv[v]));
        const uint32_t other = (uint32_t)__shfl_xor((int)bits, 1);
        // only the pass's ncol columns hold its results (the other MFMA
        // columns repeat its last one): a unit is stored once, final
        if (4 * (ln >> 4) + v < p_ncol && (ln & 1) == 0)
          store_agent(a.tact + (size_t)pr * (c.I >> 1) + 8 * (p_j0 + s) + ((ln & 15) >> 1),
                      ((unsigned long long)tag << 32) | bits | (other << 16));
      }
    }
  };
  const int n_items = c.n * njs;
  int unit = 0;
  for (int item = g; item < n_items; item += NG) {
    const int pi = item / njs, js = item - pi * njs;   // uniform
    // routing by ballots (pair pi serves iff it is its expert's first pair);
    // column j of the expert is its j-th pair in ascending order, the order of
    // the reference's stable counting sort (moe_common.cpp:146-216)
    const int e = __shfl(myid, pi);
    const uint64_t match = __ballot(myvalid && myid == e);
    if (!((unsigned)e < (unsigned)c.E && (__ffsll((long long)match) - 1) == pi)) continue;   // uniform
    const int cnt = __builtin_amdgcn_readfirstlane(__popcll(match));
    const bool inm = (match >> lane) & 1;
    const uint64_t lt = lanemask_lt(lane);
    const int dst = inm ? __popcll(match & lt) : cnt + __popcll(~match & lt);
    const int colpair = __builtin_amdgcn_ds_permute(dst << 2, lane);   // lane l: pair of column l
    const int eu = __builtin_amdgcn_readfirstlane(e);
    const int j0 = js * S;
    const size_t blk = (size_t)eu * NI1 + j0;   // S consecutive slices: contiguous weights and metadata
    const char* wg = w13 + ((blk + sg) * 2 * G1 + g0) * 1024;     // gate: + g KB, up: + (G1 + g) KB
    for (int cb0 = 0; cb0 < cnt; cb0 += P, ++unit) {
      const int ncol = min(P, cnt - cb0);
      // this unit's LDS operands (the previous unit's readers passed the last barrier)
      if (cb0 == 0) {
        const unsigned char* msrc = w13_m + blk * 80 * G1;
        stage_lds(meta, S * 5 * G1, wave, kFusedWaves, lane, [&](int k) { return (const void*)(msrc + 16 * k); });
      }
      int xr;   // LDS row of this lane's column
      if (a.x_all) {
        xr = tok_of(__shfl(colpair, (cb0 + min(r, ncol - 1)) & 63));
      } else {
        // the pass's hidden rows: row cc at xs + cc * H, in 1 KB chunks (H % 512 == 0)
        for (int cc = 0; cc < ncol; ++cc) {   // uniform
          const char* src =
              reinterpret_cast<const char*>(c.x + (size_t)tok_of(__shfl(colpair, (cb0 + cc) & 63)) * H) + 16 * lane;
          unsigned char* xd = reinterpret_cast<unsigned char*>(xs + (size_t)cc * H);
          for (int ch = wave; ch < (HI >> 6); ch += kFusedWaves)
            __builtin_amdgcn_global_load_lds(src + 1024 * ch, xd + 1024 * ch, 16, 0, 0);
        }
        xr = min(r, ncol - 1);
      }
      const uint16_t* xrow = xs + xr * H + 32 * q;
      issue_order_fence();
      u32x4_t wgv[NB], wuv[NB];
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        const char* p = wg + (size_t)gi * 1024;
        wgv[gi] = ldg16(p + lane16);
        wuv[gi] = ldg16(p + (size_t)G1 * 1024 + lane16);
      }
      wait_copies_and_sync<2 * NB>();   // metadata and x rows are in LDS
      if (pend) epilogue();   // the previous unit, while this unit's weights arrive
      f32x4_t accg = {0, 0, 0, 0}, accu = {0, 0, 0, 0};
      for (int gb = 0; gb < ng; gb += NB) {
        if (gb > 0) {
#pragma unroll
          for (int gi = 0; gi < NB; ++gi) {
            const char* p = wg + (size_t)(gb + gi) * 1024;
            wgv[gi] = ldg16(p + lane16);
            wuv[gi] = ldg16(p + (size_t)G1 * 1024 + lane16);
          }
        }
#pragma unroll
        for (int gi = 0; gi < NB; ++gi) {
          const int gg = g0 + gb + gi;
          u32x4_t A[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) A[i] = lds16(xrow + 128 * gg + 8 * i);
          f32x4_t X = {0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i) X = mfma16<ACT>(A[i], ones4<ACT>(), X);
          f32x4_t Gg = {0, 0, 0, 0}, Gu = {0, 0, 0, 0};
          const uint32_t wgw[4] = {wgv[gi].x, wgv[gi].y, wgv[gi].z, wgv[gi].w};
          const uint32_t wuw[4] = {wuv[gi].x, wuv[gi].y, wuv[gi].z, wuv[gi].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            Gg = mfma16<ACT>(A[i], deq4<ACT>(wgw[i]), Gg);
            Gu = mfma16<ACT>(A[i], deq4<ACT>(wuw[i]), Gu);
          }
          const uint32_t sc = reinterpret_cast<const uint32_t*>(ms)[r * G1 + gg];
          const uint32_t zz = ms[64 * G1 + r * G1 + gg];
          fold(accg, Gg, X, scale_of<SDT>(sc & 0xffffu), off + (float)(zz & 0xfu));
          fold(accu, Gu, X, scale_of<SDT>(sc >> 16), off + (float)(zz >> 4));
        }
      }
      float* rsw = red + ((unit & 1) * S + sg) * RB;
      *reinterpret_cast<f32x4_t*>(rsw + ((wi * 2 + 0) * 64 + lane) * 4) = accg;
      *reinterpret_cast<f32x4_t*>(rsw + ((wi * 2 + 1) * 64 + lane) * 4) = accu;
      __syncthreads();   // the sums are visible; metadata and x rows are free for the next unit
      pend = true;
      p_buf = unit & 1;
      p_ncol = ncol;
      p_j0 = j0;
      p_cb0 = cb0;
      p_colpair = colpair;
    }
  }
  if (pend) epilogue();
  else __builtin_amdgcn_s_waitcnt(0);   // served nothing: no hidden-row copy outlives the workgroup
}

// ---------------------------------------------------------------- down role
// Down item (token t, RT consecutive 16-row tiles of H from tile0, within one
// quad of 64 rows).  LDS: act rows [8][I] | metadata [8][RT][SEC] | outputs
// [8][16 RT] f32 | state [8] | routing weights [8] f32.
template <int ACT, int SDT, int NB, int RT>
__device__ __forceinline__ void fused_down(const SchedArgs& c, const W4Args& a, const char* w2,
                                           const unsigned char* w2_m, int t, int tile0, unsigned char* smem) {
  const int K = c.K, E = c.E, H = c.H, I = c.I;
  const int MQ = H >> 6, G2 = I >> 7, SEC = w2_meta_sec_bytes(G2);
  const int m = tile0 >> 2, jj = tile0 & 3;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int q = lane >> 4, r = lane & 15;
  const unsigned lane16 = 16u * (unsigned)lane;
  uint16_t* as = reinterpret_cast<uint16_t*>(smem);
  unsigned char* meta = smem + (size_t)kFusedWaves * I * 2;
  float* outs = reinterpret_cast<float*>(meta + (size_t)kFusedWaves * RT * SEC);
  int* state = reinterpret_cast<int*>(outs + 16 * RT * kFusedWaves);   // 0 invalid id, 1 valid, 2 wait gave up
  float* tws = reinterpret_cast<float*>(state + kFusedWaves);
  constexpr float off = W4Consts<ACT>::offset;
  // the combine's routing weights, copied into LDS now (wave 0's wait below
  // covers the copy; no registers held)
  if (tid < K) __builtin_amdgcn_global_load_lds(c.tw + t * K + tid, tws, 4, 0, 0);
  if (wave < K) {   // uniform: wave k takes routed expert k of token t
    const int i = t * K + wave;
    const int e = __builtin_amdgcn_readfirstlane(c.ids[i]);
    // an invalid id computes on expert 0 and its output is ignored
    const bool ok = (unsigned)e < (unsigned)E;
    const size_t sec0 = ((size_t)(ok ? e : 0) * MQ + m) * 4 + jj;   // the RT tiles: contiguous
    unsigned char* mdst = meta + wave * RT * SEC;
    for (int l = lane; l < RT * SEC / 16; l += 64)
      __builtin_amdgcn_global_load_lds(w2_m + sec0 * SEC + 16 * l, mdst + (l - lane) * 16, 16, 0, 0);
    const char* wb = w2 + sec0 * G2 * 1024 + lane16;   // tile rt: + rt * G2 KB
    u32x4_t wv[RT][NB];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) wv[rt][gi] = ldg16(wb + (size_t)(rt * G2 + gi) * 1024);   // in flight during the wait
    int st = ok ? 1 : 0;
    if (ok) {
      // act row i: I/2 tagged units; slice j's units are the line at unit 8j.
      // read_row reads, checks and unpacks the whole row into LDS.
      const unsigned tag = dispatch_tag32();
      const unsigned long long* row = a.tact + (size_t)i * (I >> 1);
      const int nunits = I >> 1;
      unsigned* dst = reinterpret_cast<unsigned*>(as + (size_t)wave * I);
      auto read_row = [&]() {
        bool whole = true;
        for (int u0 = 0; u0 < nunits; u0 += 64 * kUnitBatch) {
          unsigned long long v[kUnitBatch];
#pragma unroll
          for (int b = 0; b < kUnitBatch; ++b) {
            const int u = u0 + 64 * b + lane;
            v[b] = u < nunits ? load_agent(row + u) : ((unsigned long long)tag << 32);
          }
#pragma unroll
          for (int b = 0; b < kUnitBatch; ++b) {
            const int u = u0 + 64 * b + lane;
            whole = whole && (unsigned)(v[b] >> 32) == tag;
            if (u < nunits) dst[u] = (unsigned)v[b];
          }
        }
        return __all(whole);
      };
      // Poll by reading the whole row: the read that finds every unit
      // tagged is also the one that delivers the row (one round trip after
      // the last unit lands; a first pass over per-slice sentinel units
      // added one: bs 1 / 2 / 8 10.60 / 14.30 / 30.4 -> 10.47 / 14.13 /
      // 30.1 us, same box).
      for (int polls = 0; !read_row();) {
        if (++polls > kSpinMax) {
          st = 2;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (st == 2 && lane == 0) store_agent(a.tact + (size_t)64 * (I >> 1), 1ull);
    }
    if (lane == 0) state[wave] = st;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's metadata and first weights
    issue_order_fence();
    const uint16_t* arow = as + (size_t)wave * I + 8 * q;
    f32x4_t acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4_t{0, 0, 0, 0};
    for (int gb = 0; gb < G2; gb += NB) {
      if (gb > 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int gi = 0; gi < NB; ++gi) wv[rt][gi] = ldg16(wb + (size_t)(rt * G2 + gb + gi) * 1024);
      }
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        const int g2 = gb + gi;
        u32x4_t A[4];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) A[cc] = lds16(arow + 128 * g2 + 32 * cc);
        f32x4_t X = {0, 0, 0, 0};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) X = mfma16<ACT>(A[cc], ones4<ACT>(), X);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          f32x4_t G = {0, 0, 0, 0};
          const uint32_t ww[4] = {wv[rt][gi].x, wv[rt][gi].y, wv[rt][gi].z, wv[rt][gi].w};
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) G = mfma16<ACT>(A[cc], deq4<ACT>(ww[cc]), G);
          const unsigned char* sec = mdst + rt * SEC;
          fold(acc[rt], G, X, scale_of<SDT>(reinterpret_cast<const uint16_t*>(sec)[16 * g2 + r]),
               off + w2_zero(sec, G2, g2, r));
        }
      }
    }
    if (lane < 16)   // column 0: lanes (r, q = 0)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) outs[16 * (RT * wave + rt) + lane] = acc[rt].x;
  }
  __syncthreads();
  if (tid < 16 * RT) {
    float yv = 0.0f;
    bool gave_up = false;
#pragma unroll
    for (int k = 0; k < kW4FusedWaves; ++k) {
      const int s = k < K ? state[k] : 0;
      if (s) {
        gave_up |= s == 2;
        const float prod = tws[k] * outs[16 * RT * k + tid];
        yv = yv + prod;
      }
    }
    c.y[(size_t)t * H + 16 * tile0 + tid] = gave_up ? (uint16_t)0x7fc0u : from_f32<ACT>(yv);
  }
}

// ---------------------------------------------------------------- kernel
// The leading arguments repeat fields of a: gfx950 preloads the first
// kernel-argument dwords into SGPRs at wave launch
// (-amdgpu-kernarg-preload-count), so the role choice, the ids read and the
// weight addresses do not wait for an argument fetch.
template <int ACT, int SDT, int NB1, int NW, int S, int NB2, int RT>
__global__ __launch_bounds__(kW4FusedWaves * kWave) __attribute__((amdgpu_waves_per_eu(4)))
void w4a16_decode_kernel(const int32_t* ids, const uint16_t* x, const char* w13, const unsigned char* w13_m,
                         const char* w2, const unsigned char* w2_m, int n1, int njs, W4Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  SchedArgs c = a.c;
  c.ids = ids;
  c.x = x;
  const int b = blockIdx.x;
  if (b < n1) {   // uniform: n1 gate_up workgroups, then the down items
    if (n1 == c.n * njs) {   // one workgroup per item
      const int item = b / njs;
      fused_gate_up_one<ACT, SDT, NB1, NW, S>(c, a, w13, w13_m, item, b - item * njs, smem);
    } else {
      fused_gate_up<ACT, SDT, NB1, NW, S>(c, a, w13, w13_m, b, n1, njs, smem);
    }
  } else {
    const int nt = (c.H >> 4) / RT, d = b - n1, t = d / nt;
    fused_down<ACT, SDT, NB2, RT>(c, a, w2, w2_m, t, RT * (d - t * nt), smem);
  }
}

template <int ACT, int SDT, int NB1, int NW, int S, int NB2, int RT>
static hipError_t launch_fused_t(const W4Args& a, int njs, int ngu, size_t lds, hipStream_t st) {
  if (lds > kMaxLds)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(w4a16_decode_kernel<ACT, SDT, NB1, NW, S, NB2, RT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  const int n1 = ngu, n2 = a.c.T * (a.c.H >> 4) / RT;
  hipLaunchKernelGGL((w4a16_decode_kernel<ACT, SDT, NB1, NW, S, NB2, RT>), dim3(n1 + n2), dim3(kW4FusedWaves * kWave),
                     lds, st, a.c.ids, a.c.x, (const char*)a.w13, a.w13_m, (const char*)a.w2, a.w2_m, n1, njs, a);
  return hipGetLastError();
}

template <int ACT, int SDT, int NW, int S, int RT>
static hipError_t dispatch_fused_nb(const W4Args& a, int nb1, int nb2, int njs, int ngu, size_t lds,
                                    hipStream_t st) {
#define FUSED_NB2(NB1_)                                                                        \
  if (nb1 == NB1_) {                                                                           \
    if (nb2 == 6) return launch_fused_t<ACT, SDT, NB1_, NW, S, 6, RT>(a, njs, ngu, lds, st); \
    if (nb2 == 4) return launch_fused_t<ACT, SDT, NB1_, NW, S, 4, RT>(a, njs, ngu, lds, st); \
    if (nb2 == 3) return launch_fused_t<ACT, SDT, NB1_, NW, S, 3, RT>(a, njs, ngu, lds, st); \
    if (nb2 == 2) return launch_fused_t<ACT, SDT, NB1_, NW, S, 2, RT>(a, njs, ngu, lds, st); \
    if (nb2 == 1) return launch_fused_t<ACT, SDT, NB1_, NW, S, 1, RT>(a, njs, ngu, lds, st); \
  }
  FUSED_NB2(1) FUSED_NB2(2) FUSED_NB2(3) FUSED_NB2(4)
#undef FUSED_NB2
  return hipErrorInvalidValue;
}

template <int ACT, int SDT>
static hipError_t dispatch_fused(const W4Args& a, const W4FusedPlan& p, hipStream_t st) {
  if (p.nw == 8) return dispatch_fused_nb<ACT, SDT, 8, 1, 1>(a, p.nb1, p.nb2, p.njs, p.ngu, p.lds, st);
  if (p.rt == 2) return dispatch_fused_nb<ACT, SDT, 4, 2, 2>(a, p.nb1, p.nb2, p.njs, p.ngu, p.lds, st);
  return dispatch_fused_nb<ACT, SDT, 4, 2, 1>(a, p.nb1, p.nb2, p.njs, p.ngu, p.lds, st);
}

// largest of {1, 2, 3, 4, 6} (up to cap) that divides need
static int fused_batch(int need, int cap) {
  static const int sizes[] = {1, 2, 3, 4, 6};
  int b = 1;
  for (int s : sizes)
    if (s <= cap && need % s == 0) b = s;
  return b;
}

// Slots: workgroups resident at once (2 per CU at the kernel's register
// budget).  Down items take 2 tiles where that makes every workgroup of the
// call resident at once, or where 1-tile items would need more than one round
// of slots; otherwise 1 (more items in flight).
W4FusedPlan w4a16_fused_plan(int T, int K, int H, int I, int x_all, int p1_cols, int num_cu) {
  W4FusedPlan p{};
  const int n = T * K, G1 = H / 128, G2 = I / 128;
  p.nw = (n <= kW4WideMaxPairs && G1 % 8 == 0) ? 8 : 4;
  const int S = kW4FusedWaves / p.nw;
  p.njs = (I / 16) / S;
  p.nb1 = fused_batch(G1 / p.nw, 4);
  p.nb2 = fused_batch(G2, 6);
  const long slots = 2L * num_cu, items = (long)n * p.njs, tiles = (long)T * (H / 16);
  // gate_up workgroups: one per item, or one per slot taking several items
  const bool pipelined = items >= kPipelinedItemsPerSlot * slots;
  const long n1 = pipelined ? slots : items;
  p.ngu = (int)(n1 > 0 ? n1 : 1);
  p.rt = 1;
  if (p.nw == 4 && (H / 16) % 2 == 0 && (tiles > slots || (n1 + tiles > slots && n1 + tiles / 2 <= slots))) p.rt = 2;
  const size_t gate_up = w4_fused_gate_up_lds_bytes(H, x_all ? T : p1_cols, p.nw);
  const size_t down = w4_fused_down_lds_bytes(I, p.rt);
  p.lds = gate_up > down ? gate_up : down;
  // A down item that needs more than one weight batch (I/128 > 6) sits on the
  // critical path when no pipelined gate_up work overlaps it: MiniMax-M2 shape
  // (I = 1536) at bs 1, same-box graph replays, 22.7-22.9 us in one launch
  // against 19.7-20.1 us in two; at bs 8 (pipelined) one launch is 1.5 us faster.
  const bool down_chained = G2 > p.nb2 && !pipelined;
  p.ok = K <= kW4FusedWaves && n <= kW4FusedMaxPairs && G1 % p.nw == 0 && (I / 16) % S == 0 && I <= kTagActMaxI &&
         !down_chained && p.lds <= device_max_lds();
  return p;
}

hipError_t launch_w4a16_fused(const W4Args& a, const W4FusedPlan& p, int act, hipStream_t st) {
  if (!p.ok) return hipErrorInvalidValue;
  if (act == 1) return a.sdt == 1 ? dispatch_fused<1, 1>(a, p, st) : dispatch_fused<1, 0>(a, p, st);
  return a.sdt == 1 ? dispatch_fused<0, 1>(a, p, st) : dispatch_fused<0, 0>(a, p, st);
}

}  // namespace mimoe
