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
//   w2 words [e][m (H/64)][jj 4][g2 (I/128)][64 lanes][16 B]: lane 16q+r word
//     cc holds row h = 64m+16jj+r, k = 128g2+32cc+8q+(0..7) (same pair packing).
//   w2 metadata, one section of w2_meta_sec_bytes(G2) bytes (40*G2 rounded up
//     to 16) per (e, m, jj) (G2 = I/128): scales u16 [g2][r], then zeros
//     [g2][r/2] (row r in nibble r&1).
//
// Paths (chosen on the host); rows of act/eout are indexed by pair i = t*K+k:
//   decode (T*K <= 64, K <= kDownMaxK): two launches.  Phase 1 (gate_up +
//     SiLU*mul -> act) has a work item per pair; an item serves its expert iff
//     it is the expert's first pair, the others exit at once.  The down kernel
//     has a workgroup per (token, 16-row tile) with a wave per routed expert,
//     and combines in LDS.
//   sorted (any other T, K): the routing kernel (with 64-row tiles of each
//     expert's rows), the grouped GEMMs gate_up (-> act) and down (-> eout),
//     and the combine kernel.
#pragma clang fp contract(off)
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"
#include "mi_moe_sched.hpp"
#include "w4a16_device.hpp"

namespace mimoe {

// ================================================================ phase 1
// Register budgets, as waves per SIMD: phase 1 spills above 4; the down
// kernel (8-wave workgroups) fits 6 without spills, i.e. 3 workgroups per CU.
constexpr int kP1WavesPerEU = 4;
constexpr int kDownWavesPerEU = 6;
// Workgroup (item, slices j = S*js .. S*js+S-1 of 16 rows): gate/up rows of
// the item's expert over all H (the NW waves split the H/128 groups), every
// routed pair of the expert in passes of p1_cols columns; SiLU*mul into
// act[pair].  Each wave keeps the weights of NB groups x S slices in flight
// together (NB, from the host, divides the wave's groups); the column sums X of a
// group are shared by the S slices.  Lanes of columns past the pass read the
// pass's last column, so the loop body has no branches; their results are
// never stored.  Hidden rows: with a.x_all the rows of all T tokens are copied
// into LDS at kernel start, in parallel with the routing read; otherwise the
// rows of each pass's columns are copied once the routing is known.  Work
// item = pair index; the items of an expert's later pairs exit at once.
// LDS (w4_p1_lds_bytes): red [S][wave][gate,up][64][4] f32 | metadata S x 80*G1 B | x rows.
template <int ACT, int SDT, int NB, int S, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(kP1WavesPerEU)))
void w4a16_phase1_kernel(const int32_t* ids, const uint16_t* x, const char* w13, const unsigned char* w13_m, int T,
                         int n, int E, int H, int I, int x_all, int K, W4Args a) {
  // the leading arguments repeat fields of a: gfx950 preloads the first 14
  // dwords of them into SGPRs at wave launch (-amdgpu-kernarg-preload-count),
  // so the x copy, the ids read and the weight addresses do not wait for a
  // kernel-argument fetch
  SchedArgs c = a.c;
  c.ids = ids;
  c.x = x;
  c.T = T;
  c.n = n;
  c.E = E;
  c.H = H;
  c.I = I;
  c.K = K;
  extern __shared__ __align__(16) unsigned char smem[];
  const int G1 = H >> 7, NI1 = I >> 4, P = a.p1_cols, HI = H >> 3;
  float* red = reinterpret_cast<float*>(smem);
  unsigned char* meta = smem + S * p1_red_bytes(NW);
  uint16_t* xs = reinterpret_cast<uint16_t*>(meta + S * 80 * G1);
  const int item = blockIdx.y, j0 = blockIdx.x * S;   // grid (I/16/S, items): an item's slices adjacent
  // the wave index, the expert and its column count are uniform: readfirstlane
  // keeps them (and the weight addresses made from them) in SGPRs, so a weight
  // load is a scalar base plus the lane's 16-byte offset
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int q = lane >> 4, r = lane & 15;
  const unsigned lane16 = 16u * (unsigned)lane;
  if (x_all)   // uniform; x is [T][H] contiguous
    stage_lds(reinterpret_cast<unsigned char*>(xs), c.T * HI, wave, NW, lane,
              [&](int k) { return (const void*)(c.x + 8 * (size_t)k); });
  const BallotCols cl = ballot_cols(c, item, lane);
  if (!cl.serve) {   // uniform
    __builtin_amdgcn_s_waitcnt(0);   // no copy into LDS outlives the workgroup
    return;
  }
  // pair index of column col; every lane of the wave calls it
  auto pair_of = [&](int col) { return __shfl(cl.colpair, col & 63); };
  // token of a pair (pairs are token-major)
  const float rk = 1.0f / (float)c.K;
  auto tok_of = [&](int pair) { return div_small(pair, rk); };
  const int e = __builtin_amdgcn_readfirstlane(cl.e), cnt = __builtin_amdgcn_readfirstlane(cl.cnt);
  const size_t blk = (size_t)e * NI1 + j0;   // S consecutive slices: contiguous weights and metadata
  const unsigned char* msrc = w13_m + blk * 80 * G1;
  stage_lds(meta, S * 5 * G1, wave, NW, lane, [&](int k) { return (const void*)(msrc + 16 * k); });
  const int g0 = G1 * wave / NW, ng = G1 * (wave + 1) / NW - g0;   // equal for all waves (G1 % NW == 0)
  const char* wg = w13 + (blk * 2 * G1 + g0) * 1024;   // slice s: + 2*G1 KB; lane: + lane16
  constexpr float off = W4Consts<ACT>::offset;
  for (int cb0 = 0; cb0 < cnt; cb0 += P) {
    const int ncol = min(P, cnt - cb0);
    int xr;   // LDS row of this lane's column
    if (x_all) {
      xr = tok_of(pair_of(cb0 + min(r, ncol - 1)));
    } else {
      // the pass's hidden rows: row cc at xs + cc * H, in 1 KB chunks of 64
      // lanes x 16 B (H % 512 == 0: whole chunks), chunk ch by wave ch % NW
      for (int cc = 0; cc < ncol; ++cc) {   // uniform
        const char* src = reinterpret_cast<const char*>(c.x + (size_t)tok_of(pair_of(cb0 + cc)) * H) + 16 * lane;
        unsigned char* dst = reinterpret_cast<unsigned char*>(xs + (size_t)cc * H);
        for (int ch = wave; ch < (HI >> 6); ch += NW) __builtin_amdgcn_global_load_lds(src + 1024 * ch, dst + 1024 * ch, 16, 0, 0);
      }
      xr = min(r, ncol - 1);
    }
    const uint16_t* xrow = xs + xr * H + 32 * q;
    f32x4_t accg[S], accu[S];
#pragma unroll
    for (int s = 0; s < S; ++s) accg[s] = accu[s] = f32x4_t{0, 0, 0, 0};
    issue_order_fence();
    for (int gb = 0; gb < ng; gb += NB) {
      u32x4_t wgv[S][NB], wuv[S][NB];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int gi = 0; gi < NB; ++gi) {
          const char* p = wg + ((size_t)s * 2 * G1 + gb + gi) * 1024;
          wgv[s][gi] = ldg16(p + lane16);
          wuv[s][gi] = ldg16(p + (size_t)G1 * 1024 + lane16);
        }
      if (gb == 0) wait_copies_and_sync<2 * NB * S>();   // metadata and x rows are in LDS
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) {
        const int g = g0 + gb + gi;
        u32x4_t A[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) A[i] = lds16(xrow + 128 * g + 8 * i);
        f32x4_t X = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) X = mfma16<ACT>(A[i], ones4<ACT>(), X);
#pragma unroll
        for (int s = 0; s < S; ++s) {
          f32x4_t Gg = {0, 0, 0, 0}, Gu = {0, 0, 0, 0};
          const uint32_t wgw[4] = {wgv[s][gi].x, wgv[s][gi].y, wgv[s][gi].z, wgv[s][gi].w};
          const uint32_t wuw[4] = {wuv[s][gi].x, wuv[s][gi].y, wuv[s][gi].z, wuv[s][gi].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            Gg = mfma16<ACT>(A[i], deq4<ACT>(wgw[i]), Gg);
            Gu = mfma16<ACT>(A[i], deq4<ACT>(wuw[i]), Gu);
          }
          const unsigned char* ms = meta + s * 80 * G1;
          const uint32_t sc = reinterpret_cast<const uint32_t*>(ms)[r * G1 + g];
          const uint32_t zz = ms[64 * G1 + r * G1 + g];
          fold(accg[s], Gg, X, scale_of<SDT>(sc & 0xffffu), off + (float)(zz & 0xfu));
          fold(accu[s], Gu, X, scale_of<SDT>(sc >> 16), off + (float)(zz >> 4));
        }
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float* rs = red + s * (p1_red_bytes(NW) / 4);
      *reinterpret_cast<f32x4_t*>(rs + ((wave * 2 + 0) * 64 + lane) * 4) = accg[s];
      *reinterpret_cast<f32x4_t*>(rs + ((wave * 2 + 1) * 64 + lane) * 4) = accu[s];
    }
    __syncthreads();
    if (tid < 64 * S) {   // thread (slice s, lane ln)
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
        if (4 * (ln >> 4) + v < ncol)   // the pass's columns (the others repeat its last one)
          a.act[(size_t)p * c.I + 16 * (j0 + s) + (ln & 15)] = from_f32<ACT>(silu_mul_fast(gv[v], uv[v]));
      }
    }
    __syncthreads();   // red and xs are reused by the next pass
  }
}

// Down projection of RT consecutive row tiles (16 rows each) over all I for 16
// token columns: acc[rt] += sum over groups of s * (G - (offset + z) X).  A
// rows come from LDS (arow: this lane's column, k offset 8q), weights from wb
// (tile rt at wb + rt*G2 KB, G2 words of 16 B per lane, NB groups x RT tiles
// in flight together), metadata sections from secs (tile rt at secs +
// rt*SEC).  The column sums X of a group are shared by the RT tiles.  Waits
// for the LDS copies and barriers after the first batch of loads is issued.
template <int ACT, int SDT, int NB, int RT>
__device__ __forceinline__ void down_tiles(const char* wb, unsigned lane16, const uint16_t* arow,
                                           const unsigned char* secs, int SEC, int G2, int r,
                                           f32x4_t (&acc)[RT]) {
  constexpr float off = W4Consts<ACT>::offset;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x4_t{0, 0, 0, 0};
  issue_order_fence();
  for (int gb = 0; gb < G2; gb += NB) {
    u32x4_t wv[RT][NB];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int gi = 0; gi < NB; ++gi) wv[rt][gi] = ldg16(wb + ((size_t)rt * G2 + gb + gi) * 1024 + lane16);
    if (gb == 0) wait_copies_and_sync<NB * RT>();   // the LDS operands are in place
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
        const unsigned char* sec = secs + rt * SEC;
        fold(acc[rt], G, X, scale_of<SDT>(reinterpret_cast<const uint16_t*>(sec)[16 * g2 + r]),
             off + w2_zero(sec, G2, g2, r));
      }
    }
  }
}

// ================================================================ down (decode)
// Workgroup (token t, RT consecutive 16-row tiles of H), one wave per routed
// expert k < K of the token (K <= kDownMaxK): wave k computes out_k = W2[e_k]
// act[t*K+k] for the tiles; then y[t, tiles] = cast(sum_k w[t,k] * out_k)
// over the valid ids in k order -- Stage C1 + C2 of
// Int8-gemm/q8_gemm.cpp:593-641.  The token's act rows are contiguous and are
// copied into LDS while the ids are read; a token without a valid id gets
// y = 0 (Int8-gemm/q8_gemm.cpp:329-332).  No workspace traffic besides act,
// no cross-workgroup communication.
// LDS: act rows [K][I] | metadata [K][RT][SEC] | outputs [K][16 RT] f32 | valid [K].
template <int ACT, int SDT, int NB, int RT>
__global__ __launch_bounds__(kDownMaxK * 64) __attribute__((amdgpu_waves_per_eu(kDownWavesPerEU)))
void w4a16_down_token_kernel(const int32_t* ids, const uint16_t* act, const char* w2, const unsigned char* w2_m, int K,
                             int E, int H, int I, const float* tw, uint16_t* y, W4Args a) {
  // the leading arguments repeat fields of a (the first 14 dwords are preloaded
  // into SGPRs; see phase 1)
  extern __shared__ __align__(16) unsigned char smem[];
  const int MQ = H >> 6, G2 = I >> 7, II = I >> 3;
  const int SEC = w2_meta_sec_bytes(G2);
  const int t = blockIdx.y, tile0 = blockIdx.x * RT, m = tile0 >> 2, jj0 = tile0 & 3;   // grid (H/16/RT, T)
  // the wave index and the wave's expert id are uniform (SGPRs; see phase 1)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int q = lane >> 4, r = lane & 15;
  const unsigned lane16 = 16u * (unsigned)lane;
  uint16_t* as = reinterpret_cast<uint16_t*>(smem);
  unsigned char* meta = smem + (size_t)K * I * 2;
  float* outs = reinterpret_cast<float*>(meta + (size_t)K * RT * SEC);
  int* valid = reinterpret_cast<int*>(outs + 16 * RT * K);
  const int i = t * K + wave;   // this wave's pair
  const int e = __builtin_amdgcn_readfirstlane(ids[i]);
  stage_lds(reinterpret_cast<unsigned char*>(as), K * II, wave, K, lane,
            [&](int k) { return (const void*)(act + (size_t)t * K * I + 8 * (size_t)k); });
  // a wave with an invalid id computes on expert 0 and its output is ignored,
  // so every wave runs the same code (one barrier each)
  const bool ok = (unsigned)e < (unsigned)E;
  const size_t sec0 = ((size_t)(ok ? e : 0) * MQ + m) * 4 + jj0;   // RT tiles within one quad: contiguous
  unsigned char* mdst = meta + wave * RT * SEC;
  for (int l = lane; l < RT * SEC / 16; l += 64)
    __builtin_amdgcn_global_load_lds(w2_m + sec0 * SEC + 16 * l, mdst + (l - lane) * 16, 16, 0, 0);
  if (lane == 0) valid[wave] = ok;
  const char* wb = w2 + sec0 * G2 * 1024;
  f32x4_t acc[RT];
  down_tiles<ACT, SDT, NB, RT>(wb, lane16, as + wave * I + 8 * q, mdst, SEC, G2, r, acc);
  if (lane < 16)   // column 0: lanes (r, q = 0)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) outs[16 * (RT * wave + rt) + lane] = acc[rt].x;
  __syncthreads();
  if (tid < 16 * RT) {
    float yv = 0.0f;
    for (int k = 0; k < K; ++k)
      if (valid[k]) {
        const float prod = tw[t * K + k] * outs[16 * RT * k + tid];
        yv = yv + prod;
      }
    y[(size_t)t * H + 16 * tile0 + tid] = from_f32<ACT>(yv);
  }
}

// ================================================================ grouped GEMMs (sorted path)
// Work item: a row tile (up to kGemmRows = 64 routed rows of one expert, from
// the routing kernel's tile list) x a block of output rows (gate_up: 8 gate/up
// slices; down: 4 quads of 64 rows), each wave owning 16-row weight tiles of
// the block over all of K, so no cross-wave reduction.
// Per 128-k group the workgroup stages the tile's activation rows (bf16, row
// stride kGemmRowStride) and their sums into LDS, double-buffered with one
// barrier per group; each wave holds its 16 weight rows of the group (16 B per
// lane) in registers, and the next group's loads are issued before the
// current group is computed.  The workgroup's scales and zeros for all of K
// (contiguous in the metadata layout) are copied into LDS once at the start,
// so a step issues no per-lane metadata loads.  The MFMA A operand
// is 16 rows of the tile (sub-tiles of 16 rows; only the sub-tiles holding
// rows are computed), B the dequantized weights:
//   acc += s * (sum_k x (magic + q) - (offset + z) * sum_k x)   per group,
// the same arithmetic as the decode kernels, with the row sums from v_dot2
// instead of a ones-MFMA.  Only the waves of sub-tiles that hold rows store
// staged rows.  Every weight byte is read and dequantized once per
// row tile, so an expert with many rows streams its weights a few times and
// the MFMAs work on full 16-row operands.
// LDS (kGemmLds, w4_gemm13_lds_bytes, w4_gemm2_lds_bytes): staged rows
// [2][kGemmABytes] | row sums [2][kGemmRows] f32 | pair of each row
// [kGemmRows] | the workgroup's metadata (gemm13: 4 * kGemm13Blocks slice
// blocks of 80*G1 B; gemm2: 4 * kGemm2Quads sections of w2_meta_sec_bytes(G2) B)

// Copy nbytes (a multiple of 16) from global to LDS with the workgroup's
// threads; the caller's barrier makes them visible.
__device__ __forceinline__ void gemm_copy_meta(unsigned char* dst, const unsigned char* src, int nbytes, int tid) {
  for (int k = tid; k < (nbytes >> 4); k += kBlock)
    *reinterpret_cast<u32x4_t*>(dst + 16 * k) = ldg16(src + 16 * k);
}

// The staging thread's 32 values of its row (4 x 16 B) and their sum over the
// row's 128 values (v_dot2 with (1, 1), then the row's 4 threads, which are
// adjacent lanes).
template <int ACT>
__device__ __forceinline__ float gemm_row_sum(const u32x4_t (&v)[4]) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (ACT == 1)
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[k]),
                                              __builtin_bit_cast(bf16x2_t, 0x3f803f80u), acc, false);
      else
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w[k]),
                                     __builtin_bit_cast(f16x2_t, 0x3c003c00u), acc, false);
    }
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  return acc;
}

__device__ __forceinline__ void gemm_stage_store(unsigned char* buf, float* sums, int srow, int spart,
                                                 const u32x4_t (&v)[4], float sum) {
  unsigned char* d = buf + srow * kGemmRowStride + spart * 64;
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(d + 16 * i) = v[i];
  if (spart == 0) sums[srow] = sum;
}

// acc[p][s] += scale[p] * (W_p x - cz[p] * sum x) for the sub-tiles holding
// rows, for NP weight sets (gate and up, or one down tile) of the group: the
// A operand of a sub-tile is read from LDS once for all of them.  MFMA i takes
// from lane 16q + r the values at k = 32q + 8i + (0..7) of the group (QMAJOR:
// the w13 word order) or at k = 32i + 8q + (0..7) (the w2 word order).
template <int ACT, int NP, bool QMAJOR>
__device__ __forceinline__ void gemm_group(const unsigned char* buf, const float* sums, int nsub, int q,
                                           int r, const u32x4_t (&B)[NP][4], const float (&scale)[NP],
                                           const float (&cz)[NP], f32x4_t (&acc)[NP][4]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s < nsub) {   // uniform
      u32x4_t A[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        A[i] = lds16(buf + (16 * s + r) * kGemmRowStride + (QMAJOR ? 64 * q + 16 * i : 64 * i + 16 * q));
      const f32x4_t X = *reinterpret_cast<const f32x4_t*>(sums + 16 * s + 4 * q);
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        f32x4_t G = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) G = mfma16<ACT>(A[i], B[p][i], G);
        fold(acc[p][s], G, X, scale[p], cz[p]);
      }
    }
  }
}

// gate_up + SiLU*mul: work item (row tile, kGemm13Blocks consecutive blocks of
// 4 slices, a slice = 16 gate and 16 up rows); wave w owns slice w of each
// block, so a staged activation row serves 2 * kGemm13Blocks weight tiles per
// wave.  act[pair] gets the slices' 16 values each.
template <int ACT, int SDT>
__global__ __launch_bounds__(kBlock) void w4a16_gemm13_kernel(const int32_t* ntiles, const int32_t* tiles,
                                                             const int32_t* tok, const uint16_t* x, const void* w13,
                                                             const unsigned char* w13_m, int H_, int I_, W4Args a0) {
  // the leading arguments repeat fields of a0 (the first 14 dwords are
  // preloaded into SGPRs, so the tile lookup does not wait for an argument fetch)
  W4Args a = a0;
  a.c.rg.ntiles = const_cast<int32_t*>(ntiles);
  a.c.rg.tiles = const_cast<int32_t*>(tiles);
  a.c.rg.tok = const_cast<int32_t*>(tok);
  a.c.x = x;
  a.w13 = w13;
  a.w13_m = w13_m;
  a.c.H = H_;
  a.c.I = I_;
  constexpr int NB = kGemm13Blocks;
  const SchedArgs& c = a.c;
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = c.H, NI1 = c.I >> 4, G1 = H >> 7, NSB = NI1 / (4 * NB);
  const int ti = blockIdx.x / NSB, sb = blockIdx.x - ti * NSB;
  if (ti >= *c.rg.ntiles) return;   // uniform
  const int4 tl = reinterpret_cast<const int4*>(c.rg.tiles)[ti];
  const int e = tl.x, row0 = tl.y, rows = tl.z, nsub = (rows + 15) >> 4;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int srow = tid >> 2, spart = tid & 3;
  const int spair = c.rg.tok[row0 + min(srow, rows - 1)];
  const uint16_t* xsrc = c.x + (size_t)(spair / c.K) * H + 32 * spart;
  float* sums0 = reinterpret_cast<float*>(smem + 2 * kGemmABytes);
  int* pairs = reinterpret_cast<int*>(sums0 + 2 * kGemmRows);   // the tile's pair indices
  unsigned char* meta = smem + kGemmLds;                         // [4 * NB slices][80 * G1]
  gemm_copy_meta(meta, a.w13_m + ((size_t)e * NI1 + 4 * NB * sb) * 80 * G1, 4 * NB * 80 * G1, tid);
  const char* wg[NB];
  const uint32_t* msc[NB];
  const unsigned char* mz[NB];
#pragma unroll
  for (int p = 0; p < NB; ++p) {
    const int jl = 4 * p + wave;   // slice within the workgroup's blocks
    wg[p] = (const char*)a.w13 + ((size_t)e * NI1 + 4 * NB * sb + jl) * 2 * G1 * 1024 + lane * 16;
    const unsigned char* mb = meta + jl * 80 * G1;
    msc[p] = reinterpret_cast<const uint32_t*>(mb) + r * G1;
    mz[p] = mb + 64 * G1 + r * G1;
  }
  constexpr float off = W4Consts<ACT>::offset;

  // only the waves of the sub-tiles holding rows store staged activations
  // (uniform per wave); every wave loads, so the loads stay unconditional
  const bool stager = wave < nsub;
  u32x4_t sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sv[i] = ldg16(xsrc + 8 * i);
  u32x4_t wc[2 * NB];
#pragma unroll
  for (int p = 0; p < NB; ++p) {
    wc[2 * p] = ldg16(wg[p]);
    wc[2 * p + 1] = ldg16(wg[p] + (size_t)G1 * 1024);
  }
  if (spart == 0) pairs[srow] = spair;
  if (stager) gemm_stage_store(smem, sums0, srow, spart, sv, gemm_row_sum<ACT>(sv));
  __syncthreads();
  f32x4_t acc[2 * NB][4];
#pragma unroll
  for (int p = 0; p < 2 * NB; ++p)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[p][s] = f32x4_t{0, 0, 0, 0};
  for (int g = 0; g < G1; ++g) {
    const int b = g & 1;
    const bool more = g + 1 < G1;   // uniform
    const int gn = more ? g + 1 : g;
    // next group: issued before this one is computed
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = ldg16(xsrc + 128 * gn + 8 * i);
    u32x4_t wn[2 * NB];
#pragma unroll
    for (int p = 0; p < NB; ++p) {
      wn[2 * p] = ldg16(wg[p] + (size_t)gn * 1024);
      wn[2 * p + 1] = ldg16(wg[p] + (size_t)(G1 + gn) * 1024);
    }
    {
      u32x4_t B[2 * NB][4];
      float sc[2 * NB], cz[2 * NB];
#pragma unroll
      for (int p = 0; p < 2 * NB; ++p) {
        const uint32_t w4[4] = {wc[p].x, wc[p].y, wc[p].z, wc[p].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) B[p][i] = deq4<ACT>(w4[i]);
      }
#pragma unroll
      for (int p = 0; p < NB; ++p) {
        const uint32_t scc = msc[p][g], zzc = mz[p][g];
        sc[2 * p] = scale_of<SDT>(scc & 0xffffu);
        sc[2 * p + 1] = scale_of<SDT>(scc >> 16);
        cz[2 * p] = off + (float)(zzc & 0xfu);
        cz[2 * p + 1] = off + (float)((zzc >> 4) & 0xfu);
      }
      gemm_group<ACT, 2 * NB, true>(smem + b * kGemmABytes, sums0 + b * kGemmRows, nsub, q, r, B, sc, cz, acc);
    }
    if (more && stager)
      gemm_stage_store(smem + (b ^ 1) * kGemmABytes, sums0 + (b ^ 1) * kGemmRows, srow, spart, sv,
                       gemm_row_sum<ACT>(sv));
#pragma unroll
    for (int p = 0; p < 2 * NB; ++p) wc[p] = wn[p];
    __syncthreads();
  }
#pragma unroll
  for (int p = 0; p < NB; ++p)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < nsub) {
        const float gv[4] = {acc[2 * p][s].x, acc[2 * p][s].y, acc[2 * p][s].z, acc[2 * p][s].w};
        const float uv[4] = {acc[2 * p + 1][s].x, acc[2 * p + 1][s].y, acc[2 * p + 1][s].z, acc[2 * p + 1][s].w};
        const int j = 4 * NB * sb + 4 * p + wave;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * s + 4 * q + v;
          if (row < rows)
            a.act[(size_t)pairs[row] * c.I + 16 * j + r] = from_f32<ACT>(silu_mul_fast(gv[v], uv[v]));
        }
      }
    }
}

// down: work item (row tile, kGemm2Quads consecutive quads m.. of H, a quad =
// 64 rows); wave w owns the 16-row tile 64m + 16w of each quad, so a staged
// activation row serves kGemm2Quads weight tiles (the rows are re-staged by
// every workgroup of the tile: 2 quads halve that traffic).  eout[pair] gets
// the tiles' values rounded to the activation dtype (the precision of the
// act rows they come from; half the fp32 bytes written here and read by the
// combine kernel, which sums over k in fp32).
template <int ACT, int SDT>
__global__ __launch_bounds__(kBlock) void w4a16_gemm2_kernel(const int32_t* ntiles, const int32_t* tiles,
                                                            const int32_t* tok, const uint16_t* act, const void* w2,
                                                            const unsigned char* w2_m, int H_, int I_, W4Args a0) {
  // the leading arguments repeat fields of a0 (preloaded; see the gate_up GEMM)
  W4Args a = a0;
  a.c.rg.ntiles = const_cast<int32_t*>(ntiles);
  a.c.rg.tiles = const_cast<int32_t*>(tiles);
  a.c.rg.tok = const_cast<int32_t*>(tok);
  a.act = const_cast<uint16_t*>(act);
  a.w2 = w2;
  a.w2_m = w2_m;
  a.c.H = H_;
  a.c.I = I_;
  const SchedArgs& c = a.c;
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = c.H, I = c.I, G2 = I >> 7, MQ = H >> 6, NMB = MQ / kGemm2Quads;
  const int SEC = w2_meta_sec_bytes(G2);
  const int ti = blockIdx.x / NMB, m0 = (blockIdx.x - ti * NMB) * kGemm2Quads;
  if (ti >= *c.rg.ntiles) return;   // uniform
  const int4 tl = reinterpret_cast<const int4*>(c.rg.tiles)[ti];
  const int e = tl.x, row0 = tl.y, rows = tl.z, nsub = (rows + 15) >> 4;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int srow = tid >> 2, spart = tid & 3;
  const int spair = c.rg.tok[row0 + min(srow, rows - 1)];
  const uint16_t* asrc = a.act + (size_t)spair * I + 32 * spart;
  const char* wb[kGemm2Quads];
  const unsigned char* sec[kGemm2Quads];
  float* sums0 = reinterpret_cast<float*>(smem + 2 * kGemmABytes);
  int* pairs = reinterpret_cast<int*>(sums0 + 2 * kGemmRows);
  unsigned char* meta = smem + kGemmLds;   // [kGemm2Quads quads][4 tiles][SEC], contiguous in HBM
  gemm_copy_meta(meta, a.w2_m + ((size_t)e * MQ + m0) * 4 * SEC, kGemm2Quads * 4 * SEC, tid);
#pragma unroll
  for (int p = 0; p < kGemm2Quads; ++p) {
    const size_t tile = ((size_t)e * MQ + m0 + p) * 4 + wave;
    wb[p] = (const char*)a.w2 + tile * G2 * 1024 + lane * 16;
    sec[p] = meta + (p * 4 + wave) * SEC;
  }
  constexpr float off = W4Consts<ACT>::offset;

  const bool stager = wave < nsub;
  u32x4_t sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sv[i] = ldg16(asrc + 8 * i);
  u32x4_t wc[kGemm2Quads];
#pragma unroll
  for (int p = 0; p < kGemm2Quads; ++p) wc[p] = ldg16(wb[p]);
  if (spart == 0) pairs[srow] = spair;
  if (stager) gemm_stage_store(smem, sums0, srow, spart, sv, gemm_row_sum<ACT>(sv));
  __syncthreads();
  f32x4_t acc[kGemm2Quads][4];
#pragma unroll
  for (int p = 0; p < kGemm2Quads; ++p)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[p][s] = f32x4_t{0, 0, 0, 0};
  for (int g2 = 0; g2 < G2; ++g2) {
    const int b = g2 & 1;
    const bool more = g2 + 1 < G2;   // uniform
    const int gn = more ? g2 + 1 : g2;
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = ldg16(asrc + 128 * gn + 8 * i);
    u32x4_t wn[kGemm2Quads];
#pragma unroll
    for (int p = 0; p < kGemm2Quads; ++p) wn[p] = ldg16(wb[p] + (size_t)gn * 1024);
    {
      u32x4_t B[kGemm2Quads][4];
      float scp[kGemm2Quads], czp[kGemm2Quads];
#pragma unroll
      for (int p = 0; p < kGemm2Quads; ++p) {
        const uint32_t w4[4] = {wc[p].x, wc[p].y, wc[p].z, wc[p].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) B[p][i] = deq4<ACT>(w4[i]);
        scp[p] = scale_of<SDT>(reinterpret_cast<const uint16_t*>(sec[p])[16 * g2 + r]);
        czp[p] = off + w2_zero(sec[p], G2, g2, r);
      }
      gemm_group<ACT, kGemm2Quads, false>(smem + b * kGemmABytes, sums0 + b * kGemmRows, nsub, q, r, B, scp,
                                           czp, acc);
    }
    if (more && stager)
      gemm_stage_store(smem + (b ^ 1) * kGemmABytes, sums0 + (b ^ 1) * kGemmRows, srow, spart, sv,
                       gemm_row_sum<ACT>(sv));
#pragma unroll
    for (int p = 0; p < kGemm2Quads; ++p) wc[p] = wn[p];
    __syncthreads();
  }
  uint16_t* eout = reinterpret_cast<uint16_t*>(c.eout);
#pragma unroll
  for (int p = 0; p < kGemm2Quads; ++p)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < nsub) {
        const float vv[4] = {acc[p][s].x, acc[p][s].y, acc[p][s].z, acc[p][s].w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * s + 4 * q + v;
          if (row < rows) eout[(size_t)pairs[row] * H + 64 * (m0 + p) + 16 * wave + r] = from_f32<ACT>(vv[v]);
        }
      }
    }
}

template <int ACT, int SDT>
static hipError_t launch_gemm_t(const W4Args& a, int tiles_max, hipStream_t st, hipEvent_t mid) {
  const int g13 = tiles_max * (a.c.I / 64 / kGemm13Blocks), g2 = tiles_max * (a.c.H / 64 / kGemm2Quads);
  const size_t lds13 = w4_gemm13_lds_bytes(a.c.H), lds2 = w4_gemm2_lds_bytes(a.c.I);
  if (lds13 > kMaxLds)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(w4a16_gemm13_kernel<ACT, SDT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds13);
  if (lds2 > kMaxLds)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(w4a16_gemm2_kernel<ACT, SDT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds2);
  hipLaunchKernelGGL((w4a16_gemm13_kernel<ACT, SDT>), dim3(g13), dim3(kBlock), lds13, st, a.c.rg.ntiles, a.c.rg.tiles,
                     a.c.rg.tok, a.c.x, a.w13, a.w13_m, a.c.H, a.c.I, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (mid && (err = hipEventRecord(mid, st)) != hipSuccess) return err;
  hipLaunchKernelGGL((w4a16_gemm2_kernel<ACT, SDT>), dim3(g2), dim3(kBlock), lds2, st, a.c.rg.ntiles, a.c.rg.tiles,
                     a.c.rg.tok, (const uint16_t*)a.act, a.w2, a.w2_m, a.c.H, a.c.I, a);
  return hipGetLastError();
}

hipError_t launch_w4a16_gemm(const W4Args& a, int act, int tiles_max, hipStream_t st, hipEvent_t mid) {
  if (!w4_sorted_fits(a.c.H, a.c.I, device_max_lds())) return hipErrorInvalidValue;
  if (act == 1) return a.sdt == 1 ? launch_gemm_t<1, 1>(a, tiles_max, st, mid) : launch_gemm_t<1, 0>(a, tiles_max, st, mid);
  return a.sdt == 1 ? launch_gemm_t<0, 1>(a, tiles_max, st, mid) : launch_gemm_t<0, 0>(a, tiles_max, st, mid);
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

// w2: one thread per device u32 word: (e, quad m, row tile jj, group g2,
// lane, chunk cc of the group).
__global__ void awq_repack_w2(const int32_t* __restrict__ src, uint32_t* __restrict__ dst, int E,
                              int H, int I) {
  const int G2 = I >> 7, MQ = H >> 6;
  const size_t total = (size_t)E * MQ * 4 * G2 * 256;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int cc = idx & 3, lane = (idx >> 2) & 63;
    size_t t = idx >> 8;
    const int g2 = t % G2; t /= G2;
    const int jj = t % 4; t /= 4;
    const int m = t % MQ;
    const int e = (int)(t / MQ);
    const int h = 64 * m + 16 * jj + (lane & 15);
    const int k0 = 128 * g2 + 32 * cc + 8 * (lane >> 4);
    const int32_t* base = src + (size_t)e * I * (H / 8);
    uint32_t word = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) word |= awq_nib(base, H, k0 + 2 * p + hh, h) << (4 * p + 16 * hh);
    dst[idx] = word;
  }
}

// w2 metadata: one section of w2_meta_sec_bytes(G2) bytes per (e, m, jj):
// scales u16 [g2][r], then zeros [g2][r/2] (row r in nibble r&1); one thread
// per (e, m, jj, g2, row pair).
__global__ void awq_repack_w2_meta(const uint16_t* __restrict__ scales, const int32_t* __restrict__ qzeros,
                                   unsigned char* __restrict__ m_dst, int E, int H, int I) {
  const int G2 = I >> 7, MQ = H >> 6, SEC = w2_meta_sec_bytes(G2);
  const size_t total = (size_t)E * MQ * 4 * G2 * 8;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int r2 = idx & 7;
    size_t t = idx >> 3;
    const int g2 = t % G2; t /= G2;
    const int jj = t % 4; t /= 4;
    const int m = t % MQ;
    const int e = (int)(t / MQ);
    unsigned char* sec = m_dst + (((size_t)e * MQ + m) * 4 + jj) * SEC;
    const int32_t* zb = qzeros + (size_t)e * G2 * (H / 8);
    uint32_t zz = 0;
    for (int hh = 0; hh < 2; ++hh) {
      const int r = 2 * r2 + hh, h = 64 * m + 16 * jj + r;
      reinterpret_cast<uint16_t*>(sec)[16 * g2 + r] = scales[((size_t)e * G2 + g2) * H + h];
      zz |= awq_nib(zb, H, g2, h) << (4 * hh);
    }
    sec[32 * G2 + 8 * g2 + r2] = (unsigned char)zz;
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
  hipLaunchKernelGGL(awq_repack_w2_meta, dim3(grid_for((size_t)E * MQ * 4 * G2 * 8)), dim3(256), 0, st,
                     w2s, w2z, d2m, E, H, I);
  return hipGetLastError();
}

// ================================================================ launchers
template <int ACT, int SDT, int NB, int S, int NW>
static void launch_p1(const W4Args& a, int grid, size_t lds, hipStream_t st) {
  if (lds > kMaxLds)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(w4a16_phase1_kernel<ACT, SDT, NB, S, NW>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  const int njs = (a.c.I >> 4) / S;
  hipLaunchKernelGGL((w4a16_phase1_kernel<ACT, SDT, NB, S, NW>), dim3(njs, grid / njs), dim3(NW * kWave), lds, st,
                     a.c.ids, a.c.x, (const char*)a.w13, a.w13_m, a.c.T, a.c.n, a.c.E, a.c.H, a.c.I, a.x_all, a.c.K, a);
}

// (NB, S, NW) instantiated for phase 1.  S > 1 measured slower on the
// decode shapes (occupancy), so only S = 1 is built; NW = 8 waves (K split 8
// ways) for the smallest calls.
template <int ACT, int SDT>
static hipError_t dispatch_p1(const W4Args& a, int nb, int s, int nw, int grid, size_t lds, hipStream_t st) {
#define P1_CASE(NB_, S_, NW_) \
  if (nb == NB_ && s == S_ && nw == NW_) { launch_p1<ACT, SDT, NB_, S_, NW_>(a, grid, lds, st); return hipGetLastError(); }
  P1_CASE(1, 1, 4) P1_CASE(2, 1, 4) P1_CASE(3, 1, 4) P1_CASE(4, 1, 4) P1_CASE(6, 1, 4) P1_CASE(8, 1, 4)
  P1_CASE(1, 1, 8) P1_CASE(2, 1, 8) P1_CASE(3, 1, 8) P1_CASE(4, 1, 8)
#undef P1_CASE
  return hipErrorInvalidValue;
}

// (NB, RT) pairs instantiated for the down kernel.  RT > 1 (2-4 tiles per
// wave) measured no faster on the decode shapes, so only RT = 1 is built.
template <int ACT, int SDT>
static hipError_t dispatch_p2(const W4Args& a, int nb, int rt, int grid, size_t lds, hipStream_t st) {
#define P2_CASE(NB_, RT_)                                                                           \
  if (nb == NB_ && rt == RT_) {                                                                     \
    if (lds > kMaxLds)                                                                              \
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(w4a16_down_token_kernel<ACT, SDT, NB_, RT_>), \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);              \
    hipLaunchKernelGGL((w4a16_down_token_kernel<ACT, SDT, NB_, RT_>), dim3((a.c.H >> 4) / RT_, grid / ((a.c.H >> 4) / RT_)), \
                       dim3(64 * a.c.K), lds, st, a.c.ids, (const uint16_t*)a.act, (const char*)a.w2, a.w2_m, \
                       a.c.K, a.c.E, a.c.H, a.c.I, a.c.tw, a.c.y, a);                                \
    return hipGetLastError();                                                                       \
  }
  P2_CASE(1, 1) P2_CASE(2, 1) P2_CASE(3, 1) P2_CASE(4, 1) P2_CASE(6, 1) P2_CASE(8, 1)
#undef P2_CASE
  return hipErrorInvalidValue;
}

// largest size in `sizes` that divides `need`
static int pick_div(const int* sizes, int count, int need) {
  int b = 1;
  for (int i = 0; i < count; ++i)
    if (need % sizes[i] == 0) b = sizes[i];
  return b;
}

// Launch geometry of the decode path: batch sizes divide the per-wave group
// counts (S slices per phase-1 workgroup and RT row tiles per down wave are 1:
// larger values measured no faster on the decode shapes).  The token-major
// down kernel spills at NB = 12 within its 6-waves-per-SIMD register budget,
// so NB <= 8 there.
W4Plan w4a16_plan(int H, int I) {
  static const int nb1[] = {1, 2, 3, 4, 6, 8}, nb2[] = {1, 2, 3, 4, 6, 8};
  W4Plan p;
  p.nb1 = pick_div(nb1, 6, H / 512);
  p.s1 = 1;
  p.nb2 = pick_div(nb2, 6, I / 128);
  p.rt2 = 1;
  return p;
}

template <int ACT, int SDT>
static hipError_t launch_w4_t(const W4Args& a, const W4Plan& p, int grid1, int grid2, hipStream_t st,
                              hipEvent_t mid) {
  // the smallest calls: gate_up's K split over 8 waves (shorter chains per wave)
  const int G1 = a.c.H / 128;
  const int nw1 = w4_p1_waves(a.c.n, a.c.H);
  // the batch divides the wave's groups; 1-4 are built for every wave count
  int nb1 = nw1 == 4 ? p.nb1 : min(p.nb1, 4);
  while ((G1 / nw1) % nb1) --nb1;
  const size_t lds1 = w4_p1_lds_bytes(a.c.H, a.x_all ? a.c.T : a.p1_cols, p.s1, nw1);
  const size_t lds2 = w4_down_token_lds_bytes(a.c.I, a.c.K, p.rt2);
  if (lds1 > device_max_lds() || lds2 > device_max_lds()) return hipErrorInvalidValue;
  hipError_t err = dispatch_p1<ACT, SDT>(a, nb1, p.s1, nw1, grid1 / p.s1, lds1, st);
  if (err != hipSuccess) return err;
  if (mid && (err = hipEventRecord(mid, st)) != hipSuccess) return err;
  return dispatch_p2<ACT, SDT>(a, p.nb2, p.rt2, grid2 / p.rt2, lds2, st);
}

// Decode path (T*K <= 64, K <= kDownMaxK): grid1 = T*K * I/16 (phase 1),
// grid2 = T * H/16 (down kernel, writes y); the plan divides them by its
// slice / tile counts.  mid (optional) is recorded between the two launches.
hipError_t launch_w4a16(const W4Args& a, const W4Plan& p, int act, int grid1, int grid2, hipStream_t st,
                        hipEvent_t mid) {
  if (act == 1) return a.sdt == 1 ? launch_w4_t<1, 1>(a, p, grid1, grid2, st, mid) : launch_w4_t<1, 0>(a, p, grid1, grid2, st, mid);
  return a.sdt == 1 ? launch_w4_t<0, 1>(a, p, grid1, grid2, st, mid) : launch_w4_t<0, 0>(a, p, grid1, grid2, st, mid);
}

}  // namespace mimoe
