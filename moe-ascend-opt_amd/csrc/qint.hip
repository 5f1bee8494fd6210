// qint.hip -- Q8_0 / Q4_0 weights with Q8_0-quantized activations: the
// reference CPU algorithm (moe_forward_ptr_impl, Int8-gemm/q8_gemm.cpp:
// 276-646) on gfx950.
//
// Arithmetic per output (m, n), as the reference micro-kernels
// (Int8-gemm/gemm_kernels.cpp:102-179, 254-358):
//     isum_kb = sum_{i<32} a_q * w_q            (exact int32, v_dot4_i32_i8)
//     c      += ((float)isum_kb * dw[n,kb]) * da[m,kb]
// with w_q = int8 (Q8_0) or nibble-8 (Q4_0: dot with the unsigned nibble,
// then subtract 8 * sum(a_q) of the block).  Each lane owns one weight row;
// the four waves of a workgroup split the k blocks and their fp32 partial
// sums are added in wave order.
//
// Device weight layout: tiles of 64 weight rows ("lanes") x all K blocks.
//   gate_up: [E][I/32 slices] tiles; lane r<32 is gate row 32s+r, lane r>=32
//            is up row I+32s+r-32, so SiLU*mul pairs lanes r and r+32 and one
//            slice yields one Q8_0 block of the intermediate.
//   down:    [E][H/64] tiles; lane r = row 64hb+r.
//   A row's block splits into four quarters q of 8 elements: Q8_0 8 bytes,
//   Q4_0 one word holding elements 8q+m (low nibble of byte m) and 8q+4+m
//   (high nibble), so (w & 0x0F0F0F0F) and (w >> 4 & 0x0F0F0F0F) line up with
//   activation dwords 2q and 2q+1.  Inside a tile, blocks go in groups of 4
//   along K (the last group may hold fewer, G) and a group is stored
//   [lane][quarter][block in group][quarter bytes] (QLay): a lane-per-row
//   reader takes the row's whole group, the grouped GEMM one 16-byte (Q4_0)
//   or 32-byte (Q8_0) run per lane and group.
//   scales: [tile][block][64 lanes] (fp16 or bf16 bits).
#pragma clang fp contract(off)
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"
#include "mi_moe_sched.hpp"
#include "handover.hpp"

namespace mimoe {

template <int QT>
struct QFmt {
  static constexpr int chunks = QT == 0 ? 2 : 1;
  static constexpr int block_bytes = chunks * 64 * 16;  // one (tile, block)
};

// Byte offset inside a tile of (block kb, lane, quarter q); WB bytes per quarter.
template <int QT>
struct QLay {
  static constexpr int WB = QT == 0 ? 8 : 4;
  __host__ __device__ static size_t off(int KB, int kb, int lane, int q) {
    const int g0 = kb & ~3, G = KB - g0 < 4 ? KB - g0 : 4, b = kb - g0;
    return (size_t)g0 * QFmt<QT>::block_bytes + (size_t)lane * (4 * WB * G) + q * (WB * G) + b * WB;
  }
};

// One block of one lane as the legacy 16-byte chunks: w0 = quarters 0-3 (Q4_0)
// or 0-1 (Q8_0), w1 = Q8_0 quarters 2-3.
template <int QT>
__device__ __forceinline__ void load_block(const char* wtile, int KB, int kb, int lane, u32x4_t& w0,
                                           u32x4_t& w1) {
  if constexpr (QT == 1) {
    uint32_t v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const uint32_t*>(wtile + QLay<1>::off(KB, kb, lane, q));
    w0 = u32x4_t{v[0], v[1], v[2], v[3]};
    w1 = u32x4_t{0, 0, 0, 0};
  } else {
    u32x2_t v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const u32x2_t*>(wtile + QLay<0>::off(KB, kb, lane, q));
    w0 = u32x4_t{v[0].x, v[0].y, v[1].x, v[1].y};
    w1 = u32x4_t{v[2].x, v[2].y, v[3].x, v[3].y};
  }
}

template <int QT>
__device__ __forceinline__ void unpack_w(const u32x4_t w0, const u32x4_t w1, int (&wd)[8]) {
  if constexpr (QT == 0) {
    wd[0] = (int)w0.x; wd[1] = (int)w0.y; wd[2] = (int)w0.z; wd[3] = (int)w0.w;
    wd[4] = (int)w1.x; wd[5] = (int)w1.y; wd[6] = (int)w1.z; wd[7] = (int)w1.w;
  } else {
    const uint32_t w[4] = {w0.x, w0.y, w0.z, w0.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      wd[2 * d] = (int)(w[d] & 0x0f0f0f0fu);
      wd[2 * d + 1] = (int)((w[d] >> 4) & 0x0f0f0f0fu);
    }
  }
}

// Exact int32 dot of one 32-element block (Int8-gemm/gemm_kernels.cpp:
// 109-133 for Q8_0, 262-309 for Q4_0).
template <int QT>
__device__ __forceinline__ int block_isum(const int (&wd)[8], const int* xv, int xsum) {
  int s = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) s = __builtin_amdgcn_sdot4(wd[j], xv[j], s, false);
  if constexpr (QT == 1) s -= 8 * xsum;
  return s;
}

// Integer decode path (lane-per-row kernels): the NW waves of a workgroup
// split K, and a wave's first batch of weight groups is issued before the
// activations are staged.  NW = 8 for the smallest calls (kQDecWideMaxPairs
// routed pairs or fewer: few workgroups, each wave's chain is shorter; a
// top-10 token is 10 pairs), 4 above (occupancy; 8 waves at 16 pairs measured
// slower).
constexpr int kQDecWideMaxPairs = 12;
// The one-launch decode kernel serves every call of the decode path (up to
// 64 routed pairs: one wave's ballot routes them), with the gate_up K split
// over two workgroups up to kQFusedMaxPairs.  Same-box graph replays, config
// 1 shape (Q8_0, H=2048, I=768, top-8): T = 1 / 2 / 4 / 8 17.05-17.07 /
// 26.89-26.95 / 40.20-40.28 / 67.34-67.80 us, against 19.90-20.07 /
// 28.22-28.86 / 40.31-40.54 / 67.76-68.33 us in two launches.
constexpr int kQFusedPairsLimit = kWave;

// One lane's row weights (whole 4-block layout groups, as 16-byte loads) and
// the blocks' raw scale bits for up to NG_ groups (Q8_0: 32 VGPRs of weights
// per group, Q4_0: 16).  kQBatchGroups: the phase kernels' batch, 64 VGPRs of
// weights in the 8-wave form (the smallest calls: a wave's whole share of K
// for H = 2048), 32 in the 4-wave form (occupancy).
template <int QT, int NG_>
struct QRowBatch {
  static constexpr int NV = 4 * QFmt<QT>::chunks;   // 16-byte loads per group
  static constexpr int NG = NG_;                    // groups per batch
  u32x4_t v[NG][NV];
  uint32_t sw[NG][4];
};
template <int QT, int NW>
constexpr int kQBatchGroups = (QT == 0 ? 1 : 2) * (NW == 8 ? 2 : 1);

// Issue the loads of the whole groups gs, gs+4, .. (up to NG) that start below
// kb1 and lie inside the row (g + 4 <= KB); a partial last group is left to
// rows_dot's per-block tail.
template <int QT, int NG>
__device__ __forceinline__ void rows_issue(QRowBatch<QT, NG>& B, const char* wtile, const uint16_t* stile,
                                           int lane, int gs, int kb1, int KB) {
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int g0 = gs + 4 * j;
    if (g0 < kb1 && g0 + 4 <= KB) {   // uniform
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(wtile + QLay<QT>::off(KB, g0, lane, 0));
#pragma unroll
      for (int i = 0; i < QRowBatch<QT, NG>::NV; ++i) B.v[j][i] = p[i];
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) B.sw[j][bb] = stile[(g0 + bb) * 64 + lane];
    }
  }
}

// Dot of this lane's weight row against the staged activations for k blocks
// [kb0, kb1), accumulating into acc[c] for the cntp staged tokens, block by
// block in ascending order.  B holds the first batch (rows_issue at
// kb0 & ~3) when `issued`; later batches are loaded here.  Blocks of a group
// outside the range are skipped (the neighbouring wave reads the same group,
// mostly from the cache).
template <int QT, int SC, int NG>
__device__ __forceinline__ void rows_dot(QRowBatch<QT, NG>& B, bool issued, const char* wtile, const uint16_t* stile,
                                         int lane, int kb0, int kb1, const int8_t* xq, const float* xd,
                                         const int* xs, int K, int KB, int cntp, float (&acc)[kQTokPerPass]) {
  auto block = [&](int kb, const u32x4_t& w0, const u32x4_t& w1, float dw) {
    int wd[8];
    unpack_w<QT>(w0, w1, wd);
#pragma unroll
    for (int cc = 0; cc < kQTokPerPass; ++cc) {
      if (cc >= cntp) break;
      const int* xv = reinterpret_cast<const int*>(xq + cc * K + kb * 32);
      const int s = block_isum<QT>(wd, xv, QT == 1 ? xs[cc * KB + kb] : 0);
      const float t1 = (float)s * dw;
      const float t2 = t1 * xd[cc * KB + kb];
      acc[cc] = acc[cc] + t2;
    }
  };
  const int gs0 = kb0 & ~3, KBw = KB & ~3;   // KBw: end of the whole groups
  for (int gs = gs0; gs < kb1 && gs < KBw; gs += 4 * NG) {
    if (gs != gs0 || !issued) rows_issue<QT, NG>(B, wtile, stile, lane, gs, kb1, KB);
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int g0 = gs + 4 * j;
      if (g0 >= kb1 || g0 >= KBw) break;   // uniform
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        if (g0 + bb < kb0 || g0 + bb >= kb1) continue;   // uniform
        const float dw = to_f32<SC>(B.sw[j][bb]);
        if constexpr (QT == 1) {
          block(g0 + bb, u32x4_t{B.v[j][0][bb], B.v[j][1][bb], B.v[j][2][bb], B.v[j][3][bb]},
                u32x4_t{0, 0, 0, 0}, dw);
        } else {
          // quarter q of block bb: dwords 2bb, 2bb+1 of the 32-byte run v[2q], v[2q+1]
          const int h = 2 * (bb & 1), i = bb >> 1;
          block(g0 + bb, u32x4_t{B.v[j][i][h], B.v[j][i][h + 1], B.v[j][2 + i][h], B.v[j][2 + i][h + 1]},
                u32x4_t{B.v[j][4 + i][h], B.v[j][4 + i][h + 1], B.v[j][6 + i][h], B.v[j][6 + i][h + 1]}, dw);
        }
      }
    }
  }
  // a partial last group (KB % 4 != 0): per-block loads
  for (int kb = max(kb0, KBw); kb < kb1; ++kb) {
    u32x4_t w0, w1;
    load_block<QT>(wtile, KB, kb, lane, w0, w1);
    block(kb, w0, w1, to_f32<SC>(stile[kb * 64 + lane]));
  }
}

struct QLds {
  int8_t* xq;   // [kQTokPerPass][Kmax]
  float* xd;    // [kQTokPerPass][KBmax]
  int* xs;      // [kQTokPerPass][KBmax]
  float* red;   // [kQDecWavesMax][kQTokPerPass][64]
  int* route;
};

__device__ __forceinline__ QLds carve(unsigned char* smem, int Kmax) {
  QLds L;
  const int KBmax = Kmax / 32;
  L.xq = reinterpret_cast<int8_t*>(smem);
  L.xd = reinterpret_cast<float*>(smem + kQTokPerPass * Kmax);
  L.xs = reinterpret_cast<int*>(L.xd + kQTokPerPass * KBmax);
  L.red = reinterpret_cast<float*>(L.xs + kQTokPerPass * KBmax);
  L.route = reinterpret_cast<int*>(L.red + kQDecWavesMax * kQTokPerPass * 64);
  return L;
}

// ---------------------------------------------------------------- phase 1
// TAG: the one-launch kernel's form: the intermediate blocks go to tagged
// units (q_tag_units per pair row) instead of act_q / act_d.  KS = 2: the
// workgroups come in pairs kh = 0, 1 per (item, slice), each over half of K
// (the waves of the pair split K in 16 parts); kh = 0 hands its gate and up
// sums to kh = 1 as tagged units, and kh = 1 adds them to its own
// (half 0 + half 1) before the activation.
template <int QT, int ACT, int SC, int NW, bool TAG = false, int KS = 1>
__device__ __forceinline__ void q_phase1(const QArgs& a, int e, int cnt, const int* pairs, int sl, const QLds& L,
                                         int kh = 0) {
  const SchedArgs& c = a.c;
  // wave index uniform (SGPR): the K range and the batch branches below are scalar
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int KB = c.H / 32, S = c.I / 32;
  const int kb0 = KB * (kh * NW + wave) / (KS * NW), kb1 = KB * (kh * NW + wave + 1) / (KS * NW);
  const int kbs = KB * kh / KS, kbe = KB * (kh + 1) / KS;   // this workgroup's blocks
  const size_t tile = (size_t)e * S + sl;
  constexpr int kNG = TAG ? (kQBatchGroups<QT, NW> + 1) / 2 : kQBatchGroups<QT, NW>;
  const char* wtile = (const char*)a.w13 + tile * KB * QFmt<QT>::block_bytes;
  const uint16_t* stile = a.w13_d + tile * KB * 64;
  // the first weight batch is in flight while the activations are staged
  QRowBatch<QT, kNG> B;
  rows_issue<QT, kNG>(B, wtile, stile, lane, kb0 & ~3, kb1, KB);

  for (int cb0 = 0; cb0 < cnt; cb0 += kQTokPerPass) {
    const int cntp = min(kQTokPerPass, cnt - cb0);
    // Stage A for the staged tokens (Int8-gemm/q8_gemm.cpp:360-377): 8 lanes
    // per 32-value block, 4 values each, the block's amax and byte sum over
    // the 8 lanes by shuffles (a max and an integer sum: the same d and bytes
    // as quant_block_q8_0); every lane runs the same trip count
    const float rk = 1.0f / (float)c.K;
    const int p8 = lane & 7, KBw = kbe - kbs, nblk = cntp * KBw;
    const float rkbw = 1.0f / (float)KBw;
    for (int b0 = 0; b0 < nblk; b0 += NW * kWave / 8) {
      const int idx = b0 + (tid >> 3);
      const bool okb = idx < nblk;
      const int ix = okb ? idx : 0;
      const int cc = div_small(ix, rkbw), kb = kbs + ix - cc * KBw;
      const int pr = pairs[cb0 + cc];
      const int t = c.n < (1 << 21) ? div_small(pr, rk) : pr / c.K;   // uniform choice
      const u32x2_t w = *reinterpret_cast<const u32x2_t*>(c.x + (size_t)t * c.H + kb * 32 + 4 * p8);
      const float v[4] = {to_f32<ACT>(w.x & 0xffffu), to_f32<ACT>(w.x >> 16), to_f32<ACT>(w.y & 0xffffu),
                          to_f32<ACT>(w.y >> 16)};
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float av = __builtin_fabsf(v[j]);
        amax = av > amax ? av : amax;
      }
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) {
        const float o = __shfl_xor(amax, m, 8);
        amax = o > amax ? o : amax;
      }
      float id;
      const float d = q8_block_scale(amax, &id);
      int qsum = 0;
      uint32_t word = 0;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int8_t q = q8_round(v[h] * id);
        qsum += q;
        word |= ((uint32_t)(uint8_t)q) << (8 * h);
      }
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) qsum += __shfl_xor(qsum, m, 8);
      if (okb) {
        *reinterpret_cast<uint32_t*>(L.xq + cc * c.H + kb * 32 + 4 * p8) = word;
        if (p8 == 0) {
          L.xd[cc * KB + kb] = d;
          L.xs[cc * KB + kb] = qsum;
        }
      }
    }
    __syncthreads();
    float acc[kQTokPerPass];
#pragma unroll
    for (int cc = 0; cc < kQTokPerPass; ++cc) acc[cc] = 0.0f;
    rows_dot<QT, SC, kNG>(B, cb0 == 0, wtile, stile, lane, kb0, kb1, L.xq, L.xd, L.xs, c.H, KB,
                                        cntp, acc);
#pragma unroll
    for (int cc = 0; cc < kQTokPerPass; ++cc)
      if (cc < cntp) L.red[(wave * kQTokPerPass + cc) * 64 + lane] = acc[cc];
    __syncthreads();
    if (tid < kQTokPerPass * 32) {
      // thread t -> token cc = t/32, intermediate column r = t%32 of the slice
      const int cc = tid >> 5, r = tid & 31;
      const int ccl = cc < cntp ? cc : 0;
      float g = L.red[(0 * kQTokPerPass + ccl) * 64 + r];
      float u = L.red[(0 * kQTokPerPass + ccl) * 64 + r + 32];
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        g = g + L.red[(w * kQTokPerPass + ccl) * 64 + r];
        u = u + L.red[(w * kQTokPerPass + ccl) * 64 + r + 32];
      }
      if constexpr (KS == 2) {
        // the K halves: gate and up sums of (column cc, row r) as two units
        unsigned long long* pu = a.tact + q_part_unit0(c.I) + ((size_t)pairs[cb0 + ccl] * S + sl) * 64;
        const unsigned tag = dispatch_tag32();
        if (kh == 0) {
          if (cc < cntp) {
            store_agent(pu + r, ((unsigned long long)tag << 32) | __float_as_uint(g));
            store_agent(pu + 32 + r, ((unsigned long long)tag << 32) | __float_as_uint(u));
          }
        } else {
          unsigned long long vg = 0, vu = 0;
          for (int polls = 0;; ++polls) {
            vg = load_agent(pu + r);
            vu = load_agent(pu + 32 + r);
            if (__all((unsigned)(vg >> 32) == tag && (unsigned)(vu >> 32) == tag)) break;
            if (polls > kSpinMax) {   // gave up: the pair's output becomes NaN
              vg = vu = 0x7fc00000ull;
              if (tid == 0) store_agent(a.tact + (size_t)64 * (c.I >> 1), 1ull);
              break;
            }
            __builtin_amdgcn_s_sleep(1);
          }
          g = __uint_as_float((unsigned)vg) + g;
          u = __uint_as_float((unsigned)vu) + u;
        }
      }
      const float act = silu_mul(g, u);
      // Q8_0 re-quantization of the 32-value intermediate block
      // (pack_A_q8_0, Int8-gemm/gemm_kernels.cpp:394-425)
      float amax = __builtin_fabsf(act);
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) {
        const float o = __shfl_xor(amax, m, 32);
        amax = o > amax ? o : amax;
      }
      float id;
      const float d = q8_block_scale(amax, &id);
      const int8_t q = q8_round(act * id);
      if constexpr (TAG) {
        // lane r % 4 == 0 packs bytes r..r+3 of the block into one unit; the
        // 8 units of a (pair, slice) are one 64-byte line, its scale one unit
        const uint32_t b = (uint32_t)(uint8_t)q;
        const uint32_t w = b | ((uint32_t)__shfl_down((int)b, 1, 32) << 8) |
                           ((uint32_t)__shfl_down((int)b, 2, 32) << 16) | ((uint32_t)__shfl_down((int)b, 3, 32) << 24);
        if (kh == KS - 1 && cc < cntp) {
          unsigned long long* row = a.tact + (size_t)pairs[cb0 + cc] * q_tag_units(c.I);
          const unsigned long long tg = (unsigned long long)dispatch_tag32() << 32;
          if ((r & 3) == 0) store_agent(row + 8 * sl + (r >> 2), tg | w);
          if (r == 0) store_agent(row + (c.I >> 2) + sl, tg | __float_as_uint(d));
        }
      } else if (cc < cntp) {
        const size_t row = (size_t)pairs[cb0 + cc];
        a.act_q[row * c.I + 32 * sl + r] = q;
        if (r == 0) a.act_d[row * S + sl] = d;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- phase 2
template <int QT, int ACT, int SC, int NW>
__device__ void q_phase2(const QArgs& a, const RouteView& rv, int ui, int hb, const QLds& L) {
  const SchedArgs& c = a.c;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int e = __builtin_amdgcn_readfirstlane(rv.active[ui]);
  const int p0 = __builtin_amdgcn_readfirstlane(rv.starts[e]), cnt = __builtin_amdgcn_readfirstlane(rv.starts[e + 1]) - p0;
  const int KB2 = c.I / 32, HB = c.H / 64;
  const int kb0 = KB2 * wave / NW, kb1 = KB2 * (wave + 1) / NW;
  const size_t tile = (size_t)e * HB + hb;
  const char* wtile = (const char*)a.w2 + tile * KB2 * QFmt<QT>::block_bytes;
  const uint16_t* stile = a.w2_d + tile * KB2 * 64;
  QRowBatch<QT, kQBatchGroups<QT, NW>> B;   // in flight while the intermediate rows are staged
  rows_issue<QT, kQBatchGroups<QT, NW>>(B, wtile, stile, lane, kb0 & ~3, kb1, KB2);

  for (int cb0 = 0; cb0 < cnt; cb0 += kQTokPerPass) {
    const int cntp = min(kQTokPerPass, cnt - cb0);
    const float rkb = 1.0f / (float)KB2;
    for (int idx = tid; idx < cntp * KB2; idx += NW * kWave) {
      const int cc = div_small(idx, rkb), kb = idx - cc * KB2;
      const size_t row = (size_t)rv.pair[p0 + cb0 + cc];
      const u32x4_t* src = reinterpret_cast<const u32x4_t*>(a.act_q + row * c.I + kb * 32);
      const u32x4_t q0 = src[0], q1 = src[1];
      u32x4_t* dst = reinterpret_cast<u32x4_t*>(L.xq + cc * c.I + kb * 32);
      dst[0] = q0;
      dst[1] = q1;
      if constexpr (QT == 1) {
        const uint32_t ws[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        int s = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) s = __builtin_amdgcn_sdot4((int)ws[j], 0x01010101, s, false);
        L.xs[cc * KB2 + kb] = s;
      }
      L.xd[cc * KB2 + kb] = a.act_d[row * KB2 + kb];
    }
    __syncthreads();
    float acc[kQTokPerPass];
#pragma unroll
    for (int cc = 0; cc < kQTokPerPass; ++cc) acc[cc] = 0.0f;
    rows_dot<QT, SC, kQBatchGroups<QT, NW>>(B, cb0 == 0, wtile, stile, lane, kb0, kb1, L.xq, L.xd, L.xs, c.I, KB2,
                                        cntp, acc);
#pragma unroll
    for (int cc = 0; cc < kQTokPerPass; ++cc)
      if (cc < cntp) L.red[(wave * kQTokPerPass + cc) * 64 + lane] = acc[cc];
    __syncthreads();
    for (int cc = wave; cc < cntp; cc += NW) {
      float v = L.red[(0 * kQTokPerPass + cc) * 64 + lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) v = v + L.red[(w * kQTokPerPass + cc) * 64 + lane];
      c.eout[(size_t)rv.pair[p0 + cb0 + cc] * c.H + 64 * hb + lane] = v;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- kernels

// Work items: up to kQBallotMaxPairs routed pairs, one per pair (the item
// serves its expert iff it is the expert's first pair; ballot routing, the
// expert's pair list staged in LDS); above, one per active expert of the
// counting sort (in LDS, or the routing kernel's arrays).
// The leading arguments repeat fields of a0: gfx950 preloads the first 14
// dwords of them into SGPRs at wave launch (-amdgpu-kernarg-preload-count), so
// the ids read, the weight addresses and the x staging do not wait for a
// kernel-argument fetch.
template <int QT, int ACT, int SC, int NW>
__global__ __launch_bounds__(NW * kWave) void q_phase1_kernel(const int32_t* ids, const void* w13, const uint16_t* w13_d,
                                                             const uint16_t* x, int n, int E, int H, int I, int K,
                                                             QArgs a0) {
  QArgs a = a0;
  a.c.ids = ids;
  a.w13 = w13;
  a.w13_d = w13_d;
  a.c.x = x;
  a.c.n = n;
  a.c.E = E;
  a.c.H = H;
  a.c.I = I;
  a.c.K = K;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_U;
  const QLds L = carve(smem, a.c.H);
  const int item = blockIdx.y, sl = blockIdx.x;   // grid (I/32 slices, items)
  if (a.c.n <= kWave) {   // uniform: one ballot over all ids, no sort
    const int tid = threadIdx.x;
    const BallotCols cl = ballot_cols(a.c, item, tid & 63);   // every wave: same result
    if (!cl.serve) return;   // uniform
    if (tid < kWave) L.route[tid] = cl.colpair;
    __syncthreads();
    q_phase1<QT, ACT, SC, NW>(a, __builtin_amdgcn_readfirstlane(cl.e), __builtin_amdgcn_readfirstlane(cl.cnt),
                              L.route, sl, L);
    return;
  }
  if (a.c.n <= kQBallotMaxPairs) {   // uniform: ballots over 2-3 batches of 64 ids
    const int tid = threadIdx.x;
    int e, cnt;
    const bool serve = a.c.n <= 128 ? ballot_route_n<2>(a.c, item, tid, L.route, e, cnt)
                                    : ballot_route_n<3>(a.c, item, tid, L.route, e, cnt);
    if (!serve) return;   // uniform
    __syncthreads();
    q_phase1<QT, ACT, SC, NW>(a, __builtin_amdgcn_readfirstlane(e), __builtin_amdgcn_readfirstlane(cnt), L.route,
                              sl, L);
    return;
  }
  const RouteView rv = sched_route(a.c, L.route, &s_U);
  if (item >= rv.U) return;
  const int e = __builtin_amdgcn_readfirstlane(rv.active[item]), p0 = __builtin_amdgcn_readfirstlane(rv.starts[e]);
  q_phase1<QT, ACT, SC, NW>(a, e, __builtin_amdgcn_readfirstlane(rv.starts[e + 1]) - p0, rv.pair + p0, sl, L);
}

template <int QT, int ACT, int SC, int NW>
__global__ __launch_bounds__(NW * kWave) void q_phase2_kernel(QArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_U;
  const QLds L = carve(smem, a.c.I);
  const RouteView rv = sched_route(a.c, L.route, &s_U);
  const int ui = blockIdx.y;   // grid (H/64 blocks, items)
  if (ui >= rv.U) return;
  q_phase2<QT, ACT, SC, NW>(a, rv, ui, blockIdx.x, L);
}

// Down projection at decode sizes, token-major with the combine fused:
// workgroup (token t, 16-row tile of H), one wave per routed expert k < K
// (K <= kDownMaxK).  Lane (q, r) of wave k computes row r of the tile over
// quarter q of I (the row's exact block dots, block order within the
// quarter), the quarters are summed in order, and y[t, tile] = cast(sum_k
// w[t,k] * out_k) over the valid ids in k order -- Stage C1 + C2 of
// Int8-gemm/q8_gemm.cpp:593-641 without an eout round trip.  A wave with an
// invalid id computes on expert 0 and is left out of the sum; a token with
// no valid id gets y = 0.
// LDS: act bytes [K][I] | act d [K][I/32] | act byte sums [K][I/32] | quarter
// partials [K][64] | outputs [K][16] | valid [K].

template <int QT, int ACT, int SC>
__global__ __launch_bounds__(kDownMaxK * 64) void q_down_token_kernel(const int32_t* ids, const void* w2,
                                                                      const uint16_t* w2_d, const int8_t* act_q,
                                                                      const float* act_d, int K, int E, int H, int I,
                                                                      QArgs a0) {
  // the leading arguments repeat fields of a0 (preloaded into SGPRs; see
  // q_phase1_kernel)
  QArgs a = a0;
  a.c.ids = ids;
  a.w2 = w2;
  a.w2_d = w2_d;
  a.act_q = const_cast<int8_t*>(act_q);
  a.act_d = const_cast<float*>(act_d);
  a.c.K = K;
  a.c.E = E;
  a.c.H = H;
  a.c.I = I;
  const SchedArgs& c = a.c;
  extern __shared__ __align__(16) unsigned char smem[];
  const int KB2 = I / 32, HB = H / 64;
  const int t = blockIdx.y, jt = blockIdx.x;   // grid (H/16 tiles, T)
  // the wave index and the wave's expert id are uniform (SGPRs)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int q = lane >> 4, r = lane & 15;
  int8_t* xq = reinterpret_cast<int8_t*>(smem);
  float* xd = reinterpret_cast<float*>(smem + (size_t)K * I);
  int* xs = reinterpret_cast<int*>(xd + K * KB2);
  float* part = reinterpret_cast<float*>(xs + K * KB2);
  float* outs = part + K * 64;
  int* valid = reinterpret_cast<int*>(outs + K * 16);
  const int e = __builtin_amdgcn_readfirstlane(c.ids[t * K + wave]);
  const bool ok = (unsigned)e < (unsigned)c.E;
  // this lane's row in the 64-row layout tile, and its quarter of the blocks
  const int row = (jt & 3) * 16 + r;
  const size_t tile = (size_t)(ok ? e : 0) * HB + (jt >> 2);
  const char* wtile = (const char*)a.w2 + tile * KB2 * QFmt<QT>::block_bytes;
  const uint16_t* stile = a.w2_d + tile * KB2 * 64;
  const int kb0 = KB2 * q / 4, kb1 = KB2 * (q + 1) / 4;
  QRowBatch<QT, 2> B;   // both groups a quarter can touch, in flight while the rows are staged
  rows_issue<QT, 2>(B, wtile, stile, row, kb0 & ~3, kb1, KB2);
  const float rkb = 1.0f / (float)KB2;
  for (int idx = tid; idx < K * KB2; idx += K * 64) {
    const int cc = div_small(idx, rkb), kb = idx - cc * KB2;
    const size_t prow = (size_t)t * K + cc;   // pair rows of a token are contiguous
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(a.act_q + prow * I + kb * 32);
    const u32x4_t q0 = src[0], q1 = src[1];
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(xq + cc * I + kb * 32);
    dst[0] = q0;
    dst[1] = q1;
    if constexpr (QT == 1) {
      const uint32_t ws[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      int sum = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) sum = __builtin_amdgcn_sdot4((int)ws[j], 0x01010101, sum, false);
      xs[cc * KB2 + kb] = sum;
    }
    xd[cc * KB2 + kb] = a.act_d[prow * KB2 + kb];
  }
  if (lane == 0) valid[wave] = ok;
  __syncthreads();
  float acc[kQTokPerPass];
#pragma unroll
  for (int cc = 0; cc < kQTokPerPass; ++cc) acc[cc] = 0.0f;
  rows_dot<QT, SC, 2>(B, true, wtile, stile, row, kb0, kb1, xq + wave * I, xd + wave * KB2, xs + wave * KB2, I,
                      KB2, 1, acc);
  part[wave * 64 + lane] = acc[0];
  __syncthreads();
  if (lane < 16) {
    const float* pw = part + wave * 64;
    outs[wave * 16 + lane] = ((pw[lane] + pw[16 + lane]) + pw[32 + lane]) + pw[48 + lane];
  }
  __syncthreads();
  if (tid < 16) {
    float y = 0.0f;
    for (int k = 0; k < K; ++k)
      if (valid[k]) {
        const float prod = c.tw[t * K + k] * outs[16 * k + tid];
        y = y + prod;
      }
    c.y[(size_t)t * H + 16 * jt + tid] = from_f32<ACT>(y);
  }
}

// ---------------------------------------------------------------- one launch
// The Q8_0 / Q4_0 decode layer in one launch for the smallest calls (up to
// kQDecWideMaxPairs routed pairs, top-k <= 8), 8-wave workgroups:
//  * [0, n1): gate_up items (pair i, 32-row slice sl), the phase-1 routine
//    above (ballot routing over all ids; the item serves its expert iff i is
//    the expert's first pair), its intermediate Q8_0 blocks written as tagged
//    units (handover.hpp);
//  * [n1, n1 + T * H/16): down items (token t, 16-row tile jt), the
//    token-major down routine with the combine (Int8-gemm/q8_gemm.cpp:
//    593-641); wave k < K reads the intermediate row of pair t*K+k from the
//    units.
// A down wave issues its weight loads first, then reads the whole row with
// coherent loads, checks every tag and unpacks it into LDS, reading it again
// until every unit is there (config 1 T = 2 / 4 / 8: 0.4-0.7 us faster than a
// first pass over the per-slice scale units, same box).  The waits
// end: workgroups start in index order, so the gate_up items a down item reads
// from are resident or finished when it starts, and they wait on nothing.
// The wait is still bounded (kSpinMax polls); a wave that gives up makes its
// token's tile NaN and sets the buffer's timeout unit.
template <int QT, int ACT, int SC>
__device__ __forceinline__ void q_fused_down(const QArgs& a, int t, int jt, unsigned char* smem) {
  const SchedArgs& c = a.c;
  const int K = c.K, I = c.I, H = c.H, KB2 = I / 32, HB = H / 64;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int q = lane >> 4, r = lane & 15;
  int8_t* xq = reinterpret_cast<int8_t*>(smem);
  float* xd = reinterpret_cast<float*>(smem + (size_t)kQFusedWaves * I);
  int* xs = reinterpret_cast<int*>(xd + kQFusedWaves * KB2);
  float* part = reinterpret_cast<float*>(xs + kQFusedWaves * KB2);
  float* outs = part + kQFusedWaves * 64;
  int* state = reinterpret_cast<int*>(outs + kQFusedWaves * 16);   // 0 invalid id, 1 valid, 2 wait gave up
  float* tws = reinterpret_cast<float*>(state + kQFusedWaves);
  // the combine's routing weights, copied into LDS now (covered by the
  // barrier's wait below; no registers held)
  if (tid < K) __builtin_amdgcn_global_load_lds(c.tw + t * K + tid, tws, 4, 0, 0);
  if (wave < K) {   // uniform: wave k takes routed expert k of token t
    const int i = t * K + wave;
    const int e = __builtin_amdgcn_readfirstlane(c.ids[i]);
    // an invalid id computes on expert 0 and its output is ignored
    const bool ok = (unsigned)e < (unsigned)c.E;
    const int row = (jt & 3) * 16 + r;   // this lane's row in the 64-row layout tile
    const size_t tile = (size_t)(ok ? e : 0) * HB + (jt >> 2);
    const char* wtile = (const char*)a.w2 + tile * KB2 * QFmt<QT>::block_bytes;
    const uint16_t* stile = a.w2_d + tile * KB2 * 64;
    const int kb0 = KB2 * q / 4, kb1 = KB2 * (q + 1) / 4;
    QRowBatch<QT, 2> B;   // both groups a quarter can touch, in flight during the wait
    rows_issue<QT, 2>(B, wtile, stile, row, kb0 & ~3, kb1, KB2);
    int st = ok ? 1 : 0;
    if (ok) {
      const unsigned tag = dispatch_tag32();
      const unsigned long long* units = a.tact + (size_t)i * q_tag_units(I);
      const int nq = I >> 2, nunits = q_tag_units(I);
      unsigned* dq = reinterpret_cast<unsigned*>(xq + (size_t)wave * I);
      float* dd = xd + wave * KB2;
      auto read_row = [&]() {
        bool whole = true;
        for (int u0 = 0; u0 < nunits; u0 += 64 * 4) {
          unsigned long long v[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int u = u0 + 64 * b + lane;
            v[b] = u < nunits ? load_agent(units + u) : ((unsigned long long)tag << 32);
          }
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int u = u0 + 64 * b + lane;
            whole = whole && (unsigned)(v[b] >> 32) == tag;
            if (u < nq) dq[u] = (unsigned)v[b];
            else if (u < nunits) dd[u - nq] = __uint_as_float((unsigned)v[b]);
          }
        }
        return __all(whole);
      };
      for (int polls = 0; !read_row();) {
        if (++polls > kSpinMax) {
          st = 2;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (st == 2 && lane == 0) store_agent(a.tact + (size_t)64 * (I >> 1), 1ull);
      if constexpr (QT == 1) {   // Q4_0: the blocks' byte sums (this wave's own LDS row: in order)
        for (int kb = lane; kb < KB2; kb += 64) {
          const int* wq = reinterpret_cast<const int*>(xq + (size_t)wave * I + 32 * kb);
          int sum = 0;
#pragma unroll
          for (int j = 0; j < 8; ++j) sum = __builtin_amdgcn_sdot4(wq[j], 0x01010101, sum, false);
          xs[wave * KB2 + kb] = sum;
        }
      }
    }
    if (lane == 0) state[wave] = st;
    float acc[kQTokPerPass];
#pragma unroll
    for (int cc = 0; cc < kQTokPerPass; ++cc) acc[cc] = 0.0f;
    rows_dot<QT, SC, 2>(B, true, wtile, stile, row, kb0, kb1, xq + (size_t)wave * I, xd + wave * KB2,
                        xs + wave * KB2, I, KB2, 1, acc);
    part[wave * 64 + lane] = acc[0];
    if (lane < 16) {   // the quarters in order (this wave's own partials)
      const float* pw = part + wave * 64;
      outs[wave * 16 + lane] = ((pw[lane] + pw[16 + lane]) + pw[32 + lane]) + pw[48 + lane];
    }
  }
  __syncthreads();
  if (tid < 16) {
    float y = 0.0f;
    bool gave_up = false;
#pragma unroll
    for (int k = 0; k < kQFusedWaves; ++k) {
      const int sk = k < K ? state[k] : 0;
      if (sk) {
        gave_up |= sk == 2;
        const float prod = tws[k] * outs[16 * k + tid];
        y = y + prod;
      }
    }
    c.y[(size_t)t * H + 16 * jt + tid] = gave_up ? (uint16_t)0x7fc0u : from_f32<ACT>(y);   // NaN in bf16 and fp16
  }
}

// The leading arguments repeat fields of a0 (preloaded into SGPRs; see
// q_phase1_kernel).
template <int QT, int ACT, int SC, int KS>
__global__ __launch_bounds__(kQFusedWaves * kWave) __attribute__((amdgpu_waves_per_eu(4)))
void q_decode_kernel(const int32_t* ids, const uint16_t* x, const void* w13, const uint16_t* w13_d, const void* w2,
                     const uint16_t* w2_d, int n1, int I, QArgs a0) {
  QArgs a = a0;
  a.c.ids = ids;
  a.c.x = x;
  a.w13 = w13;
  a.w13_d = w13_d;
  a.w2 = w2;
  a.w2_d = w2_d;
  a.c.I = I;
  extern __shared__ __align__(16) unsigned char smem[];
  const int b = blockIdx.x, S1 = I >> 5;
  if (b < n1) {   // uniform: gate_up item (pair, slice)
    const QLds L = carve(smem, a.c.H);
    const int item = b / (KS * S1), rem = b - item * KS * S1, sl = rem / KS;
    const int tid = threadIdx.x;
    const BallotCols cl = ballot_cols(a.c, item, tid & 63);   // every wave: same result
    if (!cl.serve) return;   // uniform
    if (tid < kWave) L.route[tid] = cl.colpair;
    __syncthreads();
    q_phase1<QT, ACT, SC, kQFusedWaves, true, KS>(a, __builtin_amdgcn_readfirstlane(cl.e),
                                                 __builtin_amdgcn_readfirstlane(cl.cnt), L.route, sl, L, rem - sl * KS);
  } else {
    const int nt = a.c.H >> 4, d = b - n1, t = d / nt;
    q_fused_down<QT, ACT, SC>(a, t, d - t * nt, smem);
  }
}

// Dynamic LDS beyond kMaxLds needs the kernel's opt-in.
template <class Kern>
static void lds_opt_in(Kern k, size_t lds) {
  if (lds > kMaxLds)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

template <int QT, int ACT, int SC, int NW>
static hipError_t launch_q_nw(const QArgs& a, int grid1, int grid2, size_t route, bool token_down,
                              hipStream_t st) {
  const size_t l1 = q_stage_bytes(a.c.H) + route;
  lds_opt_in(q_phase1_kernel<QT, ACT, SC, NW>, l1);
  hipLaunchKernelGGL((q_phase1_kernel<QT, ACT, SC, NW>), dim3(a.c.I / 32, grid1 / (a.c.I / 32)), dim3(NW * kWave),
                     l1, st, a.c.ids, a.w13, a.w13_d, a.c.x, a.c.n, a.c.E, a.c.H, a.c.I, a.c.K, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (token_down) {
    const size_t l2 = q_down_token_lds_bytes(a.c.I, a.c.K);
    lds_opt_in(q_down_token_kernel<QT, ACT, SC>, l2);
    hipLaunchKernelGGL((q_down_token_kernel<QT, ACT, SC>), dim3(a.c.H / 16, a.c.T), dim3(64 * a.c.K), l2, st,
                       a.c.ids, a.w2, a.w2_d, (const int8_t*)a.act_q, (const float*)a.act_d, a.c.K, a.c.E, a.c.H,
                       a.c.I, a);
    return hipGetLastError();
  }
  const size_t l2 = q_stage_bytes(a.c.I) + route;
  lds_opt_in(q_phase2_kernel<QT, ACT, SC, NW>, l2);
  hipLaunchKernelGGL((q_phase2_kernel<QT, ACT, SC, NW>), dim3(a.c.H / 64, grid2 / (a.c.H / 64)), dim3(NW * kWave),
                     l2, st, a);
  return hipGetLastError();
}

template <int QT, int ACT, int SC>
static hipError_t launch_q_t(const QArgs& a, int grid1, int grid2, bool token_down, hipStream_t st) {
  const size_t route = q_route_lds_bytes(a.c.E, a.c.n);
  if (!q_lpr_fits(a.c.H, a.c.I, a.c.E, a.c.n, a.c.K, token_down, device_max_lds())) return hipErrorInvalidValue;
  return a.c.n <= kQDecWideMaxPairs ? launch_q_nw<QT, ACT, SC, 8>(a, grid1, grid2, route, token_down, st)
                                    : launch_q_nw<QT, ACT, SC, 4>(a, grid1, grid2, route, token_down, st);
}

// token_down: the down projection and the combine in one token-major launch
// (decode sizes); otherwise expert-major down into eout (the caller combines).
hipError_t launch_qint(const QArgs& a, int qt, int act, int sc, int grid1, int grid2, bool token_down,
                       hipStream_t st) {
  const bool td = token_down;
  if (qt == 0) {
    if (act == 1) return sc == 1 ? launch_q_t<0, 1, 1>(a, grid1, grid2, td, st) : launch_q_t<0, 1, 0>(a, grid1, grid2, td, st);
    return sc == 1 ? launch_q_t<0, 0, 1>(a, grid1, grid2, td, st) : launch_q_t<0, 0, 0>(a, grid1, grid2, td, st);
  }
  if (act == 1) return sc == 1 ? launch_q_t<1, 1, 1>(a, grid1, grid2, td, st) : launch_q_t<1, 1, 0>(a, grid1, grid2, td, st);
  return sc == 1 ? launch_q_t<1, 0, 1>(a, grid1, grid2, td, st) : launch_q_t<1, 0, 0>(a, grid1, grid2, td, st);
}

template <int QT, int ACT, int SC, int KS>
static hipError_t launch_q_fused_ks(const QArgs& a, size_t lds, hipStream_t st) {
  lds_opt_in(q_decode_kernel<QT, ACT, SC, KS>, lds);
  const int n1 = a.c.n * (a.c.I / 32) * KS, n2 = a.c.T * (a.c.H / 16);
  hipLaunchKernelGGL((q_decode_kernel<QT, ACT, SC, KS>), dim3(n1 + n2), dim3(kQFusedWaves * kWave), lds, st,
                     a.c.ids, a.c.x, a.w13, a.w13_d, a.w2, a.w2_d, n1, a.c.I, a);
  return hipGetLastError();
}
// K split over two workgroups per gate_up item up to kQFusedMaxPairs routed pairs
template <int QT, int ACT, int SC>
static hipError_t launch_q_fused_t(const QArgs& a, size_t lds, hipStream_t st) {
  return a.c.n <= kQFusedMaxPairs ? launch_q_fused_ks<QT, ACT, SC, 2>(a, lds, st)
                                  : launch_q_fused_ks<QT, ACT, SC, 1>(a, lds, st);
}

// LDS of the one-launch kernel, or 0 if it does not serve the call.
size_t q_fused_lds(int n, int K, int H, int I, int E) {
  if (n > kQFusedPairsLimit || K > kQFusedWaves || I > kTagActMaxI || H % 64 != 0) return 0;
  const size_t gate_up = q_stage_bytes(H) + q_route_lds_bytes(E, n), down = q_fused_down_lds_bytes(I);
  const size_t lds = gate_up > down ? gate_up : down;
  return lds <= device_max_lds() ? lds : 0;
}

hipError_t launch_q_fused(const QArgs& a, int qt, int act, int sc, hipStream_t st) {
  const size_t lds = q_fused_lds(a.c.n, a.c.K, a.c.H, a.c.I, a.c.E);
  if (!lds || !a.tact) return hipErrorInvalidValue;
  if (qt == 0) {
    if (act == 1) return sc == 1 ? launch_q_fused_t<0, 1, 1>(a, lds, st) : launch_q_fused_t<0, 1, 0>(a, lds, st);
    return sc == 1 ? launch_q_fused_t<0, 0, 1>(a, lds, st) : launch_q_fused_t<0, 0, 0>(a, lds, st);
  }
  if (act == 1) return sc == 1 ? launch_q_fused_t<1, 1, 1>(a, lds, st) : launch_q_fused_t<1, 1, 0>(a, lds, st);
  return sc == 1 ? launch_q_fused_t<1, 0, 1>(a, lds, st) : launch_q_fused_t<1, 0, 0>(a, lds, st);
}

// ---------------------------------------------------------------- grouped GEMMs (int8 MFMA)
// Sorted path for the prefill sizes: the routing kernel's row tiles (up to
// kGemmRows = 64 routed rows of one expert) x a 64-row block of the output,
// with v_mfma_i32_16x16x32_i8 giving the exact int32 dot of one 32-element
// block for 16 rows x 16 output rows, then per element, in k-block order,
//     c += ((float)isum * dw[n, kb]) * da[m, kb]
// (Int8-gemm/gemm_kernels.cpp:156-179; Q4_0: dot with nibble - 8,
// :262-309).  The first product is bit-identical to the reference's; the
// second is fused with the add (one rounding fewer than its vmulq + vmlaq,
// inside the fp32 tolerance).  Wave w owns output rows 16w..16w+15 of the
// block for all rows of the tile (NSUB sub-tiles of 16) and all of K.
// Activations were Q8_0-quantized once per token (x) or are the intermediate
// Q8_0 rows (act); the workgroup stages kQgStage blocks of the tile's rows and
// their scales into LDS per step, double-buffered, and each wave loads its
// weights for the next step before computing the current one.
// MFMA operands: A = the wave's 16 weight rows, B = 16 tile rows (lane 16q + r:
// row r, bytes 8q..8q+7 of the block for both); D lane 16q + r = tile row r of
// the sub-tile x weight rows 4q..4q+3, so a lane needs one activation scale
// per sub-tile and four weight scales per block.
//
// Two exact rewrites keep the VALU work at two fma per output and block:
// * the accumulator starts from the bits of 1.5 * 2^23 (kQgBias), so with
//   |isum| < 2^22 the int32 result read as a float is 1.5 * 2^23 + isum, and
//   fma(that, dw, -1.5 * 2^23 * dw) = round(isum * dw): the product
//   1.5 * 2^23 * dw is exact (dw has at most 11 significant bits) and the fma
//   rounds once;
// * Q4_0 nibbles n enter the MFMA as bytes 16 * (n - 8) (n ^ 8 in the high
//   half of the byte), so the int32 result is 16 * isum exactly, the first
//   product 16 * round(isum * dw), and the activation scale is staged as
//   da / 16 (powers of two: the same products and roundings).
// The activation scales of a step are staged [row][block] (one 16-byte read
// per sub-tile and step), the weight scales of the workgroup's 64 weight rows
// [block][row]: wave 0 loads them, 8 bytes per lane, and each wave reads the
// 4-row quads it needs, 16 lanes to an address.  Tiles of 3-4 sub-tiles
// (CONV) stage them as fp32 pairs (dw, -1.5 * 2^23 * dw), converted once by
// wave 0, which saves each lane 8 VALU ops per block; smaller tiles stage the
// fp16/bf16 bits and convert per lane, keeping wave 0's staging short (a
// small tile's step is short and waits on it).
constexpr int kQgStage = 4;                          // 32-element blocks per step
constexpr int kQgRowStride = kQgStage * 32 + 16;     // bytes per staged row (pad spreads the banks)
constexpr int kQgABytes = kGemmRows * kQgRowStride;  // 9216
constexpr int kQgDaBytes = kGemmRows * kQgStage * 4;  // activation scales [row][block] f32
constexpr int kQgDwBytes = kQgStage * 64 * 8;         // weight scales [block][64 rows] (dw, nb) f32 or bits
constexpr int kQgBufBytes = kQgABytes + kQgDaBytes + kQgDwBytes;
// LDS: [2][kQgBufBytes] staging (after the K loop, the gate_up epilogue's act
// tile [64][kQgActStride] f32 reuses it) | pairs [64]
constexpr int kQgActStride = 36;   // 32 columns + pad (16-byte rows, spread banks)
static_assert(kGemmRows * kQgActStride * 4 <= 2 * kQgBufBytes, "act tile fits the staging buffers");
constexpr size_t kQgLds = 2 * (size_t)kQgBufBytes + kGemmRows * 4;
constexpr int kQgBias = 0x4B400000;      // bits of 1.5 * 2^23
constexpr float kQgBiasF = 12582912.0f;  // 1.5 * 2^23

// A weight scale as the GEMMs use it: dw (fp32) and nb = -1.5 * 2^23 * dw.
template <int SC>
__device__ __forceinline__ void qg_wscale(uint32_t bits, float& dw, float& nb) {
  dw = to_f32<SC>(bits);
  nb = -kQgBiasF * dw;
}

// The int8 MFMA of one 32-element block from the bias accumulator: lane
// 16q + r of the result holds kQgBias + (weight row 4q + i) . (tile row r)
// for i < 4 (Q4_0: kQgBias + 16 * isum).
__device__ __forceinline__ i32x4_t qg_mfma(long wb, long av) {
  i32x4_t d = {kQgBias, kQgBias, kQgBias, kQgBias};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(wb, av, d, 0, 0, 0);
}

// The first scaled product of a block, round(isum * dw) (Q4_0: 16 times it),
// from an MFMA result read as a float: fma(1.5 * 2^23 + isum, dw, nb).
__device__ __forceinline__ float qg_scaled(int dbits, float dw, float nb) {
  return __builtin_fmaf(__int_as_float(dbits), dw, nb);
}

// one thread's share of a step's staging: a 32-byte block of its row and the
// block's scale; in wave 0 also 4 weight scales (block lane / 16, rows
// 4 * (lane % 16) .. +3)
struct QgStage { u32x4_t v[2]; float d; u32x2_t dw; };

__device__ __forceinline__ QgStage qg_load(const int8_t* rowq, const float* rowd, int kb0, int sblk,
                                           const uint16_t* stile, bool w0, int lane) {
  QgStage s;
  const u32x4_t* p = reinterpret_cast<const u32x4_t*>(rowq + 32 * (kb0 + sblk));
  s.v[0] = p[0];
  s.v[1] = p[1];
  s.d = rowd[kb0 + sblk];
  if (w0) s.dw = *reinterpret_cast<const u32x2_t*>(stile + (kb0 + (lane >> 4)) * 64 + 4 * (lane & 15));
  return s;
}

template <int QT, int SC, bool CONV>
__device__ __forceinline__ void qg_store(unsigned char* buf, int srow, int sblk, const QgStage& s, bool w0,
                                         int lane) {
  *reinterpret_cast<u32x4_t*>(buf + srow * kQgRowStride + 32 * sblk) = s.v[0];
  *reinterpret_cast<u32x4_t*>(buf + srow * kQgRowStride + 32 * sblk + 16) = s.v[1];
  reinterpret_cast<float*>(buf + kQgABytes)[srow * kQgStage + sblk] = QT == 1 ? s.d * 0.0625f : s.d;
  if (w0 && !CONV) {
    *reinterpret_cast<u32x2_t*>(buf + kQgABytes + kQgDaBytes + (lane >> 4) * 128 + 8 * (lane & 15)) = s.dw;
  } else if (w0) {
    float d[4], nb[4];
    qg_wscale<SC>(s.dw.x & 0xffffu, d[0], nb[0]);
    qg_wscale<SC>(s.dw.x >> 16, d[1], nb[1]);
    qg_wscale<SC>(s.dw.y & 0xffffu, d[2], nb[2]);
    qg_wscale<SC>(s.dw.y >> 16, d[3], nb[3]);
    f32x4_t* o = reinterpret_cast<f32x4_t*>(buf + kQgABytes + kQgDaBytes + (lane >> 4) * 512 + 32 * (lane & 15));
    o[0] = f32x4_t{d[0], nb[0], d[1], nb[1]};
    o[1] = f32x4_t{d[2], nb[2], d[3], nb[3]};
  }
}

// MFMA B bytes: Q8_0 as stored; Q4_0 as 16 * (n - 8), elements 8q..8q+7
template <int QT>
__device__ __forceinline__ long qg_wbytes(uint64_t w) {
  if constexpr (QT == 0) {
    return (long)w;
  } else {
    // n ^ 8 (the 4-bit two's complement of n - 8) in the high half of each
    // byte: one 3-input bit operation for the high nibbles, a shift and one
    // for the low ones (the constants sit in registers: gfx9 VOP3 takes no
    // literal)
    uint32_t k8 = 0x88888888u, kf0 = 0xf0f0f0f0u;
    asm("" : "+v"(k8));
    asm("" : "+v"(kf0));
    const uint32_t w32 = (uint32_t)w;
    const uint32_t hi = (w32 ^ k8) & kf0;
    const uint32_t lo = ((w32 << 4) ^ k8) & kf0;
    return (long)((uint64_t)lo | ((uint64_t)hi << 32));
  }
}

// acc[s] += round(isum * dw) * da (fused) for block `sblk` of the step and the
// NSUB sub-tiles, given dw and nb = -1.5 * 2^23 * dw of weight rows 4q..4q+3;
// dq[s] = the staged activation scales of tile row 16s + r for the step's
// blocks.
template <int NSUB>
__device__ __forceinline__ void qg_block(const unsigned char* buf, int sblk, int r, int q, long wb,
                                         const float (&dws)[4], const float (&nb)[4], const f32x4_t (&dq)[4],
                                         f32x4_t (&acc)[4]) {
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    const long av = *reinterpret_cast<const long*>(buf + (16 * s + r) * kQgRowStride + 32 * sblk + 8 * q);
    const i32x4_t d = qg_mfma(wb, av);
    const float da = dq[s][sblk];
    const int dv[4] = {d.x, d.y, d.z, d.w};
    float* ac = reinterpret_cast<float*>(&acc[s]);
#pragma unroll
    for (int i = 0; i < 4; ++i) ac[i] = __builtin_fmaf(qg_scaled(dv[i], dws[i], nb[i]), da, ac[i]);
  }
}

// The wave's weights of one step (kQgStage = 4 blocks, one layout group):
// lane 16q + r takes quarter q of weight row tl = tlb + r for the 4 blocks,
// one contiguous run (Q4_0 16 bytes, Q8_0 32 bytes).
static_assert(kQgStage == 4, "a step is one 4-block layout group");
template <int QT>
struct QgWSet {
  uint64_t w[kQgStage];
  __device__ __forceinline__ void load(const char* wtile, int KB, int kb0, int tl, int q) {
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(wtile + QLay<QT>::off(KB, kb0, tl, q));
    if constexpr (QT == 1) {
      const u32x4_t v = p[0];
#pragma unroll
      for (int b = 0; b < 4; ++b) w[b] = v[b];
    } else {
      const u32x4_t v0 = p[0], v1 = p[1];
      w[0] = (uint64_t)v0.x | ((uint64_t)v0.y << 32);
      w[1] = (uint64_t)v0.z | ((uint64_t)v0.w << 32);
      w[2] = (uint64_t)v1.x | ((uint64_t)v1.y << 32);
      w[3] = (uint64_t)v1.z | ((uint64_t)v1.w << 32);
    }
  }
};

// One GEMM over K = 32*KB for the tile's NSUB*16 rows (rowq/rowd: this
// thread's staging row) against the wave's 16 weight rows (tile lanes
// tlb..tlb+15 of the weight tile wtile, scales stile), accumulating into acc.
// Loads run D steps ahead through a ring of register sets, one batch per
// step: the weights of step st + D and the activation rows of step
// st + 1 + D (staged into LDS, double-buffered, one step before use).  The
// memory counter drains in issue order, so a batch holds both kinds: waiting
// for the rows to stage never waits for weights issued after them.  The
// kernels use D = 1: on MI355X rings of 2 and 3 steps measured slower at
// every tile size (small tiles are bound by load-instruction issue, not by
// the latency a deeper ring hides).
template <int QT, int SC, int NSUB, int D>
__device__ __forceinline__ void qg_gemm(unsigned char* smem, const int8_t* rowq, const float* rowd, int KB,
                                        const char* wtile, const uint16_t* stile, int tlb, int tid,
                                        f32x4_t (&acc)[4]) {
  constexpr bool CONV = NSUB >= 3;         // weight scales staged as fp32 pairs
  const bool stager = (tid >> 6) < NSUB;   // waves holding the tile's rows
  const int lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int srow = tid >> 2, sblk = tid & 3;   // staging: row, block within the step
  const int tl = tlb + r;
  const bool w0 = (tid >> 6) == 0;             // wave 0 also stages the weight scales
  const int NS = KB / kQgStage;                // steps (KB is a multiple of kQgStage)
  // ring: weights of step j in ws[j % D], staging of step j in sv[j % D]
  QgWSet<QT> ws[D];
  QgStage sv[D];
#pragma unroll
  for (int u = 0; u < D; ++u) {
    ws[u].load(wtile, KB, min(u, NS - 1) * kQgStage, tl, q);
    sv[u] = qg_load(rowq, rowd, min(u, NS - 1) * kQgStage, sblk, stile, w0, lane);
  }
  if (stager) qg_store<QT, SC, CONV>(smem, srow, sblk, sv[0], w0, lane);
  sv[0] = qg_load(rowq, rowd, min(D, NS - 1) * kQgStage, sblk, stile, w0, lane);
  __syncthreads();
  for (int st0 = 0; st0 < NS; st0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int st = st0 + u;
      const bool live = st < NS;       // uniform
      const bool more = st + 1 < NS;   // uniform
      const unsigned char* buf = smem + (st & 1) * kQgBufBytes;
      if (live) {
        f32x4_t dq[4];
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
          dq[s] = *reinterpret_cast<const f32x4_t*>(buf + kQgABytes + (16 * s + r) * kQgStage * 4);
#pragma unroll
        for (int b = 0; b < kQgStage; ++b) {
          float dws[4], nb[4];
          if constexpr (CONV) {
            const f32x4_t* scp =
                reinterpret_cast<const f32x4_t*>(buf + kQgABytes + kQgDaBytes + b * 512 + (tlb + 4 * q) * 8);
            const f32x4_t s0 = scp[0], s1 = scp[1];
            dws[0] = s0.x; nb[0] = s0.y; dws[1] = s0.z; nb[1] = s0.w;
            dws[2] = s1.x; nb[2] = s1.y; dws[3] = s1.z; nb[3] = s1.w;
          } else {
            const u32x2_t raw =
                *reinterpret_cast<const u32x2_t*>(buf + kQgABytes + kQgDaBytes + b * 128 + (tlb + 4 * q) * 2);
            const uint32_t rw[4] = {raw.x & 0xffffu, raw.x >> 16, raw.y & 0xffffu, raw.y >> 16};
#pragma unroll
            for (int i = 0; i < 4; ++i) qg_wscale<SC>(rw[i], dws[i], nb[i]);
          }
          qg_block<NSUB>(buf, b, r, q, qg_wbytes<QT>(ws[u].w[b]), dws, nb, dq, acc);
          // keep each block's scaling next to its MFMAs: left free, the fma
          // chains sink below all of the step's MFMAs and every MFMA result and
          // scale of the step is live at once
#pragma unroll
          for (int s = 0; s < NSUB; ++s) asm volatile("" : "+v"(acc[s]));
        }
      }
      const int un = (u + 1) % D;   // ring slot of step st + 1 (constant once unrolled)
      ws[u].load(wtile, KB, min(st + D, NS - 1) * kQgStage, tl, q);
      if (more && stager) qg_store<QT, SC, CONV>(smem + ((st & 1) ^ 1) * kQgBufBytes, srow, sblk, sv[un], w0, lane);
      if (stager)   // uniform per wave
        sv[un] = qg_load(rowq, rowd, min(st + 1 + D, NS - 1) * kQgStage, sblk, stile, w0, lane);
      __syncthreads();
    }
  }
}

// gate_up + SiLU*mul + Q8_0 intermediate: work item (row tile, slice s = the
// 64-lane weight tile of gate rows 32s..32s+31 and up rows I+32s..); waves 0-1
// gate rows 0-15 / 16-31, waves 2-3 the matching up rows.  The slice's 32
// intermediate values of a row form one Q8_0 block (pack_A_q8_0,
// Int8-gemm/gemm_kernels.cpp:394-425).
template <int QT, int SC>
__global__ __launch_bounds__(kBlock) void q_gemm13_kernel(const int32_t* ntiles, const int32_t* tiles,
                                                         const int32_t* tokl, const int8_t* xq, const float* xd,
                                                         const void* w13, const uint16_t* w13_d, QArgs a0) {
  // the leading arguments repeat fields of a0 (preloaded into SGPRs; see
  // q_phase1_kernel)
  QArgs a = a0;
  a.c.rg.ntiles = const_cast<int32_t*>(ntiles);
  a.c.rg.tiles = const_cast<int32_t*>(tiles);
  a.c.rg.tok = const_cast<int32_t*>(tokl);
  a.xq = xq;
  a.xd = xd;
  a.w13 = w13;
  a.w13_d = w13_d;
  const SchedArgs& c = a.c;
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = c.H, I = c.I, S = I / 32, KB = H / 32;
  const int ti = blockIdx.x / S, sl = blockIdx.x - ti * S;
  if (ti >= *c.rg.ntiles) return;   // uniform
  const int4 tlv = reinterpret_cast<const int4*>(c.rg.tiles)[ti];
  const int e = tlv.x, row0 = tlv.y, rows = tlv.z, nsub = (rows + 15) >> 4;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int srow = tid >> 2;
  const int spair = c.rg.tok[row0 + min(srow, rows - 1)];
  const int tok = spair / c.K;
  float* actt = reinterpret_cast<float*>(smem);   // [64 rows][kQgActStride], after the K loop
  int* pairs = reinterpret_cast<int*>(smem + 2 * kQgBufBytes);
  if ((tid & 3) == 0) pairs[srow] = spair;
  const size_t tile = (size_t)e * S + sl;
  f32x4_t acc[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) acc[s] = f32x4_t{0, 0, 0, 0};
  {
    const int8_t* rq = a.xq + (size_t)tok * H;
    const float* rd = a.xd + (size_t)tok * KB;
    const char* wt = (const char*)a.w13 + tile * KB * QFmt<QT>::block_bytes;
    const uint16_t* stl = a.w13_d + tile * KB * 64;
    const int tlb = (wave & 1) * 16 + (wave >> 1) * 32;
    switch (nsub) {   // uniform
      case 1: qg_gemm<QT, SC, 1, 1>(smem, rq, rd, KB, wt, stl, tlb, tid, acc); break;
      case 2: qg_gemm<QT, SC, 2, 1>(smem, rq, rd, KB, wt, stl, tlb, tid, acc); break;
      case 3: qg_gemm<QT, SC, 3, 1>(smem, rq, rd, KB, wt, stl, tlb, tid, acc); break;
      default: qg_gemm<QT, SC, 4, 1>(smem, rq, rd, KB, wt, stl, tlb, tid, acc); break;
    }
  }
  // up waves hand their sums to the gate waves; acc[s] = tile row 16s + r,
  // slice columns (wave & 1) * 16 + 4q .. +3
  if (wave >= 2)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      *reinterpret_cast<f32x4_t*>(actt + (16 * s + r) * kQgActStride + (wave - 2) * 16 + 4 * q) = acc[s];
  __syncthreads();
  if (wave < 2)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f32x4_t* p = reinterpret_cast<f32x4_t*>(actt + (16 * s + r) * kQgActStride + wave * 16 + 4 * q);
      f32x4_t u = *p;
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = silu_mul(acc[s][i], u[i]);
      *p = u;
    }
  __syncthreads();
  // thread (row tid/4, 8 columns): amax over the row's 32 values, then q
  {
    const int row = tid >> 2, c8 = (tid & 3) * 8;
    float v[8];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      v[k] = actt[row * kQgActStride + c8 + k];
      const float av = __builtin_fabsf(v[k]);
      amax = av > amax ? av : amax;
    }
#pragma unroll
    for (int m = 1; m <= 2; m <<= 1) {
      const float o = __shfl_xor(amax, m);
      amax = o > amax ? o : amax;
    }
    float id;
    const float d = q8_block_scale(amax, &id);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo |= (uint32_t)(uint8_t)q8_round(v[k] * id) << (8 * k);
      hi |= (uint32_t)(uint8_t)q8_round(v[k + 4] * id) << (8 * k);
    }
    if (row < rows) {
      const size_t p = (size_t)pairs[row];
      *reinterpret_cast<u32x2_t*>(a.act_q + p * I + 32 * sl + c8) = u32x2_t{lo, hi};
      if (c8 == 0) a.act_d[p * S + sl] = d;
    }
  }
}

// down: work item (row tile, 64-row block hb of H = one weight tile); wave w
// owns output rows 64hb + 16w..+15.  eout[pair] gets the fp32 sums (the combine
// kernel follows).
template <int QT, int SC>
__global__ __launch_bounds__(kBlock) void q_gemm2_kernel(const int32_t* ntiles, const int32_t* tiles,
                                                        const int32_t* tok, const int8_t* act_q, const float* act_d,
                                                        const void* w2, const uint16_t* w2_d, QArgs a0) {
  // the leading arguments repeat fields of a0 (preloaded; see q_gemm13_kernel)
  QArgs a = a0;
  a.c.rg.ntiles = const_cast<int32_t*>(ntiles);
  a.c.rg.tiles = const_cast<int32_t*>(tiles);
  a.c.rg.tok = const_cast<int32_t*>(tok);
  a.act_q = const_cast<int8_t*>(act_q);
  a.act_d = const_cast<float*>(act_d);
  a.w2 = w2;
  a.w2_d = w2_d;
  const SchedArgs& c = a.c;
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = c.H, I = c.I, HB = H / 64, KB2 = I / 32;
  const int ti = blockIdx.x / HB, hb = blockIdx.x - ti * HB;
  if (ti >= *c.rg.ntiles) return;   // uniform
  const int4 tlv = reinterpret_cast<const int4*>(c.rg.tiles)[ti];
  const int e = tlv.x, row0 = tlv.y, rows = tlv.z, nsub = (rows + 15) >> 4;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int srow = tid >> 2;
  const int spair = c.rg.tok[row0 + min(srow, rows - 1)];
  int* pairs = reinterpret_cast<int*>(smem + 2 * kQgBufBytes);
  if ((tid & 3) == 0) pairs[srow] = spair;
  const size_t tile = (size_t)e * HB + hb;
  f32x4_t acc[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) acc[s] = f32x4_t{0, 0, 0, 0};
  {
    const int8_t* rq = a.act_q + (size_t)spair * I;
    const float* rd = a.act_d + (size_t)spair * KB2;
    const char* wt = (const char*)a.w2 + tile * KB2 * QFmt<QT>::block_bytes;
    const uint16_t* stl = a.w2_d + tile * KB2 * 64;
    switch (nsub) {   // uniform
      case 1: qg_gemm<QT, SC, 1, 1>(smem, rq, rd, KB2, wt, stl, 16 * wave, tid, acc); break;
      case 2: qg_gemm<QT, SC, 2, 1>(smem, rq, rd, KB2, wt, stl, 16 * wave, tid, acc); break;
      case 3: qg_gemm<QT, SC, 3, 1>(smem, rq, rd, KB2, wt, stl, 16 * wave, tid, acc); break;
      default: qg_gemm<QT, SC, 4, 1>(smem, rq, rd, KB2, wt, stl, 16 * wave, tid, acc); break;
    }
  }
  // acc[s] = tile row 16s + r, output rows 64hb + 16 * wave + 4q .. +3
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int row = 16 * s + r;
    if (s < nsub && row < rows)
      *reinterpret_cast<f32x4_t*>(c.eout + (size_t)pairs[row] * H + 64 * hb + 16 * wave + 4 * q) = acc[s];
  }
}

template <int QT, int SC>
static hipError_t launch_qg_t(const QArgs& a, int tiles_max, hipStream_t st) {
  hipLaunchKernelGGL((q_gemm13_kernel<QT, SC>), dim3(tiles_max * (a.c.I / 32)), dim3(kBlock), kQgLds, st,
                     a.c.rg.ntiles, a.c.rg.tiles, a.c.rg.tok, a.xq, a.xd, a.w13, a.w13_d, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((q_gemm2_kernel<QT, SC>), dim3(tiles_max * (a.c.H / 64)), dim3(kBlock), kQgLds, st,
                     a.c.rg.ntiles, a.c.rg.tiles, a.c.rg.tok, (const int8_t*)a.act_q, (const float*)a.act_d, a.w2,
                     a.w2_d, a);
  return hipGetLastError();
}

hipError_t launch_qint_gemm(const QArgs& a, int qt, int sc, int tiles_max, hipStream_t st) {
  if (qt == 0) return sc == 1 ? launch_qg_t<0, 1>(a, tiles_max, st) : launch_qg_t<0, 0>(a, tiles_max, st);
  return sc == 1 ? launch_qg_t<1, 1>(a, tiles_max, st) : launch_qg_t<1, 0>(a, tiles_max, st);
}

// ---------------------------------------------------------------- weights
// Tile coordinates of wire row `row` of projection proj (0 gate_up [2I rows],
// 1 down [H rows]).
__device__ __forceinline__ void row_to_tile(int proj, int row, int I, int& tile_in_e, int& lane) {
  if (proj == 0) {
    const int up = row >= I;
    const int rr = up ? row - I : row;
    tile_in_e = rr >> 5;
    lane = (rr & 31) + 32 * up;
  } else {
    tile_in_e = row >> 6;
    lane = row & 63;
  }
}

// Q4_0 wire word (elements k..k+7 at nibbles 0..7) -> device word (byte m =
// element m | element m+4 << 4).
__device__ __forceinline__ uint32_t q4_to_dev(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t lo = (w >> (4 * m)) & 0xfu, hi = (w >> (4 * (m + 4))) & 0xfu;
    o |= (lo | (hi << 4)) << (8 * m);
  }
  return o;
}

// One thread per (e, row, block): wire -> device tile, plus its scale.
template <int QT>
__global__ void q_repack_kernel(const void* __restrict__ qs, const uint16_t* __restrict__ d,
                                void* __restrict__ wdst, uint16_t* __restrict__ ddst, int E,
                                int rows, int K, int proj, int I) {
  const int KB = K / 32;
  const size_t total = (size_t)E * rows * KB;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int kb = idx % KB;
    const size_t er = idx / KB;
    const int row = er % rows;
    const int e = (int)(er / rows);
    int ti, lane;
    row_to_tile(proj, row, I, ti, lane);
    const int tiles_per_e = proj == 0 ? I / 32 : rows / 64;
    const size_t tile = (size_t)e * tiles_per_e + ti;
    char* dst = (char*)wdst + tile * KB * QFmt<QT>::block_bytes;
    if constexpr (QT == 0) {
      const u32x4_t* src = reinterpret_cast<const u32x4_t*>((const int8_t*)qs + er * K + kb * 32);
      const u32x4_t a = src[0], b = src[1];
      const u32x2_t qv[4] = {{a.x, a.y}, {a.z, a.w}, {b.x, b.y}, {b.z, b.w}};
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x2_t*>(dst + QLay<0>::off(KB, kb, lane, q)) = qv[q];
    } else {
      const u32x4_t src = *reinterpret_cast<const u32x4_t*>((const uint32_t*)qs + er * (K / 8) + kb * 4);
      const uint32_t qv[4] = {src.x, src.y, src.z, src.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<uint32_t*>(dst + QLay<1>::off(KB, kb, lane, q)) = q4_to_dev(qv[q]);
    }
    ddst[(tile * KB + kb) * 64 + lane] = d[er * KB + kb];
  }
}

hipError_t launch_q_repack(int qt, const void* qs, const uint16_t* d, void* wdst, uint16_t* ddst,
                           int E, int rows, int K, int proj, int I, hipStream_t st) {
  const size_t total = (size_t)E * rows * (K / 32);
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  if (qt == 0)
    hipLaunchKernelGGL(q_repack_kernel<0>, dim3(grid), dim3(256), 0, st, qs, d, wdst, ddst, E, rows, K, proj, I);
  else
    hipLaunchKernelGGL(q_repack_kernel<1>, dim3(grid), dim3(256), 0, st, qs, d, wdst, ddst, E, rows, K, proj, I);
  return hipGetLastError();
}

// Online Q8_0 weight quantization of one projection of one expert
// (quantize_weight_only, Int8-gemm/q8_gemm.cpp:197-260): fp16 scale, q from
// the fp32 reciprocal of the unrounded scale.  One thread per (row, block).
template <int WDT>  // 0 fp16, 1 bf16, 2 fp32
__global__ void q8_online_quant_kernel(const void* __restrict__ w, int N, int K, int e, int proj,
                                       int I, int row_offset, void* __restrict__ wdst,
                                       uint16_t* __restrict__ ddst) {
  const int KB = K / 32;
  const size_t total = (size_t)N * KB;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int kb = idx % KB;
    const int n = (int)(idx / KB);
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const size_t off = (size_t)n * K + kb * 32 + j;
      if constexpr (WDT == 2) v[j] = ((const float*)w)[off];
      else v[j] = to_f32<WDT>(((const uint16_t*)w)[off]);
    }
    int ti, lane;
    const int row = n + row_offset;
    row_to_tile(proj == 2 ? 1 : 0, row, I, ti, lane);
    const int tiles_per_e = proj == 2 ? N / 64 : I / 32;
    const size_t tile = (size_t)e * tiles_per_e + ti;
    int8_t q[32];
    int qs;
    const float d = quant_block_q8_0(v, q, &qs);
    char* dst = (char*)wdst + tile * KB * QFmt<0>::block_bytes;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      *reinterpret_cast<u32x2_t*>(dst + QLay<0>::off(KB, kb, lane, qq)) = *reinterpret_cast<const u32x2_t*>(q + 8 * qq);
    ddst[(tile * KB + kb) * 64 + lane] = f32_to_f16(d);
  }
}

hipError_t launch_q8_online_quant(const void* w, int wdt, int N, int K, int e, int proj, int I,
                                  void* wdst, uint16_t* ddst, hipStream_t st) {
  const size_t total = (size_t)N * (K / 32);
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  const int row_offset = proj == 1 ? I : 0;
  if (wdt == 2)
    hipLaunchKernelGGL(q8_online_quant_kernel<2>, dim3(grid), dim3(256), 0, st, w, N, K, e, proj, I, row_offset, wdst, ddst);
  else if (wdt == 1)
    hipLaunchKernelGGL(q8_online_quant_kernel<1>, dim3(grid), dim3(256), 0, st, w, N, K, e, proj, I, row_offset, wdst, ddst);
  else
    hipLaunchKernelGGL(q8_online_quant_kernel<0>, dim3(grid), dim3(256), 0, st, w, N, K, e, proj, I, row_offset, wdst, ddst);
  return hipGetLastError();
}

// Per-block int32 dots of stored weights (same unpack + block_isum as the
// fused kernels): isum[m][n][kb].  One thread per (m, n, kb).
template <int QT>
__global__ void q_block_dots_kernel(const void* __restrict__ wbase, const int8_t* __restrict__ a_qs,
                                    int32_t* __restrict__ isum, int M, int N, int K, int e, int proj,
                                    int I, int tiles_per_e) {
  const int KB = K / 32;
  const size_t total = (size_t)M * N * KB;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int kb = idx % KB;
    const size_t mn = idx / KB;
    const int n = mn % N;
    const int m = (int)(mn / N);
    int ti, lane;
    row_to_tile(proj, n, I, ti, lane);
    const size_t tile = (size_t)e * tiles_per_e + ti;
    u32x4_t w0, w1;
    load_block<QT>((const char*)wbase + tile * KB * QFmt<QT>::block_bytes, KB, kb, lane, w0, w1);
    int wd[8];
    unpack_w<QT>(w0, w1, wd);
    const int* xv = reinterpret_cast<const int*>(a_qs + (size_t)m * K + kb * 32);
    int xsum = 0;
    if constexpr (QT == 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) xsum = __builtin_amdgcn_sdot4(xv[j], 0x01010101, xsum, false);
    }
    isum[idx] = block_isum<QT>(wd, xv, xsum);
  }
}

// Inverse of row_to_tile: the matrix row held by lane `lane` of tile ti.
__device__ __forceinline__ int tile_lane_row(int proj, int ti, int lane, int I) {
  if (proj == 0) return lane < 32 ? 32 * ti + lane : I + 32 * ti + lane - 32;
  return 64 * ti + lane;
}

// The grouped GEMMs' int8-MFMA block routine on given activation rows: the
// weights of one step as QgWSet loads them, qg_wbytes, qg_mfma from the bias
// accumulator and qg_scaled with qg_wscale's (dw, nb) -- the functions
// qg_block and qg_gemm call.  acc[m][n][kb] = the MFMA result minus the bias
// (Q8_0: isum; Q4_0: 16 * isum), prod[m][n][kb] = the first scaled product
// (Q8_0: round(isum * dw); Q4_0: 16 * round(isum * dw)).  A wave per (16
// lanes of a weight tile, step of kQgStage blocks, 16 activation rows).
template <int QT, int SC>
__global__ __launch_bounds__(64) void q_mfma_block_check_kernel(const void* __restrict__ wbase,
                                                                const uint16_t* __restrict__ sbase,
                                                                const int8_t* __restrict__ a_qs,
                                                                int32_t* __restrict__ acc, float* __restrict__ prod,
                                                                int M, int N, int K, int e, int proj, int I,
                                                                int tiles_per_e) {
  const int KB = K / 32;
  const int lane = threadIdx.x, q = lane >> 4, r = lane & 15;
  const int ti = blockIdx.x >> 2, tlb = (blockIdx.x & 3) * 16;
  const int kb0 = blockIdx.y * kQgStage, m0 = blockIdx.z * 16;
  const size_t tile = (size_t)e * tiles_per_e + ti;
  const char* wtile = (const char*)wbase + tile * KB * QFmt<QT>::block_bytes;
  const uint16_t* stile = sbase + tile * KB * 64;
  QgWSet<QT> ws;
  ws.load(wtile, KB, kb0, tlb + r, q);
  const int ma = min(m0 + r, M - 1);   // activation row of this lane's column
#pragma unroll
  for (int b = 0; b < kQgStage; ++b) {
    const long av = *reinterpret_cast<const long*>(a_qs + (size_t)ma * K + 32 * (kb0 + b) + 8 * q);
    const i32x4_t d = qg_mfma(qg_wbytes<QT>(ws.w[b]), av);
    const int dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tl = tlb + 4 * q + i;
      float dw, nb;
      qg_wscale<SC>(stile[(kb0 + b) * 64 + tl], dw, nb);
      if (m0 + r < M) {
        const size_t o = ((size_t)(m0 + r) * N + tile_lane_row(proj, ti, tl, I)) * KB + kb0 + b;
        acc[o] = dv[i] - kQgBias;
        prod[o] = qg_scaled(dv[i], dw, nb);
      }
    }
  }
}

hipError_t launch_q_mfma_block_check(int qt, int sdt, const void* wbase, const uint16_t* sbase, const int8_t* a_qs,
                                     int32_t* acc, float* prod, int M, int N, int K, int e, int proj, int I,
                                     int tiles_per_e, hipStream_t st) {
  const dim3 grid((unsigned)(tiles_per_e * 4), (unsigned)(K / 32 / kQgStage), (unsigned)((M + 15) / 16));
  auto kern = qt == 0 ? (sdt == 1 ? q_mfma_block_check_kernel<0, 1> : q_mfma_block_check_kernel<0, 0>)
                      : (sdt == 1 ? q_mfma_block_check_kernel<1, 1> : q_mfma_block_check_kernel<1, 0>);
  hipLaunchKernelGGL(kern, grid, dim3(64), 0, st, wbase, sbase, a_qs, acc, prod, M, N, K, e, proj, I, tiles_per_e);
  return hipGetLastError();
}

hipError_t launch_q_block_dots(int qt, const void* wbase, const int8_t* a_qs, int32_t* isum, int M,
                               int N, int K, int e, int proj, int I, int tiles_per_e, hipStream_t st) {
  const size_t total = (size_t)M * N * (K / 32);
  if (total == 0) return hipSuccess;
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  if (qt == 0)
    hipLaunchKernelGGL(q_block_dots_kernel<0>, dim3(grid), dim3(256), 0, st, wbase, a_qs, isum, M, N, K, e, proj, I, tiles_per_e);
  else
    hipLaunchKernelGGL(q_block_dots_kernel<1>, dim3(grid), dim3(256), 0, st, wbase, a_qs, isum, M, N, K, e, proj, I, tiles_per_e);
  return hipGetLastError();
}

}  // namespace mimoe
