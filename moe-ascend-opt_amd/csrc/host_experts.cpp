// host_experts.cpp -- host executor of the hybrid offload path (see
// host_experts.hpp).  Work is split into tasks of (cold expert, block of
// output rows) so every weight byte a call needs is read once per call, by
// one thread, for all the routed rows of its expert.
#include "host_experts.hpp"

#include "cpu_moe.hpp"

#include <immintrin.h>
#include <math.h>
#include <string.h>

#include <algorithm>

namespace mimoe_host {

// ---------------------------------------------------------------- formats
int num_arrays(int quant) { return quant == 2 ? 6 : 4; }

size_t expert_bytes(int quant, int64_t H, int64_t I, int idx) {
  const int64_t N13 = 2 * I;
  if (quant == 2) {   // AWQ, group 128
    switch (idx) {
      case 0: return (size_t)H * (N13 / 8) * 4;
      case 1: return (size_t)(H / 128) * (N13 / 8) * 4;
      case 2: return (size_t)(H / 128) * N13 * 2;
      case 3: return (size_t)I * (H / 8) * 4;
      case 4: return (size_t)(I / 128) * (H / 8) * 4;
      case 5: return (size_t)(I / 128) * H * 2;
      default: return 0;
    }
  }
  const size_t qdiv = quant == 1 ? 2 : 1;
  switch (idx) {
    case 0: return (size_t)N13 * H / qdiv;
    case 1: return (size_t)N13 * (H / 32) * 2;
    case 2: return (size_t)H * I / qdiv;
    case 3: return (size_t)H * (I / 32) * 2;
    default: return 0;
  }
}

namespace {

constexpr int kTokBlock = 256;    // tokens per pass (bounds the per-pair buffers)
constexpr int kQRows = 32;        // output rows per Q task
constexpr int kAwqWords = 16;     // packed words (128 columns) per W4A16 task
constexpr int kAwqOrder[8] = {0, 2, 4, 6, 1, 3, 5, 7};   // nibble slot s -> column 8j + order[s]

float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float f16_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = (float)m * 5.9604644775390625e-8f;   // m * 2^-24 (exact)
    return s ? -v : v;
  }
  if (e == 31) return bits_f32(s | 0x7f800000u | (m << 13));
  return bits_f32(s | ((e + 112u) << 23) | (m << 13));
}

inline float half_f32(uint16_t v, int dt) { return dt == 1 ? bits_f32((uint32_t)v << 16) : f16_f32(v); }

// Q8_0 of n values (n % 32 == 0): d = amax / 127, q = sat8(RNE(x / d))
// (quantize_block_q8_0, Int8-gemm/gemm_kernels.cpp:37-57); d kept as fp32.
void quant_q8_0(const float* x, int64_t n, int8_t* q, float* d) {
  for (int64_t b = 0; b < n / 32; ++b) {
    const float* v = x + 32 * b;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, fabsf(v[i]));
    const float dd = amax / 127.0f, id = dd != 0.0f ? 1.0f / dd : 0.0f;
    d[b] = dd;
    for (int i = 0; i < 32; ++i) {
      const float r = std::min(std::max(nearbyintf(v[i] * id), -128.0f), 127.0f);
      q[32 * b + i] = (int8_t)r;
    }
  }
}

// Q4_0 wire row -> int8 values: element k in u32[k/8] bits 4(k%8), value nibble - 8.
__attribute__((target_clones("avx2", "default")))
void unpack_q4_0(const uint32_t* __restrict__ u, int8_t* __restrict__ row, int64_t nwords) {
  for (int64_t j = 0; j < nwords; ++j) {
    const uint32_t w = u[j];
    for (int i = 0; i < 8; ++i) row[8 * j + i] = (int8_t)((int)((w >> (4 * i)) & 15u) - 8);
  }
}

// One output of a Q8_0 / Q4_0 row: c = sum over the 32-blocks in order of
// ((float)isum_kb * dw[kb]) * da[kb], isum the exact int32 block dot.
__attribute__((target_clones("avx2", "default")))
float q_row_dot(const int8_t* __restrict__ a, const int8_t* __restrict__ w, const float* __restrict__ dw,
                const float* __restrict__ da, int64_t KB) {
  float c = 0.0f;
  for (int64_t kb = 0; kb < KB; ++kb) {
    int32_t is = 0;
    for (int i = 0; i < 32; ++i) is += (int32_t)a[32 * kb + i] * (int32_t)w[32 * kb + i];
    const float t = (float)is * dw[kb];
    c = c + t * da[kb];
  }
  return c;
}

// Rows [n0, n1) of a Q8_0 / Q4_0 matrix ([N][K] wire rows, scales [N][K/32])
// against the Q8_0 rows of P routed pairs: out[p][n] = sum_kb (isum*dw)*da.
void q_rows(int quant, int sdt, const uint8_t* wq, const uint16_t* wd, int64_t K, int64_t n0, int64_t n1,
            const int8_t* const* aq, const float* const* ad, int64_t P, float* const* out) {
  const int64_t KB = K / 32;
  std::vector<int8_t> row(quant == 1 ? (size_t)K : 0);
  std::vector<float> dw((size_t)KB);
  for (int64_t n = n0; n < n1; ++n) {
    const int8_t* w;
    if (quant == 0) {
      w = reinterpret_cast<const int8_t*>(wq) + n * K;
    } else {
      unpack_q4_0(reinterpret_cast<const uint32_t*>(wq) + n * (K / 8), row.data(), K / 8);
      w = row.data();
    }
    for (int64_t kb = 0; kb < KB; ++kb) dw[kb] = half_f32(wd[n * KB + kb], sdt);
    for (int64_t p = 0; p < P; ++p) out[p][n] = q_row_dot(aq[p], w, dw.data(), ad[p], KB);
  }
}

// One 128-k group of a W4A16 column block of packed words (VU: one vector of
// them) for P rows: accg[p][sl][jj] = sum over the group's k, in order, of
// x_p[k] * (nibble sl of word jj) -- one vector of words per k, the 8 slot
// accumulators in registers.
#define MIMOE_VEC(name, T, n) typedef T name __attribute__((vector_size(4 * (n))))
MIMOE_VEC(vu16, uint32_t, 16); MIMOE_VEC(vi16, int32_t, 16); MIMOE_VEC(vf16, float, 16);
MIMOE_VEC(vu8, uint32_t, 8); MIMOE_VEC(vi8, int32_t, 8); MIMOE_VEC(vf8, float, 8);
MIMOE_VEC(vu4, uint32_t, 4); MIMOE_VEC(vi4, int32_t, 4); MIMOE_VEC(vf4, float, 4);
MIMOE_VEC(vu2, uint32_t, 2); MIMOE_VEC(vi2, int32_t, 2); MIMOE_VEC(vf2, float, 2);
#undef MIMOE_VEC

template <typename VU, typename VI, typename VF, int PC>
__attribute__((always_inline)) inline void awq_group_pc(const int32_t* __restrict__ q, int64_t NW, int64_t k0,
                                                        const float* const* xf, float* __restrict__ accg) {
  VF acc[PC][8];
  for (int pp = 0; pp < PC; ++pp)
    for (int sl = 0; sl < 8; ++sl) acc[pp][sl] = VF{};
  for (int64_t k = k0; k < k0 + 128; ++k) {
    VU w;
    memcpy(&w, q + k * NW, sizeof(w));
    for (int sl = 0; sl < 8; ++sl) {
      const VF v = __builtin_convertvector((VI)((w >> (uint32_t)(4 * sl)) & 15u), VF);
      for (int pp = 0; pp < PC; ++pp) acc[pp][sl] += xf[pp][k] * v;
    }
  }
  memcpy(accg, acc, sizeof(acc));
}

// Rows in pairs (one unpack of the words for both), the last one alone.
template <typename VU, typename VI, typename VF>
__attribute__((always_inline)) inline void awq_group_t(const int32_t* __restrict__ q, int64_t NW, int64_t k0,
                                                       const float* const* xf, int64_t P, float* __restrict__ accg) {
  constexpr int64_t stride = 8 * (sizeof(VF) / 4);   // floats per row of accg
  int64_t p = 0;
  for (; p + 2 <= P; p += 2) awq_group_pc<VU, VI, VF, 2>(q, NW, k0, xf + p, accg + p * stride);
  if (p < P) awq_group_pc<VU, VI, VF, 1>(q, NW, k0, xf + p, accg + p * stride);
}

// AVX-512 form of a 16-word group: a nibble slot becomes 16 floats with one
// shift and one vpermps from the table 0..15 (vpermps reads only the low 4
// bits of each index) instead of shift, mask and convert.  The multiply and
// the add stay separate, as in awq_group_pc, so every task width (and so
// every thread count) gives the same bits.  Same accg layout as awq_group_pc.
template <int PC>
__attribute__((target("avx512f"), always_inline)) inline void awq_group16_512_pc(
    const int32_t* __restrict__ q, int64_t NW, int64_t k0, const float* const* xf, float* __restrict__ accg) {
  const __m512 tab = _mm512_setr_ps(0.f, 1.f, 2.f, 3.f, 4.f, 5.f, 6.f, 7.f, 8.f, 9.f, 10.f, 11.f, 12.f, 13.f,
                                    14.f, 15.f);
  __m512 acc[PC][8];
  for (int pp = 0; pp < PC; ++pp)
    for (int sl = 0; sl < 8; ++sl) acc[pp][sl] = _mm512_setzero_ps();
  for (int64_t k = k0; k < k0 + 128; ++k) {
    const __m512i w = _mm512_loadu_si512(reinterpret_cast<const void*>(q + k * NW));
    __m512 xv[PC];
    for (int pp = 0; pp < PC; ++pp) xv[pp] = _mm512_set1_ps(xf[pp][k]);
#pragma GCC unroll 8
    for (int sl = 0; sl < 8; ++sl) {
      const __m512i idx = sl == 0 ? w : _mm512_srli_epi32(w, 4 * sl);
      const __m512 v = _mm512_permutexvar_ps(idx, tab);
      for (int pp = 0; pp < PC; ++pp) acc[pp][sl] = _mm512_add_ps(acc[pp][sl], _mm512_mul_ps(xv[pp], v));
    }
  }
  for (int pp = 0; pp < PC; ++pp)
    for (int sl = 0; sl < 8; ++sl) _mm512_storeu_ps(accg + (pp * 8 + sl) * 16, acc[pp][sl]);
}

__attribute__((target("avx512f"))) void awq_group16_512(const int32_t* q, int64_t NW, int64_t k0,
                                                        const float* const* xf, int64_t P, float* accg) {
  int64_t p = 0;
  for (; p + 2 <= P; p += 2) awq_group16_512_pc<2>(q, NW, k0, xf + p, accg + p * 128);
  if (p < P) awq_group16_512_pc<1>(q, NW, k0, xf + p, accg + p * 128);
}

const bool kHostAvx512 = __builtin_cpu_supports("avx512f");

__attribute__((target_clones("avx512f", "avx2", "default")))
void awq_group_generic(int nww, const int32_t* q, int64_t NW, int64_t k0, const float* const* xf, int64_t P,
                       float* accg) {
  switch (nww) {
    case 16: awq_group_t<vu16, vi16, vf16>(q, NW, k0, xf, P, accg); break;
    case 8: awq_group_t<vu8, vi8, vf8>(q, NW, k0, xf, P, accg); break;
    case 4: awq_group_t<vu4, vi4, vf4>(q, NW, k0, xf, P, accg); break;
    default: awq_group_t<vu2, vi2, vf2>(q, NW, k0, xf, P, accg); break;
  }
}

void awq_group(int nww, const int32_t* q, int64_t NW, int64_t k0, const float* const* xf, int64_t P, float* accg) {
  if (nww == 16 && kHostAvx512) awq_group16_512(q, NW, k0, xf, P, accg);
  else awq_group_generic(nww, q, NW, k0, xf, P, accg);
}

// Columns [8*j0, 8*j1) of an AWQ matrix (qweight [K][N/8], qzeros [K/128][N/8],
// scales [K/128][N]) against P fp32 rows xf[p] [K] with group sums xs[p]
// [K/128]: out[p][n] = sum_g s * (sum_k x_k q_kn - z * xs_g).  j1 - j0 is
// 2, 4, 8 or 16 words.
// qb points at word j0 of k row 0 and k rows are qstride words apart (N / 8
// in the wire layout, 16 in the block-major copy).
void awq_cols(const int32_t* qb, int64_t qstride, const int32_t* z, const uint16_t* s, int sdt, int64_t K,
              int64_t N, int64_t j0, int64_t j1, const float* const* xf, const float* const* xs, int64_t P,
              float* const* out) {
  const int64_t NW = N / 8, G = K / 128, nw = j1 - j0, nc = nw * 8;
  // acc / accg / sf / zf in slot-major order: index sl*nw + (j - j0)
  std::vector<float> acc((size_t)(P * nc), 0.0f), accg((size_t)(P * nc)), sf((size_t)nc), zf((size_t)nc);
  for (int64_t g = 0; g < G; ++g) {
    awq_group((int)nw, qb, qstride, 128 * g, xf, P, accg.data());
    for (int64_t j = j0; j < j1; ++j) {
      const uint32_t u = (uint32_t)z[g * NW + j];
      for (int sl = 0; sl < 8; ++sl) {
        const int64_t i = sl * nw + (j - j0);
        zf[i] = (float)((u >> (4 * sl)) & 15u);
        sf[i] = half_f32(s[g * N + 8 * j + kAwqOrder[sl]], sdt);
      }
    }
    for (int64_t p = 0; p < P; ++p) {
      float* a = &acc[p * nc];
      const float* b = &accg[p * nc];
      const float x = xs[p][g];
      for (int64_t i = 0; i < nc; ++i) a[i] += sf[i] * (b[i] - zf[i] * x);
    }
  }
  for (int64_t p = 0; p < P; ++p)
    for (int64_t j = j0; j < j1; ++j)
      for (int sl = 0; sl < 8; ++sl) out[p][8 * j + kAwqOrder[sl]] = acc[p * nc + sl * nw + (j - j0)];
}

// ---------------------------------------------------------------- W4A16 gate_up, AVX512-BF16
// With bf16 hidden rows, gate_up runs on vdpbf16ps: lane i of a 64-column
// block accumulates column 4i + s (slot s = 0..3) over k pairs,
//   acc += w(2kp + 1) * x(2kp + 1), then acc += w(2kp) * x(2kp)
// (bf16 x small-integer products are exact in fp32; the instruction treats
// bf16 denormal inputs as zero).  A k-pair word's slot s, shifted down by 4s,
// indexes a 32-entry bf16 table of 0..15 (vpermw reads 5 index bits; entries
// 16..31 repeat 0..15, so the neighbouring nibble's low bit does not matter).
const bool kHostBf16 = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                       __builtin_cpu_supports("avx512bf16");

#define MIMOE_BF16 __attribute__((target("avx512f,avx512bw,avx512bf16")))

template <int PC>
MIMOE_BF16 __attribute__((always_inline)) inline void pair_group_pc(const uint32_t* __restrict__ q, int64_t kp0,
                                                                    const uint16_t* const* xp,
                                                                    float* __restrict__ accg) {
  alignas(64) static const uint16_t tab16[32] = {
      0x0000, 0x3f80, 0x4000, 0x4040, 0x4080, 0x40a0, 0x40c0, 0x40e0, 0x4100, 0x4110, 0x4120,
      0x4130, 0x4140, 0x4150, 0x4160, 0x4170, 0x0000, 0x3f80, 0x4000, 0x4040, 0x4080, 0x40a0,
      0x40c0, 0x40e0, 0x4100, 0x4110, 0x4120, 0x4130, 0x4140, 0x4150, 0x4160, 0x4170};
  const __m512i tab = _mm512_load_si512(tab16);
  __m512 acc[PC][4];
  for (int pp = 0; pp < PC; ++pp)
    for (int sl = 0; sl < 4; ++sl) acc[pp][sl] = _mm512_setzero_ps();
  for (int64_t kp = kp0; kp < kp0 + 64; ++kp) {
    const __m512i w = _mm512_loadu_si512(reinterpret_cast<const void*>(q + 16 * kp));
    __m512i xv[PC];
    for (int pp = 0; pp < PC; ++pp) {
      int32_t x2;   // x[2kp] in the low half, x[2kp + 1] in the high half
      memcpy(&x2, xp[pp] + 2 * kp, 4);
      xv[pp] = _mm512_set1_epi32(x2);
    }
#pragma GCC unroll 4
    for (int sl = 0; sl < 4; ++sl) {
      const __m512i idx = sl == 0 ? w : _mm512_srli_epi32(w, 4 * sl);
      const __m512i v = _mm512_permutexvar_epi16(idx, tab);
      for (int pp = 0; pp < PC; ++pp)
        acc[pp][sl] = _mm512_dpbf16_ps(acc[pp][sl], (__m512bh)v, (__m512bh)xv[pp]);
    }
  }
  for (int pp = 0; pp < PC; ++pp)
    for (int sl = 0; sl < 4; ++sl) _mm512_storeu_ps(accg + (pp * 4 + sl) * 16, acc[pp][sl]);
}

// Columns [64b, 64b + 64) of the k-pair gate_up matrix of one expert against
// P bf16 rows xp[p] with fp32 group sums xs[p]:
// out[p][n] = sum_g s * (sum_k x_k q_kn - z * xs_g), as awq_cols.
MIMOE_BF16 void pair_cols(const uint32_t* pq, const uint8_t* pz, const uint16_t* ps, int sdt, int64_t K, int64_t N,
                          int64_t b, const uint16_t* const* xp, const float* const* xs, int64_t P,
                          float* const* out) {
  const int64_t G = K / 128;
  std::vector<float> acc((size_t)(P * 64), 0.0f), accg((size_t)(P * 64));
  const uint32_t* q = pq + b * (K / 2) * 16;
  for (int64_t g = 0; g < G; ++g) {
    int64_t p = 0;
    for (; p + 2 <= P; p += 2) pair_group_pc<2>(q, 64 * g, xp + p, accg.data() + p * 64);
    if (p < P) pair_group_pc<1>(q, 64 * g, xp + p, accg.data() + p * 64);
    const uint8_t* zg = pz + g * N + 64 * b;
    const uint16_t* sg = ps + g * N + 64 * b;
    for (int sl = 0; sl < 4; ++sl) {
      const __m512 zf = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i*>(zg + 16 * sl))));
      const __m256i sb = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(sg + 16 * sl));
      const __m512 sf = sdt == 1 ? _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(sb), 16))
                                 : _mm512_cvtph_ps(sb);
      for (int64_t pp = 0; pp < P; ++pp) {
        float* a = acc.data() + pp * 64 + 16 * sl;
        const __m512 gsum = _mm512_loadu_ps(accg.data() + pp * 64 + 16 * sl);
        const __m512 t = _mm512_sub_ps(gsum, _mm512_mul_ps(zf, _mm512_set1_ps(xs[pp][g])));
        _mm512_storeu_ps(a, _mm512_add_ps(_mm512_loadu_ps(a), _mm512_mul_ps(sf, t)));
      }
    }
  }
  for (int64_t pp = 0; pp < P; ++pp)
    for (int sl = 0; sl < 4; ++sl)
      for (int i = 0; i < 16; ++i) out[pp][64 * b + 4 * i + sl] = acc[(size_t)(pp * 64 + 16 * sl + i)];
}

#undef MIMOE_BF16

void prepare_pairs(ColdSet& cs) {
  const int64_t H = cs.H, I = cs.I, N = 2 * I, NW = N / 8, G = H / 128, Ec = cs.Ec;
  cs.pq.assign((size_t)(Ec * (H / 2) * (N / 4)), 0u);
  cs.pz.assign((size_t)(Ec * G * N), 0);
  cs.ps.assign((size_t)(Ec * G * N), 0);
  // slot of column offset o within an AWQ word (kAwqOrder inverted)
  int slot_of[8];
  for (int sl = 0; sl < 8; ++sl) slot_of[kAwqOrder[sl]] = sl;
  for (int64_t c = 0; c < Ec; ++c) {
    const int32_t* q = reinterpret_cast<const int32_t*>(cs.arr[0].data() + c * expert_bytes(2, H, cs.I, 0));
    const int32_t* z = reinterpret_cast<const int32_t*>(cs.arr[1].data() + c * expert_bytes(2, H, cs.I, 1));
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(cs.arr[2].data() + c * expert_bytes(2, H, cs.I, 2));
    auto nib = [&](const int32_t* m, int64_t row, int64_t n) {
      return ((uint32_t)m[row * NW + n / 8] >> (4 * slot_of[n % 8])) & 15u;
    };
    uint32_t* pq = cs.pq.data() + c * (H / 2) * (N / 4);
    for (int64_t b = 0; b < N / 64; ++b)
      for (int64_t kp = 0; kp < H / 2; ++kp)
        for (int64_t i = 0; i < 16; ++i) {
          uint32_t v = 0;
          for (int s = 0; s < 4; ++s) {
            const int64_t n = 64 * b + 4 * i + s;
            v |= nib(q, 2 * kp, n) << (4 * s) | nib(q, 2 * kp + 1, n) << (16 + 4 * s);
          }
          pq[(b * (H / 2) + kp) * 16 + i] = v;
        }
    for (int64_t g = 0; g < G; ++g)
      for (int64_t n = 0; n < N; ++n) {
        const int64_t b = n / 64, i = (n % 64) / 4, s = n % 4, at = (c * G + g) * N + 64 * b + 16 * s + i;
        cs.pz[(size_t)at] = (uint8_t)nib(z, g, n);
        cs.ps[(size_t)at] = sc[g * N + n];
      }
  }
}

}  // namespace

void prepare_host_layouts(ColdSet& cs) {
  const int64_t H = cs.H, I = cs.I, N = 2 * I, Ec = cs.Ec;
  cs.bq13.clear();
  cs.bq2.clear();
  cs.pq.clear();
  cs.pz.clear();
  cs.ps.clear();
  if (cs.quant != 2 || Ec == 0 || H % 128 != 0 || I % 128 != 0) return;
  // block-major copies of the two qweight arrays: [Ec][N/128][K][16]
  auto block_major = [&](std::vector<int32_t>& dst, int a, int64_t K, int64_t Nn) {
    dst.assign((size_t)(Ec * K * (Nn / 8)), 0);
    for (int64_t c = 0; c < Ec; ++c) {
      const int32_t* src = reinterpret_cast<const int32_t*>(cs.arr[a].data() + c * expert_bytes(2, H, I, a));
      for (int64_t b = 0; b < Nn / 128; ++b)
        for (int64_t k = 0; k < K; ++k)
          memcpy(&dst[(size_t)(((c * (Nn / 128) + b) * K + k) * 16)], src + k * (Nn / 8) + 16 * b, 64);
    }
  };
  block_major(cs.bq13, 0, H, N);
  block_major(cs.bq2, 3, I, H);
  if (kHostBf16) prepare_pairs(cs);
  // the wire qweights are not read again (zeros and scales still are)
  std::vector<uint8_t>().swap(cs.arr[0]);
  std::vector<uint8_t>().swap(cs.arr[3]);
}

int64_t forward(const ColdSet& cs, Pool& pool, const uint16_t* x, int act_dtype, const int32_t* ids,
                const float* topk_w, int64_t T, int64_t K, float* y_part) {
  const int64_t H = cs.H, I = cs.I, N13 = 2 * I, E = cs.E, Ec = cs.Ec;
  const bool awq = cs.quant == 2;
  memset(y_part, 0, sizeof(float) * (size_t)(T * H));
  if (Ec == 0 || T == 0) return 0;
  size_t eb[6];
  for (int a = 0; a < 6; ++a) eb[a] = expert_bytes(cs.quant, H, I, a);
  int64_t total = 0;
  for (int64_t t0 = 0; t0 < T; t0 += kTokBlock) {
    const int64_t t1 = std::min(T, t0 + kTokBlock), nT = t1 - t0;
    // cold pairs of the block grouped by cold expert, pair order kept
    std::vector<int64_t> start((size_t)Ec + 1, 0);
    std::vector<int32_t> cold((size_t)(nT * K), -1);
    for (int64_t i = 0; i < nT * K; ++i) {
      const int32_t e = ids[t0 * K + i];
      if (e >= 0 && e < E && cs.cold_of[e] >= 0) {
        cold[i] = cs.cold_of[e];
        ++start[cold[i] + 1];
      }
    }
    for (int64_t c = 0; c < Ec; ++c) start[c + 1] += start[c];
    const int64_t P = start[Ec];
    if (P == 0) continue;
    total += P;
    std::vector<int64_t> pair_of((size_t)P), pos_of((size_t)(nT * K), -1), fill(start.begin(), start.end() - 1);
    for (int64_t i = 0; i < nT * K; ++i)
      if (cold[i] >= 0) {
        const int64_t pos = fill[cold[i]]++;
        pair_of[pos] = i;
        pos_of[i] = pos;
      }
    // per-pair and per-token stages of a few rows run on the calling thread
    // (waking the pool costs more than the work)
    auto small_run = [&](int64_t n, const std::function<void(int64_t)>& f) {
      if (n <= 16) {
        for (int64_t i = 0; i < n; ++i) f(i);
      } else {
        pool.run(n, f);
      }
    };
    // activations of the block's tokens (W4A16: with their 128-k group sums)
    std::vector<float> xf((size_t)(nT * H));
    std::vector<float> gu((size_t)(P * N13)), out((size_t)(P * H));
    std::vector<const float*> pxf((size_t)P), pxs((size_t)P);
    std::vector<const int8_t*> paq((size_t)P);
    std::vector<const float*> pad((size_t)P);
    std::vector<float*> pgu((size_t)P), pout((size_t)P);
    std::vector<float> xs, act;
    std::vector<int8_t> xq, aq;
    std::vector<float> xd, ad;
    const int64_t G1 = H / 128, G2 = I / 128;
    if (awq) xs.resize((size_t)(nT * G1));
    small_run(nT, [&](int64_t t) {
      mimoe_cpu::half_row_to_f32(x + (t0 + t) * H, H, act_dtype, &xf[t * H]);
      if (awq) mimoe_cpu::group_sums_128(&xf[t * H], G1, &xs[t * G1]);
    });
    if (!awq) {
      xq.resize((size_t)(nT * H));
      xd.resize((size_t)(nT * (H / 32)));
      pool.run(nT, [&](int64_t t) { quant_q8_0(&xf[t * H], H, &xq[t * H], &xd[t * (H / 32)]); });
    }
    for (int64_t p = 0; p < P; ++p) {
      const int64_t t = pair_of[p] / K;
      pxf[p] = &xf[t * H];
      if (awq) pxs[p] = &xs[t * G1];
      else { paq[p] = &xq[t * H]; pad[p] = &xd[t * (H / 32)]; }
      pgu[p] = &gu[p * N13];
      pout[p] = &out[p * H];
    }
    // tasks of (cold expert with pairs, block of output columns / rows):
    // W4A16 blocks of 128 columns, each one contiguous run of the
    // block-major copy (64 columns on the k-pair copy)
    std::vector<int64_t> task_c;
    for (int64_t c = 0; c < Ec; ++c)
      if (start[c + 1] > start[c]) task_c.push_back(c);
    const int64_t nc = (int64_t)task_c.size();
    auto qblock = [&](const std::vector<int32_t>& bq, int64_t c, int64_t K, int64_t N, int64_t b) {
      return bq.data() + ((c * (N / 128) + b) * K) * 16;
    };
    const int aw = kAwqWords;
    const int64_t blk13 = awq ? (N13 / 8) / aw : N13 / kQRows;
    const int64_t blk2 = awq ? (H / 8) / aw : H / kQRows;
    // bf16 hidden rows and a k-pair copy: 64-column tasks on vdpbf16ps
    const bool pairs = awq && act_dtype == 1 && !cs.pq.empty();
    std::vector<const uint16_t*> pxp(pairs ? (size_t)P : 0);
    for (int64_t p = 0; pairs && p < P; ++p) pxp[p] = x + (t0 + pair_of[p] / K) * H;
    const int64_t blkp = N13 / 64;
    if (pairs) {
      pool.run(nc * blkp, [&](int64_t task) {
        const int64_t c = task_c[task / blkp], b = task % blkp, p0 = start[c], np = start[c + 1] - p0;
        pair_cols(cs.pq.data() + c * (H / 2) * (N13 / 4), cs.pz.data() + c * G1 * N13, cs.ps.data() + c * G1 * N13,
                  cs.scale_dtype, H, N13, b, &pxp[p0], &pxs[p0], np, &pgu[p0]);
      });
    } else pool.run(nc * blk13, [&](int64_t task) {
      const int64_t c = task_c[task / blk13], b = task % blk13, p0 = start[c], np = start[c + 1] - p0;
      if (awq) {
        awq_cols(qblock(cs.bq13, c, H, N13, b), 16,
                 reinterpret_cast<const int32_t*>(cs.arr[1].data() + c * eb[1]),
                 reinterpret_cast<const uint16_t*>(cs.arr[2].data() + c * eb[2]), cs.scale_dtype, H, N13,
                 b * aw, (b + 1) * aw, &pxf[p0], &pxs[p0], np, &pgu[p0]);
      } else {
        q_rows(cs.quant, cs.scale_dtype, cs.arr[0].data() + c * eb[0],
               reinterpret_cast<const uint16_t*>(cs.arr[1].data() + c * eb[1]), H, b * kQRows, (b + 1) * kQRows,
               &paq[p0], &pad[p0], np, &pgu[p0]);
      }
    });
    // SiLU(gate) * up, then the down projection's input rows
    act.resize((size_t)(P * I));
    if (awq) xs.assign((size_t)(P * G2), 0.0f);
    else { aq.resize((size_t)(P * I)); ad.resize((size_t)(P * (I / 32))); }
    small_run(P, [&](int64_t p) {
      float* a = &act[p * I];
      const float* g = &gu[p * N13];
      mimoe_cpu::silu_mul_row(g, g + I, I, a);
      if (awq) {
        mimoe_cpu::group_sums_128(a, G2, &xs[p * G2]);
      } else {
        quant_q8_0(a, I, &aq[p * I], &ad[p * (I / 32)]);
      }
    });
    for (int64_t p = 0; p < P; ++p) {
      pxf[p] = &act[p * I];
      if (awq) pxs[p] = &xs[p * G2];
      else { paq[p] = &aq[p * I]; pad[p] = &ad[p * (I / 32)]; }
    }
    pool.run(nc * blk2, [&](int64_t task) {
      const int64_t c = task_c[task / blk2], b = task % blk2, p0 = start[c], np = start[c + 1] - p0;
      if (awq) {
        awq_cols(qblock(cs.bq2, c, I, H, b), 16,
                 reinterpret_cast<const int32_t*>(cs.arr[4].data() + c * eb[4]),
                 reinterpret_cast<const uint16_t*>(cs.arr[5].data() + c * eb[5]), cs.scale_dtype, I, H,
                 b * aw, (b + 1) * aw, &pxf[p0], &pxs[p0], np, &pout[p0]);
      } else {
        q_rows(cs.quant, cs.scale_dtype, cs.arr[2].data() + c * eb[2],
               reinterpret_cast<const uint16_t*>(cs.arr[3].data() + c * eb[3]), I, b * kQRows, (b + 1) * kQRows,
               &paq[p0], &pad[p0], np, &pout[p0]);
      }
    });
    // weighted sum over k in ascending order
    small_run(nT, [&](int64_t t) {
      float* yr = y_part + (t0 + t) * H;
      for (int64_t k = 0; k < K; ++k) {
        const int64_t pos = pos_of[t * K + k];
        if (pos < 0) continue;
        const float w = topk_w[(t0 + t) * K + k];
        const float* o = &out[pos * H];
        for (int64_t h = 0; h < H; ++h) {
          const float prod = w * o[h];
          yr[h] = yr[h] + prod;
        }
      }
    });
  }
  return total;
}

}  // namespace mimoe_host
