// cpu_moe.cpp -- the reference's CPU fused-MoE algorithm for Q8_0 / Q4_0
// weights on x86 host cores: the CPU dispatch key of nanovllm::moe_forward and
// the CPU baseline the GPU path is measured beside.
//
// Pipeline (moe_forward_ptr_impl, Int8-gemm/q8_gemm.cpp:276-646):
//   Stage A   every token's hidden row -> Q8_0 blocks (fp32 d), once per TP shard
//   routing   stable counting sort of the (t, k) pairs by expert
//             (preprocess_moe_routing, Int8-gemm/moe_common.cpp:146-216)
//   tasks     per expert with routed rows, chunks of M_BLOCK = 32 rows
//             (Int8-gemm/q8_gemm.cpp:335-347)
//   Stage B   per task: gate_up rows c = sum_kb (isum * dw) * da in block order,
//             SiLU(gate) * up, the intermediate -> Q8_0, down rows likewise, into
//             the per-row expert outputs (expert-sorted).  When tasks * 2 <=
//             threads each task takes 2 threads: gate rows / up rows, then (after
//             the phase boundary) each thread re-activates the whole intermediate
//             and takes half of the down rows (Int8-gemm/q8_gemm.cpp:379-490);
//             otherwise one thread per task (:491-590).  The intermediate of a
//             task lives at its first routed row, not at its task index (the
//             reference's small-task path indexes it by task, which races when a
//             task has more than one row).
//   Stage C1  per token, sum over k in order of topk_w * expert row (fp32)
//   Stage C2  TP partials summed in shard order, cast to the hidden dtype (RNE)
// TP: the intermediate dimension is split over tp shards, one per NUMA node
// holding worker threads (gate/up rows and down columns of the shard,
// Int8-gemm/moe_infer.cpp:143-205); each shard's threads are pinned to their
// node and touch (repack) their shard's weights first, so first-touch places
// them on that node.
//
// Dot products: exact int32 per 32-element block on the widest instruction set
// the host has (picked at run time, overridable downwards):
//   AVX-512 VNNI / AVX-VNNI  vpdpbusd u8 x s8 -> s32 (4 products per lane):
//             Q8_0 activations enter as a ^ 0x80 = a + 128 and the stored
//             128 * sum(w) of the row's block is subtracted; Q4_0 nibbles are
//             the unsigned operand and 8 * sum(a) of the block is subtracted
//   AVX2      vpmaddubsw + vpmaddwd: Q8_0 as |w| x (a * sign(w)) (activations
//             are in [-127, 127] after Q8_0 quantization, so no pair sum
//             saturates), Q4_0 as nibble x a
//   scalar    plain int32 loops
// The scaling is ((float)isum * dw) * da added in block order, operation by
// operation (this file is built with -ffp-contract=off), SiLU uses the
// Cody-Waite + degree-7 Taylor exp of the device code, so the result is
// independent of the instruction set and of the thread count.
#include "cpu_moe.hpp"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <string>
#include <thread>

namespace mimoe_cpu {

// ---------------------------------------------------------------- scalars
namespace {

float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
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
template <class V>
void grow(V& v, size_t n) {   // size at least n; existing contents need not survive
  if (v.size() < n) v.resize(n);
}

float half_f32(uint16_t v, int dt) { return dt == 1 ? bits_f32((uint32_t)v << 16) : f16_f32(v); }

uint16_t f32_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
// fp32 -> fp16 bits, round to nearest even (overflow -> inf, subnormals kept)
uint16_t f32_f16(float f) {
  const uint32_t u = f32_bits(f), s = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);   // rounds to >= 65520: inf
  if (a < 0x38800000u) {                                   // below 2^-14: subnormal half
    const float v = bits_f32(a) * 16777216.0f;             // value / 2^-24, exact scaling
    return (uint16_t)(s | (uint32_t)nearbyintf(v));
  }
  const uint32_t mant = a & 0x7fffffu, e = (a >> 23) - 112u;
  uint32_t h = (e << 10) | (mant >> 13);
  const uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(s | h);
}
uint16_t f32_half(float f, int dt) { return dt == 1 ? f32_bf16(f) : f32_f16(f); }

// exp(x): Cody & Waite (1980) reduction n = rint(x log2 e), r = (x - n*C1) - n*C2
// with C1 = 355/512, then the degree-7 Taylor series of exp(r) (Horner) and a
// 2^n exponent-field scale -- the operation sequence of the device code.
float expf_cw(float x) {
  if (x != x) return x;
  if (x > 88.5f) return bits_f32(0x7f800000u);
  if (x < -87.0f) return 0.0f;
  const float n = nearbyintf(x * 1.44269504088896341f);
  float r = fmaf(-n, 0.693359375f, x);
  r = fmaf(-n, -2.12194440e-4f, r);
  float p = 1.98412698412698413e-4f;
  p = fmaf(p, r, 1.38888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  if (ni < -126) { p = p * bits_f32(0x00800000u); ni += 126; }
  return p * bits_f32((uint32_t)(ni + 127) << 23);
}

// Q8_0 of 32 floats (quantize_block_q8_0, Int8-gemm/gemm_kernels.cpp:25-58):
// d = amax / 127, q = sat8(RNE(x * (1/d))); returns d.
float quant_block(const float* v, int8_t* q) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, fabsf(v[i]));
  const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float x = v[i] * id;
    float r = x != x ? 0.0f : nearbyintf(x);
    r = std::min(std::max(r, -128.0f), 127.0f);
    q[i] = (int8_t)r;
  }
  return d;
}

// ---------------------------------------------------------------- row quantizers
// Q8_0 of a hidden row (Stage A) and of SiLU(gate) * up (the intermediate),
// with the biased bytes q ^ 0x80 and the int32 block sums the dot kernels
// take.  The AVX2 + FMA forms do the scalar forms' operations lane by lane:
// the same absolute maximum (NaN lanes ignored), d = amax / 127 and 1 / d,
// RNE rounding (vroundps in place of nearbyintf), the exp's fma chain and
// exponent scaling, the same division for the sigmoid -- so both write the
// same bytes and scales.
void finish_block(const int8_t* q, uint8_t* qb, int32_t* s) {
  int32_t sum = 0;
  for (int j = 0; j < 32; ++j) {
    qb[j] = (uint8_t)(q[j] ^ 0x80);
    sum += q[j];
  }
  *s = sum;
}

void quant_hidden_scalar(const uint16_t* x, int64_t n, int dt, int8_t* q, uint8_t* qb, float* d, int32_t* s) {
  float v[32];
  for (int64_t b = 0; b < n / 32; ++b) {
    for (int j = 0; j < 32; ++j) v[j] = half_f32(x[32 * b + j], dt);
    d[b] = quant_block(v, q + 32 * b);
    finish_block(q + 32 * b, qb + 32 * b, s + b);
  }
}

void quant_act_scalar(const float* gate, const float* up, int64_t n, int8_t* q, uint8_t* qb, float* d, int32_t* s) {
  float v[32];
  for (int64_t b = 0; b < n / 32; ++b) {
    for (int j = 0; j < 32; ++j) {
      const float g = gate[32 * b + j], u = up[32 * b + j];
      const float eg = expf_cw(-g);
      const float denom = 1.0f + eg;
      const float sig = g / denom;
      v[j] = u * sig;
    }
    d[b] = quant_block(v, q + 32 * b);
    finish_block(q + 32 * b, qb + 32 * b, s + b);
  }
}

#define MIMOE_AVX2 __attribute__((target("avx2,fma,f16c")))

MIMOE_AVX2 inline __m256i round_q8(__m256 x, __m256 vid) {
  const __m256 t = _mm256_mul_ps(x, vid);
  __m256 r = _mm256_round_ps(t, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  r = _mm256_andnot_ps(_mm256_cmp_ps(t, t, _CMP_UNORD_Q), r);   // NaN -> 0
  r = _mm256_min_ps(_mm256_max_ps(r, _mm256_set1_ps(-128.0f)), _mm256_set1_ps(127.0f));
  return _mm256_cvttps_epi32(r);
}

// one block of 32 values in x0..x3 (elements 0-7, 8-15, 16-23, 24-31)
MIMOE_AVX2 inline void quant32_avx2(__m256 x0, __m256 x1, __m256 x2, __m256 x3, int8_t* q, uint8_t* qb, float* d,
                                    int32_t* s) {
  const __m256 mag = _mm256_castsi256_ps(_mm256_set1_epi32(0x7fffffff));
  // max(|x|, m): a NaN in the first operand returns the second, so NaN lanes
  // are skipped as in the scalar loop
  __m256 m = _mm256_max_ps(_mm256_and_ps(x0, mag), _mm256_setzero_ps());
  m = _mm256_max_ps(_mm256_and_ps(x1, mag), m);
  m = _mm256_max_ps(_mm256_and_ps(x2, mag), m);
  m = _mm256_max_ps(_mm256_and_ps(x3, mag), m);
  __m128 h = _mm_max_ps(_mm256_castps256_ps128(m), _mm256_extractf128_ps(m, 1));
  h = _mm_max_ps(h, _mm_movehl_ps(h, h));
  h = _mm_max_ss(h, _mm_shuffle_ps(h, h, 1));
  const float amax = _mm_cvtss_f32(h);
  const float dd = amax / 127.0f, id = dd != 0.0f ? 1.0f / dd : 0.0f;
  *d = dd;
  const __m256 vid = _mm256_set1_ps(id);
  const __m256i q0 = round_q8(x0, vid), q1 = round_q8(x1, vid), q2 = round_q8(x2, vid), q3 = round_q8(x3, vid);
  __m256i t = _mm256_add_epi32(_mm256_add_epi32(q0, q1), _mm256_add_epi32(q2, q3));
  __m128i t4 = _mm_add_epi32(_mm256_castsi256_si128(t), _mm256_extracti128_si256(t, 1));
  t4 = _mm_add_epi32(t4, _mm_shuffle_epi32(t4, 0x4e));
  t4 = _mm_add_epi32(t4, _mm_shuffle_epi32(t4, 0xb1));
  *s = _mm_cvtsi128_si32(t4);
  // packs work per 128-bit lane: 4-byte groups come out as q0 lo, q1 lo,
  // q2 lo, q3 lo, q0 hi, ...; the permute restores element order
  const __m256i p = _mm256_packs_epi16(_mm256_packs_epi32(q0, q1), _mm256_packs_epi32(q2, q3));
  const __m256i o = _mm256_permutevar8x32_epi32(p, _mm256_setr_epi32(0, 4, 1, 5, 2, 6, 3, 7));
  _mm256_storeu_si256(reinterpret_cast<__m256i*>(q), o);
  _mm256_storeu_si256(reinterpret_cast<__m256i*>(qb), _mm256_xor_si256(o, _mm256_set1_epi8((char)0x80)));
}

MIMOE_AVX2 inline __m256 load_half8(const uint16_t* x, int dt) {
  const __m128i h = _mm_loadu_si128(reinterpret_cast<const __m128i*>(x));
  if (dt == 1) return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
  return _mm256_cvtph_ps(h);   // exact (NaN payloads aside, and NaN lanes quantize to 0)
}

MIMOE_AVX2 void quant_hidden_avx2(const uint16_t* x, int64_t n, int dt, int8_t* q, uint8_t* qb, float* d, int32_t* s) {
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint16_t* xb = x + 32 * b;
    quant32_avx2(load_half8(xb, dt), load_half8(xb + 8, dt), load_half8(xb + 16, dt), load_half8(xb + 24, dt),
                 q + 32 * b, qb + 32 * b, d + b, s + b);
  }
}

// expf_cw on 8 lanes
MIMOE_AVX2 inline __m256 expf_cw8(__m256 x) {
  const __m256 xc = _mm256_min_ps(_mm256_max_ps(x, _mm256_set1_ps(-87.0f)), _mm256_set1_ps(88.5f));
  const __m256 n = _mm256_round_ps(_mm256_mul_ps(xc, _mm256_set1_ps(1.44269504088896341f)),
                                   _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m256 r = _mm256_fnmadd_ps(n, _mm256_set1_ps(0.693359375f), xc);     // fmaf(-n, C1, x)
  r = _mm256_fnmadd_ps(n, _mm256_set1_ps(-2.12194440e-4f), r);          // fmaf(-n, C2, r)
  __m256 p = _mm256_set1_ps(1.98412698412698413e-4f);
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.38888888888888889e-3f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(8.33333333333333333e-3f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(4.16666666666666667e-2f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.66666666666666667e-1f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  __m256i ni = _mm256_cvttps_epi32(n);
  const __m256i hi = _mm256_cmpgt_epi32(ni, _mm256_set1_epi32(127));
  p = _mm256_blendv_ps(p, _mm256_mul_ps(p, _mm256_set1_ps(2.0f)), _mm256_castsi256_ps(hi));
  ni = _mm256_add_epi32(ni, hi);   // hi = -1 where taken
  const __m256i lo = _mm256_cmpgt_epi32(_mm256_set1_epi32(-126), ni);
  p = _mm256_blendv_ps(p, _mm256_mul_ps(p, _mm256_set1_ps(bits_f32(0x00800000u))), _mm256_castsi256_ps(lo));
  ni = _mm256_add_epi32(ni, _mm256_and_si256(lo, _mm256_set1_epi32(126)));
  __m256 e = _mm256_mul_ps(p, _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_add_epi32(ni, _mm256_set1_epi32(127)), 23)));
  e = _mm256_blendv_ps(e, _mm256_set1_ps(bits_f32(0x7f800000u)), _mm256_cmp_ps(x, _mm256_set1_ps(88.5f), _CMP_GT_OQ));
  e = _mm256_blendv_ps(e, _mm256_setzero_ps(), _mm256_cmp_ps(x, _mm256_set1_ps(-87.0f), _CMP_LT_OQ));
  return _mm256_blendv_ps(e, x, _mm256_cmp_ps(x, x, _CMP_UNORD_Q));
}

MIMOE_AVX2 inline __m256 silu_mul8(const float* gate, const float* up) {
  const __m256 g = _mm256_loadu_ps(gate), u = _mm256_loadu_ps(up);
  const __m256 eg = expf_cw8(_mm256_xor_ps(g, _mm256_set1_ps(-0.0f)));
  const __m256 denom = _mm256_add_ps(_mm256_set1_ps(1.0f), eg);
  return _mm256_mul_ps(u, _mm256_div_ps(g, denom));
}

MIMOE_AVX2 void quant_act_avx2(const float* gate, const float* up, int64_t n, int8_t* q, uint8_t* qb, float* d,
                               int32_t* s) {
  for (int64_t b = 0; b < n / 32; ++b) {
    const float* g = gate + 32 * b;
    const float* u = up + 32 * b;
    quant32_avx2(silu_mul8(g, u), silu_mul8(g + 8, u + 8), silu_mul8(g + 16, u + 16), silu_mul8(g + 24, u + 24),
                 q + 32 * b, qb + 32 * b, d + b, s + b);
  }
}

MIMOE_AVX2 void silu_mul_avx2(const float* gate, const float* up, int64_t n, float* out) {
  int64_t j = 0;
  for (; j + 8 <= n; j += 8) _mm256_storeu_ps(out + j, silu_mul8(gate + j, up + j));
  for (; j < n; ++j) out[j] = up[j] * (gate[j] / (1.0f + expf_cw(-gate[j])));
}

// sums of 128-element groups: 8 lanes of 16 elements each (lane l takes
// elements l, l + 8, ...), then the lanes in a fixed tree
MIMOE_AVX2 void group_sums_avx2(const float* a, int64_t ngroups, float* sums) {
  for (int64_t g = 0; g < ngroups; ++g) {
    const float* v = a + 128 * g;
    __m256 t[4];
    for (int i = 0; i < 4; ++i) t[i] = _mm256_loadu_ps(v + 8 * i);
    for (int i = 4; i < 16; ++i) t[i & 3] = _mm256_add_ps(t[i & 3], _mm256_loadu_ps(v + 8 * i));
    const __m256 u = _mm256_add_ps(_mm256_add_ps(t[0], t[1]), _mm256_add_ps(t[2], t[3]));
    __m128 h = _mm_add_ps(_mm256_castps256_ps128(u), _mm256_extractf128_ps(u, 1));
    h = _mm_add_ps(h, _mm_movehl_ps(h, h));
    h = _mm_add_ss(h, _mm_shuffle_ps(h, h, 1));
    sums[g] = _mm_cvtss_f32(h);
  }
}

MIMOE_AVX2 void half_to_f32_avx2(const uint16_t* x, int64_t n, int dt, float* out) {
  int64_t j = 0;
  for (; j + 8 <= n; j += 8) _mm256_storeu_ps(out + j, load_half8(x + j, dt));
  for (; j < n; ++j) out[j] = half_f32(x[j], dt);
}

// acc[j] = acc[j] + w * row[j]: a product, then a sum (no fused multiply-add)
MIMOE_AVX2 void axpy_avx2(float w, const float* row, float* acc, int64_t n) {
  const __m256 vw = _mm256_set1_ps(w);
  int64_t j = 0;
  for (; j + 8 <= n; j += 8)
    _mm256_storeu_ps(acc + j, _mm256_add_ps(_mm256_loadu_ps(acc + j), _mm256_mul_ps(vw, _mm256_loadu_ps(row + j))));
  for (; j < n; ++j) {
    const float prod = w * row[j];
    acc[j] = acc[j] + prod;
  }
}

#undef MIMOE_AVX2

void axpy_row(bool simd, float w, const float* row, float* acc, int64_t n) {
  if (simd) {
    axpy_avx2(w, row, acc, n);
    return;
  }
  for (int64_t j = 0; j < n; ++j) {
    const float prod = w * row[j];
    acc[j] = acc[j] + prod;
  }
}

}  // namespace

float half_to_f32(uint16_t v, int dt) { return half_f32(v, dt); }

// make_topk_from_logits_cpu (Int8-gemm/test/fused_moe_cpu.py:20-37): K
// selection passes over the row, then the softmax of the picks (renormalize)
// or of the whole row gathered at the picks.
void topk_softmax(const float* logits, int64_t T, int64_t E, int64_t K, int renormalize, int32_t* ids,
                  float* w) {
  std::vector<unsigned char> taken((size_t)E);
  std::vector<float> ex((size_t)(E > K ? E : K));
  for (int64_t t = 0; t < T; ++t) {
    const float* x = logits + t * E;
    int32_t* oi = ids + t * K;
    std::fill(taken.begin(), taken.end(), (unsigned char)0);
    for (int64_t k = 0; k < K; ++k) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e)
        if (!taken[(size_t)e] && (best < 0 || x[e] > x[best])) best = e;
      taken[(size_t)best] = 1;
      oi[k] = (int32_t)best;
    }
    const float m = x[oi[0]];
    float s = 0.0f;
    if (renormalize) {
      for (int64_t k = 0; k < K; ++k) {
        ex[(size_t)k] = expf_cw(x[oi[k]] - m);
        s = s + ex[(size_t)k];
      }
      for (int64_t k = 0; k < K; ++k) w[t * K + k] = ex[(size_t)k] / s;
    } else {
      for (int64_t e = 0; e < E; ++e) {
        ex[(size_t)e] = expf_cw(x[e] - m);
        s = s + ex[(size_t)e];
      }
      for (int64_t k = 0; k < K; ++k) w[t * K + k] = ex[(size_t)oi[k]] / s;
    }
  }
}

void quant_hidden_row(bool simd, const uint16_t* x, int64_t n, int dt, int8_t* q, uint8_t* qb, float* d,
                      int32_t* s) {
  if (simd) quant_hidden_avx2(x, n, dt, q, qb, d, s);
  else quant_hidden_scalar(x, n, dt, q, qb, d, s);
}

void quant_act_row(bool simd, const float* gate, const float* up, int64_t n, int8_t* q, uint8_t* qb, float* d,
                   int32_t* s) {
  if (simd) quant_act_avx2(gate, up, n, q, qb, d, s);
  else quant_act_scalar(gate, up, n, q, qb, d, s);
}

bool host_simd() {
  static const bool ok = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
                         __builtin_cpu_supports("f16c");
  return ok;
}

void silu_mul_row(const float* gate, const float* up, int64_t n, float* out) {
  if (host_simd()) {
    silu_mul_avx2(gate, up, n, out);
    return;
  }
  for (int64_t j = 0; j < n; ++j) {
    const float g = gate[j];
    out[j] = up[j] * (g / (1.0f + expf_cw(-g)));
  }
}

void group_sums_128(const float* a, int64_t ngroups, float* sums) {
  if (host_simd()) {
    group_sums_avx2(a, ngroups, sums);
    return;
  }
  for (int64_t g = 0; g < ngroups; ++g) {   // the same lanes and tree as the AVX2 form
    float lane[8];
    for (int l = 0; l < 8; ++l) {
      float t[4];
      for (int i = 0; i < 4; ++i) t[i] = a[128 * g + 8 * i + l];
      for (int i = 4; i < 16; ++i) t[i & 3] = t[i & 3] + a[128 * g + 8 * i + l];
      lane[l] = (t[0] + t[1]) + (t[2] + t[3]);
    }
    float h[4];
    for (int l = 0; l < 4; ++l) h[l] = lane[l] + lane[l + 4];
    sums[g] = (h[0] + h[2]) + (h[1] + h[3]);
  }
}

void half_row_to_f32(const uint16_t* x, int64_t n, int dt, float* out) {
  if (host_simd()) {
    half_to_f32_avx2(x, n, dt, out);
    return;
  }
  for (int64_t j = 0; j < n; ++j) out[j] = half_f32(x[j], dt);
}

// ---------------------------------------------------------------- ISA
Isa detect_isa() {
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
      __builtin_cpu_supports("avx512vnni"))
    return Isa::kAvx512Vnni;
  if (__builtin_cpu_supports("avxvnni") && __builtin_cpu_supports("avx2")) return Isa::kAvxVnni;
  if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return Isa::kAvx2;
  return Isa::kScalar;
}

bool isa_supported(Isa i) {
  __builtin_cpu_init();
  switch (i) {
    case Isa::kAvx512Vnni:
      return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
             __builtin_cpu_supports("avx512vnni");
    case Isa::kAvxVnni: return __builtin_cpu_supports("avxvnni") && __builtin_cpu_supports("avx2");
    case Isa::kAvx2: return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    default: return true;
  }
}

const char* isa_name(Isa i) {
  switch (i) {
    case Isa::kAvx512Vnni: return "avx512_vnni";
    case Isa::kAvxVnni: return "avx_vnni";
    case Isa::kAvx2: return "avx2";
    default: return "scalar";
  }
}

// ---------------------------------------------------------------- packing
// Panel layout (16 weight rows x all K blocks), per (panel p, block kb):
//   Q8_0: 512 B = [8 steps of 4 k][16 rows][4 B]
//   Q4_0: 256 B = [4 steps of 8 k][16 rows][4 B], byte j of a row: low nibble
//         k0 + j, high nibble k0 + 4 + j (the unsigned nibble n; value n - 8)
// scales d [p][kb][16] fp32; Q8_0 also wsum [p][kb][16] = 128 * sum of the 32 w.
void PackedMat::init(int qt_, int64_t N_, int64_t K_) {
  qt = qt_;
  N = N_;
  K = K_;
  const int64_t P = N / kNR, KB = K / 32;
  blk = qt == 0 ? 512 : 256;
  qs.assign((size_t)(P * KB * blk), 0);
  d.assign((size_t)(P * KB * kNR), 0.0f);
  ws.assign(qt == 0 ? (size_t)(P * KB * kNR) : 0, 0);
}

void PackedMat::set_row(int64_t n, const int8_t* w, const float* dw) {
  // w: K values (Q8_0 int8, Q4_0 value n - 8 in [-8, 7]); dw: K/32 scales
  const int64_t p = n / kNR, r = n % kNR, KB = K / 32;
  for (int64_t kb = 0; kb < KB; ++kb) {
    uint8_t* b = qs.data() + (size_t)((p * KB + kb) * blk);
    const int8_t* wb = w + 32 * kb;
    if (qt == 0) {
      int32_t s = 0;
      for (int st = 0; st < 8; ++st)
        for (int j = 0; j < 4; ++j) {
          b[st * 64 + 4 * r + j] = (uint8_t)wb[4 * st + j];
          s += wb[4 * st + j];
        }
      ws[(size_t)((p * KB + kb) * kNR + r)] = 128 * s;
    } else {
      for (int st = 0; st < 4; ++st)
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = (uint32_t)(wb[8 * st + j] + 8), hi = (uint32_t)(wb[8 * st + 4 + j] + 8);
          b[st * 64 + 4 * r + j] = (uint8_t)(lo | (hi << 4));
        }
    }
    d[(size_t)((p * KB + kb) * kNR + r)] = dw[kb];
  }
}

// ---------------------------------------------------------------- kernels
// C[m][n0 + i] for the rows m < M of A (quantized activations: bytes a [M][K],
// biased bytes ab = a ^ 0x80 [M][K], block scales ad [M][KB], block sums as
// [M][KB]) and the weight rows [n0, n1) of W (multiples of 16):
//   c = sum_kb ((float)isum_kb * dw) * da_kb, isum exact int32.
struct ARows {
  const int8_t* a;
  const uint8_t* ab;
  const float* ad;
  const int32_t* as;
  int64_t lda;   // bytes per row of a / ab; blocks per row of ad / as = K / 32
};

namespace {

constexpr int kMR = 4;   // activation rows per register block

void gemm_scalar(const PackedMat& W, const ARows& A, int M, int64_t n0, int64_t n1, float* C, int64_t ldc) {
  const int64_t KB = W.K / 32;
  for (int64_t p = n0 / kNR; p < n1 / kNR; ++p)
    for (int m = 0; m < M; ++m)
      for (int r = 0; r < kNR; ++r) {
        float c = 0.0f;
        for (int64_t kb = 0; kb < KB; ++kb) {
          const uint8_t* b = W.qs.data() + (size_t)((p * KB + kb) * W.blk);
          const int8_t* a = A.a + m * A.lda + 32 * kb;
          int32_t s = 0;
          if (W.qt == 0) {
            for (int st = 0; st < 8; ++st)
              for (int j = 0; j < 4; ++j) s += (int32_t)a[4 * st + j] * (int32_t)(int8_t)b[st * 64 + 4 * r + j];
          } else {
            for (int st = 0; st < 4; ++st)
              for (int j = 0; j < 4; ++j) {
                const uint8_t v = b[st * 64 + 4 * r + j];
                s += (int32_t)a[8 * st + j] * ((int32_t)(v & 15) - 8) + (int32_t)a[8 * st + 4 + j] * ((int32_t)(v >> 4) - 8);
              }
          }
          const float t1 = (float)s * W.d[(size_t)((p * KB + kb) * kNR + r)];
          const float t2 = t1 * A.ad[m * KB + kb];
          c = c + t2;
        }
        C[m * ldc + p * kNR + r] = c;
      }
}

// MR activation rows (compile-time) against one 16-row panel over all K.
template <int MR>
__attribute__((target("avx512f,avx512bw,avx512vnni"), always_inline)) inline void panel_avx512vnni(
    const PackedMat& W, const ARows& A, int m0, int64_t p, float* C, int64_t ldc) {
  const int64_t KB = W.K / 32;
  const __m512i nib = _mm512_set1_epi8(0x0f);
  __m512 acc[MR];
#pragma GCC unroll 4
  for (int i = 0; i < MR; ++i) acc[i] = _mm512_setzero_ps();
  for (int64_t kb = 0; kb < KB; ++kb) {
    const uint8_t* b = W.qs.data() + (size_t)((p * KB + kb) * W.blk);
    __m512i is[MR];
#pragma GCC unroll 4
    for (int i = 0; i < MR; ++i) is[i] = _mm512_setzero_si512();
    if (W.qt == 0) {
#pragma GCC unroll 8
      for (int st = 0; st < 8; ++st) {
        const __m512i w = _mm512_loadu_si512(b + 64 * st);
#pragma GCC unroll 4
        for (int i = 0; i < MR; ++i) {
          int32_t a4;
          memcpy(&a4, A.ab + (m0 + i) * A.lda + 32 * kb + 4 * st, 4);
          is[i] = _mm512_dpbusd_epi32(is[i], _mm512_set1_epi32(a4), w);
        }
      }
      const __m512i wsum = _mm512_loadu_si512(W.ws.data() + (size_t)((p * KB + kb) * kNR));
#pragma GCC unroll 4
      for (int i = 0; i < MR; ++i) is[i] = _mm512_sub_epi32(is[i], wsum);
    } else {
#pragma GCC unroll 4
      for (int st = 0; st < 4; ++st) {
        const __m512i w = _mm512_loadu_si512(b + 64 * st);
        const __m512i lo = _mm512_and_si512(w, nib), hi = _mm512_and_si512(_mm512_srli_epi16(w, 4), nib);
#pragma GCC unroll 4
        for (int i = 0; i < MR; ++i) {
          int32_t a4l, a4h;
          memcpy(&a4l, A.a + (m0 + i) * A.lda + 32 * kb + 8 * st, 4);
          memcpy(&a4h, A.a + (m0 + i) * A.lda + 32 * kb + 8 * st + 4, 4);
          is[i] = _mm512_dpbusd_epi32(is[i], lo, _mm512_set1_epi32(a4l));
          is[i] = _mm512_dpbusd_epi32(is[i], hi, _mm512_set1_epi32(a4h));
        }
      }
#pragma GCC unroll 4
      for (int i = 0; i < MR; ++i) is[i] = _mm512_sub_epi32(is[i], _mm512_set1_epi32(8 * A.as[(m0 + i) * KB + kb]));
    }
    const __m512 dw = _mm512_loadu_ps(W.d.data() + (size_t)((p * KB + kb) * kNR));
#pragma GCC unroll 4
    for (int i = 0; i < MR; ++i) {
      const __m512 t1 = _mm512_mul_ps(_mm512_cvtepi32_ps(is[i]), dw);
      const __m512 t2 = _mm512_mul_ps(t1, _mm512_set1_ps(A.ad[(m0 + i) * KB + kb]));
      acc[i] = _mm512_add_ps(acc[i], t2);
    }
  }
#pragma GCC unroll 4
  for (int i = 0; i < MR; ++i) _mm512_storeu_ps(C + (m0 + i) * ldc + p * kNR, acc[i]);
}

__attribute__((target("avx512f,avx512bw,avx512vnni")))
void gemm_avx512vnni(const PackedMat& W, const ARows& A, int M, int64_t n0, int64_t n1, float* C, int64_t ldc) {
  for (int64_t p = n0 / kNR; p < n1 / kNR; ++p)
    for (int m0 = 0; m0 < M; m0 += kMR) {
      switch (std::min(kMR, M - m0)) {
        case 1: panel_avx512vnni<1>(W, A, m0, p, C, ldc); break;
        case 2: panel_avx512vnni<2>(W, A, m0, p, C, ldc); break;
        case 3: panel_avx512vnni<3>(W, A, m0, p, C, ldc); break;
        default: panel_avx512vnni<4>(W, A, m0, p, C, ldc); break;
      }
    }
}

// 4-k dots of one activation row against 8 weight rows (one ymm of int32).
// Q8_0: the VNNI form takes the biased bytes (a + 128) and the caller removes
// 128 * sum(w); the AVX2 form is |w| x (a * sign(w)) -- with a in [-127, 127]
// (Q8_0 activations) no int16 pair sum saturates.  Q4_0: nibbles x a.
__attribute__((target("avx2,fma,avxvnni"), always_inline)) inline __m256i q8_dot_vnni(__m256i acc, __m256i w,
                                                                                     const uint8_t* ab, const int8_t*) {
  int32_t a4;
  memcpy(&a4, ab, 4);
  return _mm256_dpbusd_avx_epi32(acc, _mm256_set1_epi32(a4), w);
}
__attribute__((target("avx2,fma"), always_inline)) inline __m256i q8_dot_avx2(__m256i acc, __m256i w, const uint8_t*,
                                                                             const int8_t* a) {
  int32_t a4;
  memcpy(&a4, a, 4);
  const __m256i p16 = _mm256_maddubs_epi16(_mm256_abs_epi8(w), _mm256_sign_epi8(_mm256_set1_epi32(a4), w));
  return _mm256_add_epi32(acc, _mm256_madd_epi16(p16, _mm256_set1_epi16(1)));
}
__attribute__((target("avx2,fma,avxvnni"), always_inline)) inline __m256i q4_dot_vnni(__m256i acc, __m256i lo,
                                                                                     __m256i hi, const int8_t* a) {
  int32_t a4l, a4h;
  memcpy(&a4l, a, 4);
  memcpy(&a4h, a + 4, 4);
  acc = _mm256_dpbusd_avx_epi32(acc, lo, _mm256_set1_epi32(a4l));
  return _mm256_dpbusd_avx_epi32(acc, hi, _mm256_set1_epi32(a4h));
}
__attribute__((target("avx2,fma"), always_inline)) inline __m256i q4_dot_avx2(__m256i acc, __m256i lo, __m256i hi,
                                                                             const int8_t* a) {
  int32_t a4l, a4h;
  memcpy(&a4l, a, 4);
  memcpy(&a4h, a + 4, 4);
  const __m256i pl = _mm256_maddubs_epi16(lo, _mm256_set1_epi32(a4l));
  const __m256i ph = _mm256_maddubs_epi16(hi, _mm256_set1_epi32(a4h));
  return _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_add_epi16(pl, ph), _mm256_set1_epi16(1)));
}

// 16 rows as two ymm halves (rows 0-7: bytes [0, 32) of a step, rows 8-15:
// [32, 64)) for MR (compile-time) activation rows.  Expanded for two targets,
// each with its own dot helpers; BIASED_: Q8_0 dots include 128 * sum(w).
#define MIMOE_AVX2_PANEL(NAME, TARGET, Q8DOT, Q4DOT, BIASED_)                                               \
  template <int MR>                                                                                         \
  __attribute__((target(TARGET), always_inline)) inline void NAME(const PackedMat& W, const ARows& A, int m0, \
                                                                  int64_t p, float* C, int64_t ldc) {       \
    const int64_t KB = W.K / 32;                                                                            \
    const __m256i nib = _mm256_set1_epi8(0x0f);                                                             \
    __m256 acc[MR][2];                                                                                      \
    for (int i = 0; i < MR; ++i) acc[i][0] = acc[i][1] = _mm256_setzero_ps();                               \
    for (int64_t kb = 0; kb < KB; ++kb) {                                                                   \
      const uint8_t* b = W.qs.data() + (size_t)((p * KB + kb) * W.blk);                                     \
      __m256i is[MR][2];                                                                                    \
      for (int i = 0; i < MR; ++i) is[i][0] = is[i][1] = _mm256_setzero_si256();                           \
      if (W.qt == 0) {                                                                                      \
        for (int st = 0; st < 8; ++st)                                                                      \
          for (int h = 0; h < 2; ++h) {                                                                     \
            const __m256i w = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(b + 64 * st + 32 * h));   \
            for (int i = 0; i < MR; ++i)                                                                    \
              is[i][h] = Q8DOT(is[i][h], w, A.ab + (m0 + i) * A.lda + 32 * kb + 4 * st,                    \
                               A.a + (m0 + i) * A.lda + 32 * kb + 4 * st);                                  \
          }                                                                                                 \
        if (BIASED_)                                                                                        \
          for (int h = 0; h < 2; ++h) {                                                                     \
            const __m256i wsum = _mm256_loadu_si256(                                                        \
                reinterpret_cast<const __m256i*>(W.ws.data() + (size_t)((p * KB + kb) * kNR) + 8 * h));     \
            for (int i = 0; i < MR; ++i) is[i][h] = _mm256_sub_epi32(is[i][h], wsum);                      \
          }                                                                                                 \
      } else {                                                                                              \
        for (int st = 0; st < 4; ++st)                                                                      \
          for (int h = 0; h < 2; ++h) {                                                                     \
            const __m256i w = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(b + 64 * st + 32 * h));   \
            const __m256i lo = _mm256_and_si256(w, nib), hi = _mm256_and_si256(_mm256_srli_epi16(w, 4), nib); \
            for (int i = 0; i < MR; ++i) is[i][h] = Q4DOT(is[i][h], lo, hi, A.a + (m0 + i) * A.lda + 32 * kb + 8 * st); \
          }                                                                                                 \
        for (int i = 0; i < MR; ++i) {                                                                      \
          const __m256i c8 = _mm256_set1_epi32(8 * A.as[(m0 + i) * KB + kb]);                               \
          is[i][0] = _mm256_sub_epi32(is[i][0], c8);                                                        \
          is[i][1] = _mm256_sub_epi32(is[i][1], c8);                                                        \
        }                                                                                                   \
      }                                                                                                     \
      for (int h = 0; h < 2; ++h) {                                                                         \
        const __m256 dw = _mm256_loadu_ps(W.d.data() + (size_t)((p * KB + kb) * kNR) + 8 * h);              \
        for (int i = 0; i < MR; ++i) {                                                                      \
          const __m256 t1 = _mm256_mul_ps(_mm256_cvtepi32_ps(is[i][h]), dw);                                \
          const __m256 t2 = _mm256_mul_ps(t1, _mm256_set1_ps(A.ad[(m0 + i) * KB + kb]));                    \
          acc[i][h] = _mm256_add_ps(acc[i][h], t2);                                                         \
        }                                                                                                   \
      }                                                                                                     \
    }                                                                                                       \
    for (int i = 0; i < MR; ++i)                                                                            \
      for (int h = 0; h < 2; ++h) _mm256_storeu_ps(C + (m0 + i) * ldc + p * kNR + 8 * h, acc[i][h]);      \
  }

MIMOE_AVX2_PANEL(panel_avxvnni, "avx2,fma,avxvnni", q8_dot_vnni, q4_dot_vnni, true)
MIMOE_AVX2_PANEL(panel_avx2, "avx2,fma", q8_dot_avx2, q4_dot_avx2, false)

#define MIMOE_PANEL_LOOP(PANEL)                                                 \
  for (int64_t p = n0 / kNR; p < n1 / kNR; ++p)                                  \
    for (int m0 = 0; m0 < M; m0 += kMR) {                                        \
      switch (std::min(kMR, M - m0)) {                                           \
        case 1: PANEL<1>(W, A, m0, p, C, ldc); break;                            \
        case 2: PANEL<2>(W, A, m0, p, C, ldc); break;                            \
        case 3: PANEL<3>(W, A, m0, p, C, ldc); break;                            \
        default: PANEL<4>(W, A, m0, p, C, ldc); break;                           \
      }                                                                          \
    }

__attribute__((target("avx2,fma,avxvnni")))
void gemm_avxvnni(const PackedMat& W, const ARows& A, int M, int64_t n0, int64_t n1, float* C, int64_t ldc) {
  MIMOE_PANEL_LOOP(panel_avxvnni)
}
__attribute__((target("avx2,fma")))
void gemm_avx2(const PackedMat& W, const ARows& A, int M, int64_t n0, int64_t n1, float* C, int64_t ldc) {
  MIMOE_PANEL_LOOP(panel_avx2)
}
#undef MIMOE_PANEL_LOOP
#undef MIMOE_AVX2_PANEL

}  // namespace

// Rows [n0, n1) of W against M activation rows, on the given instruction set.
void gemm_rows(Isa isa, const PackedMat& W, const ARows& A, int M, int64_t n0, int64_t n1, float* C, int64_t ldc) {
  switch (isa) {
    case Isa::kAvx512Vnni: gemm_avx512vnni(W, A, M, n0, n1, C, ldc); break;
    case Isa::kAvxVnni: gemm_avxvnni(W, A, M, n0, n1, C, ldc); break;
    case Isa::kAvx2: gemm_avx2(W, A, M, n0, n1, C, ldc); break;
    default: gemm_scalar(W, A, M, n0, n1, C, ldc); break;
  }
}

// ---------------------------------------------------------------- topology
namespace {

std::vector<int> parse_cpulist(const std::string& s) {
  std::vector<int> out;
  std::stringstream ss(s);
  std::string tok;
  while (std::getline(ss, tok, ',')) {
    if (tok.empty()) continue;
    const size_t dash = tok.find('-');
    if (dash == std::string::npos) {
      out.push_back(atoi(tok.c_str()));
    } else {
      const int a = atoi(tok.substr(0, dash).c_str()), b = atoi(tok.substr(dash + 1).c_str());
      for (int c = a; c <= b; ++c) out.push_back(c);
    }
  }
  return out;
}

// node of each CPU (from /sys; every CPU on node 0 when it is absent)
std::vector<int> cpu_nodes(int ncpu) {
  std::vector<int> node((size_t)ncpu, 0);
  for (int nd = 0; nd < 64; ++nd) {
    std::ifstream f("/sys/devices/system/node/node" + std::to_string(nd) + "/cpulist");
    if (!f) continue;
    std::string line;
    std::getline(f, line);
    for (int c : parse_cpulist(line))
      if (c >= 0 && c < ncpu) node[(size_t)c] = nd;
  }
  return node;
}

}  // namespace

Topology host_topology(int max_threads) {
  Topology t;
  cpu_set_t set;
  CPU_ZERO(&set);
  std::vector<int> cpus;
  if (sched_getaffinity(0, sizeof(set), &set) == 0) {
    for (int c = 0; c < CPU_SETSIZE; ++c)
      if (CPU_ISSET(c, &set)) cpus.push_back(c);
  }
  if (cpus.empty()) {
    const int n = (int)std::max(1u, std::thread::hardware_concurrency());
    for (int c = 0; c < n; ++c) cpus.push_back(c);
  }
  t.affinity_cpus = (int)cpus.size();
  const std::vector<int> node = cpu_nodes(cpus.back() + 1);
  // take whole nodes' CPUs in node order until max_threads are chosen
  std::vector<int> order(cpus);
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return node[(size_t)a] < node[(size_t)b]; });
  const int want = max_threads > 0 ? std::min(max_threads, (int)order.size()) : (int)order.size();
  for (int i = 0; i < want; ++i) {
    const int c = order[(size_t)i], nd = node[(size_t)c];
    if (t.node_cpus.empty() || t.node_ids.back() != nd) {
      t.node_ids.push_back(nd);
      t.node_cpus.emplace_back();
    }
    t.node_cpus.back().push_back(c);
  }
  std::vector<int> all_nodes;
  for (int c : cpus) all_nodes.push_back(node[(size_t)c]);
  std::sort(all_nodes.begin(), all_nodes.end());
  t.affinity_nodes = (int)(std::unique(all_nodes.begin(), all_nodes.end()) - all_nodes.begin());
  return t;
}

// ---------------------------------------------------------------- pool
NodePool::NodePool(const std::vector<int>& cpus) : cpus_(cpus) {
  pool_.reset(new mimoe_pool::WorkerPool(std::max(1, (int)cpus_.size()), [this](int i) { pin(i); }));
}

void NodePool::pin(int i) {
  if (i >= (int)cpus_.size()) return;
  cpu_set_t s;
  CPU_ZERO(&s);
  CPU_SET(cpus_[(size_t)i], &s);
  (void)pthread_setaffinity_np(pthread_self(), sizeof(s), &s);
}

// ---------------------------------------------------------------- engine
Engine::Engine(int64_t E, int64_t H, int64_t I, int qt, int max_threads, int tp)
    : E_(E), H_(H), I_(I), qt_(qt), isa_(detect_isa()) {
  topo_ = host_topology(max_threads);
  // one shard per node holding chosen CPUs; a forced tp regroups the CPUs
  std::vector<std::vector<int>> groups = topo_.node_cpus;
  if (tp > 0 && tp != (int)groups.size()) {
    std::vector<int> all;
    for (auto& g : groups) all.insert(all.end(), g.begin(), g.end());
    groups.assign((size_t)tp, {});
    for (size_t i = 0; i < all.size(); ++i) groups[i * (size_t)tp / all.size()].push_back(all[i]);
    for (auto& g : groups)
      if (g.empty()) g.push_back(all.empty() ? 0 : all[0]);
  }
  tp_ = (int)groups.size();
  for (auto& g : groups) pools_.emplace_back(new NodePool(g));
  threads_ = 0;
  for (auto& p : pools_) threads_ += p->size();
  shards_.resize((size_t)tp_);
  scratch_.resize((size_t)tp_);
}

Engine::Engine(int64_t E, int64_t H, int64_t I, int qt, NumaLayout, int tp, int threads_per_node)
    : E_(E), H_(H), I_(I), qt_(qt), isa_(detect_isa()) {
  topo_ = host_topology(0);
  const std::vector<std::vector<int>>& nodes = topo_.node_cpus;
  const int ntp = tp > 0 ? tp : (int)std::max<size_t>(1, nodes.size());
  std::vector<std::vector<int>> groups;
  if ((int)nodes.size() >= ntp) {
    for (int s = 0; s < ntp; ++s) groups.push_back(nodes[(size_t)s]);
  } else {
    std::vector<int> all;
    for (auto& g : nodes) all.insert(all.end(), g.begin(), g.end());
    if (all.empty()) all.push_back(0);
    groups.assign((size_t)ntp, {});
    for (size_t i = 0; i < all.size(); ++i) groups[i * (size_t)ntp / all.size()].push_back(all[i]);
    for (auto& g : groups)
      if (g.empty()) g.push_back(all[0]);
  }
  for (auto& g : groups)
    if (threads_per_node > 0 && (int)g.size() > threads_per_node) g.resize((size_t)threads_per_node);
  tp_ = (int)groups.size();
  for (auto& g : groups) pools_.emplace_back(new NodePool(g));
  threads_ = 0;
  for (auto& p : pools_) threads_ += p->size();
  shards_.resize((size_t)tp_);
  scratch_.resize((size_t)tp_);
}

Engine::~Engine() = default;

bool Engine::shape_ok() const {
  return tp_ >= 1 && I_ % tp_ == 0 && (I_ / tp_) % 32 == 0 && H_ % 32 == 0;
}

// Wire weights -> the shards' panels.  gate_up rows of shard s: [gate rows
// s*Ish .. +Ish | up rows I + s*Ish .. +Ish]; down rows all H, columns
// [s*Ish, (s+1)*Ish) (Int8-gemm/moe_infer.cpp:143-205).  Each shard's pool
// writes its own panels (first touch on its node).
void Engine::store(const void* gate_up_qs, const uint16_t* gate_up_d, const void* down_qs, const uint16_t* down_d,
                   int scale_dtype) {
  const int64_t E = E_, H = H_, I = I_, Ish = I / tp_;
  for (int s = 0; s < tp_; ++s) {
    Shard& sh = shards_[(size_t)s];
    sh.w13.assign((size_t)E, PackedMat());
    sh.w2.assign((size_t)E, PackedMat());
    pools_[(size_t)s]->run(E, [&, s](int64_t e) {
      Shard& shd = shards_[(size_t)s];
      PackedMat& g = shd.w13[(size_t)e];
      PackedMat& dn = shd.w2[(size_t)e];
      g.init(qt_, 2 * Ish, H);
      dn.init(qt_, H, Ish);
      std::vector<int8_t> row((size_t)std::max(H, I));
      std::vector<float> dw((size_t)(std::max(H, I) / 32));
      auto wire_row = [&](const void* qs, const uint16_t* d, int64_t wrow, int64_t K, int64_t k0, int64_t kn) {
        // values k0 .. k0+kn of wire row `wrow` (K per row) -> row / dw
        for (int64_t k = 0; k < kn; ++k) {
          const int64_t kk = k0 + k;
          if (qt_ == 0) {
            row[(size_t)k] = reinterpret_cast<const int8_t*>(qs)[wrow * K + kk];
          } else {
            const uint32_t w = reinterpret_cast<const uint32_t*>(qs)[wrow * (K / 8) + kk / 8];
            row[(size_t)k] = (int8_t)((int)((w >> (4 * (kk % 8))) & 15u) - 8);
          }
        }
        for (int64_t b = 0; b < kn / 32; ++b) dw[(size_t)b] = half_f32(d[wrow * (K / 32) + k0 / 32 + b], scale_dtype);
      };
      for (int64_t j = 0; j < 2 * Ish; ++j) {
        const int64_t wrow = e * 2 * I + (j < Ish ? s * Ish + j : I + s * Ish + (j - Ish));
        wire_row(gate_up_qs, gate_up_d, wrow, H, 0, H);
        g.set_row(j, row.data(), dw.data());
      }
      for (int64_t h = 0; h < H; ++h) {
        wire_row(down_qs, down_d, e * H + h, I, s * Ish, Ish);
        dn.set_row(h, row.data(), dw.data());
      }
    });
  }
  loaded_ = true;
}

// Online Q8_0 of one projection (quantize_weight_only, Int8-gemm/q8_gemm.cpp:
// 197-260: q from the fp32 1/d, d stored as fp16) into the shards' panels.
void Engine::quantize_and_store(int64_t e, int proj, const float* w) {
  const int64_t H = H_, I = I_, Ish = I / tp_;
  const int64_t N = proj == 2 ? H : I, K = proj == 2 ? I : H;
  std::vector<int8_t> q((size_t)K);
  std::vector<float> dw((size_t)(K / 32));
  for (int s = 0; s < tp_; ++s) {
    Shard& sh = shards_[(size_t)s];
    if (sh.w13.empty()) {
      sh.w13.assign((size_t)E_, PackedMat());
      sh.w2.assign((size_t)E_, PackedMat());
    }
    PackedMat& g = sh.w13[(size_t)e];
    PackedMat& dn = sh.w2[(size_t)e];
    if (g.qs.empty()) {
      g.init(0, 2 * Ish, H);
      dn.init(0, H, Ish);
    }
  }
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t b = 0; b < K / 32; ++b) dw[(size_t)b] = f16_f32(f32_f16(quant_block(w + n * K + 32 * b, q.data() + 32 * b)));
    if (proj == 2) {
      for (int s = 0; s < tp_; ++s) shards_[(size_t)s].w2[(size_t)e].set_row(n, q.data() + s * Ish, dw.data() + s * Ish / 32);
    } else {
      const int s = (int)(n / Ish), j = (int)(n % Ish);
      shards_[(size_t)s].w13[(size_t)e].set_row(proj == 0 ? j : Ish + j, q.data(), dw.data());
    }
  }
  loaded_ = true;
}

int Engine::forward(const uint16_t* x, uint16_t* y, const float* topk_w, const int32_t* topk_ids, int64_t T,
                    int64_t K, int act_dtype, float* y_f32) {
  std::lock_guard<std::mutex> lk(call_mu_);
  const auto t0 = std::chrono::steady_clock::now();
  const int64_t E = E_, H = H_, Ish = I_ / tp_, HB = H / 32, IB = Ish / 32;
  // routing: stable counting sort by expert (Int8-gemm/moe_common.cpp:146-216)
  std::vector<int32_t> counts((size_t)E, 0), starts((size_t)E + 1, 0), scat((size_t)(T * K), -1);
  for (int64_t i = 0; i < T * K; ++i) {
    const int32_t e = topk_ids[i];
    if (e >= 0 && e < E) ++counts[(size_t)e];
  }
  for (int64_t e = 0; e < E; ++e) starts[(size_t)e + 1] = starts[(size_t)e] + counts[(size_t)e];
  const int64_t total = starts[(size_t)E];
  std::vector<int32_t> tok((size_t)std::max<int64_t>(total, 1)), fill(starts.begin(), starts.end() - 1);
  for (int64_t i = 0; i < T * K; ++i) {
    const int32_t e = topk_ids[i];
    if (e < 0 || e >= E) continue;
    const int32_t pos = fill[(size_t)e]++;
    tok[(size_t)pos] = (int32_t)(i / K);
    scat[(size_t)i] = pos;
  }
  if (total == 0) {   // Int8-gemm/q8_gemm.cpp:328-333
    if (y_f32) memset(y_f32, 0, sizeof(float) * (size_t)(T * H));
    else memset(y, 0, sizeof(uint16_t) * (size_t)(T * H));
    last_ms_ = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return 0;
  }
  // tasks of M_BLOCK rows (Int8-gemm/q8_gemm.cpp:335-347)
  struct Task { int e, count, start; };
  std::vector<Task> tasks;
  for (int64_t e = 0; e < E; ++e)
    for (int off = 0; off < counts[(size_t)e]; off += kMBlock)
      tasks.push_back({(int)e, std::min(kMBlock, counts[(size_t)e] - off), starts[(size_t)e] + off});
  const int64_t ntasks = (int64_t)tasks.size();

  // tokens with a routed pair: the only rows Stage A needs (a token with no
  // valid id gets a zero row in Stage C1 without reading its hidden row)
  std::vector<int32_t> live;
  for (int64_t t = 0; t < T; ++t)
    for (int64_t k = 0; k < K; ++k)
      if (scat[(size_t)(t * K + k)] >= 0) {
        live.push_back((int32_t)t);
        break;
      }
  const int64_t nlive = (int64_t)live.size();
  grow(part_, (size_t)(tp_ * T * H));
  float* const part = part_.data();
  // the row quantizers' vector form needs AVX2, FMA and F16C, which a vector
  // dot-product ISA alone does not imply
  const bool simd = isa_ != Isa::kScalar && host_simd();
  // per-token stages of a few tokens run on the calling thread: waking the
  // pool costs more than the work
  auto per_token = [&](NodePool& pool, int64_t n, const std::function<void(int64_t)>& f) {
    if (n * H <= (int64_t)16 * 2048) {
      for (int64_t i = 0; i < n; ++i) f(i);
    } else {
      pool.run(n, f);
    }
  };
  auto run_shard = [&](int s) {
    NodePool& pool = *pools_[(size_t)s];
    const Shard& sh = shards_[(size_t)s];
    Scratch& sc = scratch_[(size_t)s];
    // Stage A (Int8-gemm/q8_gemm.cpp:360-377), this shard's replica
    grow(sc.xq, (size_t)(T * H));
    grow(sc.xb, (size_t)(T * H));
    grow(sc.xd, (size_t)(T * HB));
    grow(sc.xs, (size_t)(T * HB));
    per_token(pool, nlive, [&](int64_t i) {
      const int64_t t = live[(size_t)i];
      quant_hidden_row(simd, x + t * H, H, act_dtype, sc.xq.data() + t * H, sc.xb.data() + t * H,
                       sc.xd.data() + t * HB, sc.xs.data() + t * HB);
    });
    // every routed row gathered in sorted order once, into the shard's
    // persistent buffers (pack_A_q8_0_from_quantized_indirect,
    // Int8-gemm/gemm_kernels.cpp:427-464): a task's rows are then one
    // contiguous block, and no task allocates
    grow(sc.ga, (size_t)(total * H));
    grow(sc.gab, (size_t)(total * H));
    grow(sc.gad, (size_t)(total * HB));
    grow(sc.gas, (size_t)(total * HB));
    per_token(pool, total, [&](int64_t r) {
      const int64_t t = tok[(size_t)r];
      memcpy(&sc.ga[(size_t)(r * H)], &sc.xq[(size_t)(t * H)], (size_t)H);
      memcpy(&sc.gab[(size_t)(r * H)], &sc.xb[(size_t)(t * H)], (size_t)H);
      memcpy(&sc.gad[(size_t)(r * HB)], &sc.xd[(size_t)(t * HB)], sizeof(float) * (size_t)HB);
      memcpy(&sc.gas[(size_t)(r * HB)], &sc.xs[(size_t)(t * HB)], sizeof(int32_t) * (size_t)HB);
    });
    auto task_rows = [&](const Task& tk) {
      return ARows{sc.ga.data() + (size_t)tk.start * H, sc.gab.data() + (size_t)tk.start * H,
                   sc.gad.data() + (size_t)tk.start * HB, sc.gas.data() + (size_t)tk.start * HB, H};
    };
    // gate_up outputs [total][2 * Ish], the intermediate's Q8_0 [total][Ish]
    // (SiLU(gate) * up, Int8-gemm/vec_simd.h:36-64, then pack_A_q8_0,
    // Int8-gemm/gemm_kernels.cpp:394-425), expert outputs [total][H]
    grow(sc.inter, (size_t)(total * 2 * Ish));
    grow(sc.aq, (size_t)(total * Ish));
    grow(sc.ab, (size_t)(total * Ish));
    grow(sc.ad, (size_t)(total * IB));
    grow(sc.as, (size_t)(total * IB));
    grow(sc.eout, (size_t)(total * H));
    float* const inter = sc.inter.data();
    float* const eout = sc.eout.data();
    // activation of rows [start, start + count), intermediate columns [c0, c1)
    auto activate = [&](const Task& tk, int64_t c0, int64_t c1) {
      for (int m = 0; m < tk.count; ++m) {
        const int64_t r = tk.start + m;
        const float* in = inter + r * 2 * Ish;
        quant_act_row(simd, in + c0, in + Ish + c0, c1 - c0, sc.aq.data() + r * Ish + c0, sc.ab.data() + r * Ish + c0,
                      sc.ad.data() + r * IB + c0 / 32, sc.as.data() + r * IB + c0 / 32);
      }
    };
    auto down_rows = [&](const Task& tk) {
      return ARows{sc.aq.data() + (size_t)tk.start * Ish, sc.ab.data() + (size_t)tk.start * Ish,
                   sc.ad.data() + (size_t)tk.start * IB, sc.as.data() + (size_t)tk.start * IB, Ish};
    };
    // P parts per task.  split_max_ 2 is the reference's rule
    // (Int8-gemm/q8_gemm.cpp:379-591): two parts per task when
    // tasks * 2 <= threads, else one.  A larger split_max_ cuts tasks into
    // about 4 parts per thread in all (at most split_max_ and one Q8_0 block
    // of intermediate columns each), which the dynamic hand-out balances.
    // Part p of gate_up takes the intermediate columns [c0, c1) (whole Q8_0
    // blocks): gate rows c0..c1 and up rows Ish + c0..c1, then activates and
    // quantizes those columns for the task's rows, so each intermediate value
    // is activated once.  Part p of down takes a range of whole 16-row panels.
    // Every output row is computed the same way whatever the split.
    int P = ntasks * 2 <= pool.size() ? 2 : 1;
    if (split_max_ > 2) {
      const int64_t want = (4 * (int64_t)pool.size() + ntasks - 1) / ntasks;
      P = (int)std::max<int64_t>(1, std::min<int64_t>(want, std::min<int64_t>(split_max_, Ish / 32)));
    }
    auto part_range = [&](int64_t units, int64_t unit, int part, int64_t& a, int64_t& b) {
      a = units * part / P * unit;
      b = units * (part + 1) / P * unit;
    };
    if (P >= 2) {
      pool.run(P * ntasks, [&](int64_t i) {
        const Task& tk = tasks[(size_t)(i / P)];
        int64_t c0, c1;
        part_range(Ish / 32, 32, (int)(i % P), c0, c1);
        if (c0 == c1) return;
        const ARows A = task_rows(tk);
        float* in = inter + (size_t)tk.start * 2 * Ish;
        gemm_rows(isa_, sh.w13[(size_t)tk.e], A, tk.count, c0, c1, in, 2 * Ish);
        gemm_rows(isa_, sh.w13[(size_t)tk.e], A, tk.count, Ish + c0, Ish + c1, in, 2 * Ish);
        activate(tk, c0, c1);
      });
      pool.run(P * ntasks, [&](int64_t i) {
        const Task& tk = tasks[(size_t)(i / P)];
        int64_t h0, h1;
        part_range(H / kNR, kNR, (int)(i % P), h0, h1);
        if (h0 == h1) return;
        gemm_rows(isa_, sh.w2[(size_t)tk.e], down_rows(tk), tk.count, h0, h1, eout + (size_t)tk.start * H, H);
      });
    } else {
      pool.run(ntasks, [&](int64_t ti) {
        const Task& tk = tasks[(size_t)ti];
        const ARows A1 = task_rows(tk);
        gemm_rows(isa_, sh.w13[(size_t)tk.e], A1, tk.count, 0, 2 * Ish, inter + (size_t)tk.start * 2 * Ish, 2 * Ish);
        activate(tk, 0, Ish);
        gemm_rows(isa_, sh.w2[(size_t)tk.e], down_rows(tk), tk.count, 0, H, eout + (size_t)tk.start * H, H);
      });
    }
    // Stage C1 (Int8-gemm/q8_gemm.cpp:593-613), in column chunks of 512 when
    // there are more than 16 routed rows to add
    float* yp = part + (size_t)s * T * H;
    const int64_t chunk = std::min<int64_t>(H, 512), nchunks = (H + chunk - 1) / chunk;
    auto combine = [&](int64_t i) {
      const int64_t t = i / nchunks, j0 = i % nchunks * chunk, n = std::min(chunk, H - j0);
      float* acc = yp + t * H + j0;
      for (int64_t j = 0; j < n; ++j) acc[j] = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const int32_t src = scat[(size_t)(t * K + k)];
        if (src < 0) continue;
        axpy_row(simd, topk_w[t * K + k], eout + (size_t)src * H + j0, acc, n);
      }
    };
    if (total <= 16) {
      for (int64_t i = 0; i < T * nchunks; ++i) combine(i);
    } else {
      pool.run(T * nchunks, combine);
    }
  };
  if (tp_ == 1) {
    run_shard(0);
  } else {
    // a shard's exception is carried to this thread after every launcher
    // has been joined
    std::vector<std::thread> launch;
    std::vector<std::exception_ptr> errs((size_t)tp_);
    try {
      for (int s = 0; s < tp_; ++s)
        launch.emplace_back([&, s] {
          try {
            pools_[(size_t)s]->pin(0);   // the shard's launcher works on its node too
            run_shard(s);
          } catch (...) {
            errs[(size_t)s] = std::current_exception();
          }
        });
    } catch (...) {
      for (auto& th : launch) th.join();
      throw;
    }
    for (auto& th : launch) th.join();
    for (auto& e : errs)
      if (e) std::rethrow_exception(e);
  }
  // Stage C2 (Int8-gemm/q8_gemm.cpp:621-641): shard order, then the cast
  per_token(*pools_[0], T, [&](int64_t t) {
    for (int64_t j = 0; j < H; ++j) {
      float acc = part[(size_t)(t * H + j)];
      for (int s = 1; s < tp_; ++s) acc = acc + part[(size_t)(s * T * H + t * H + j)];
      if (y_f32) y_f32[t * H + j] = acc;
      else y[t * H + j] = f32_half(acc, act_dtype);
    }
  });
  last_ms_ = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  return 0;
}

}  // namespace mimoe_cpu
