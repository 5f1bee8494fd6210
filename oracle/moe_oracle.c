/*
 * moe_oracle.c -- CPU restatement of the reference fused-MoE algorithm.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  Compiled with
 * -ffp-contract=off: every fp32 rounding below is explicit.  See
 * moe_oracle.h for the function-by-function reference citations.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* Conversions                                                         */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

float orc_f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31;
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) {
    if (m == 0) return u2f(s);
    /* subnormal: value = m * 2^-24, exact in fp32 */
    float v = (float)m * u2f(0x33800000u); /* 2^-24 */
    return (h >> 15) ? -v : v;
  }
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  return u2f(s | ((e + 112) << 23) | (m << 13));
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb; /* round to nearest, ties to even */
  return (uint16_t)(u >> 16);
}

uint16_t orc_f32_to_f16(float f) {
  /* IEEE binary32 -> binary16, round to nearest even, with subnormals. */
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t ax = u & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal */
    /* value / 2^-24 rounded to nearest even integer */
    float a = u2f(ax);
    float scaled = a * u2f(0x4b800000u); /* * 2^24, exact */
    float r = rintf(scaled);             /* default rounding mode: RNE */
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t e = (ax >> 23) - 112;
  uint32_t m = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry may bump exponent: correct */
  return (uint16_t)(sign | h);
}

static inline float act_to_f32(uint16_t v, int dtype) {
  return dtype == 1 ? orc_bf16_to_f32(v) : orc_f16_to_f32(v);
}
static inline uint16_t f32_to_act(float v, int dtype) {
  return dtype == 1 ? orc_f32_to_bf16(v) : orc_f32_to_f16(v);
}

/* ------------------------------------------------------------------ */
/* exp: Cody & Waite (1980) argument reduction, Taylor polynomial      */
/* ------------------------------------------------------------------ */
/* n = rint(x * log2(e)); r = (x - n*C1) - n*C2 with the Cody-Waite split of
 * ln 2 (C1 = 355/512 exactly, C2 = ln2 - C1).  exp(r) on |r| <= ~0.347 by the
 * degree-7 Taylor series 1 + r + r^2/2! + ... + r^7/7! in Horner form, then
 * scaled by 2^n through the exponent field.  Inputs past the fp32 range
 * saturate to +inf / 0. */
float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.5f) return u2f(0x7f800000u);
  if (x < -87.0f) return 0.0f;
  const float log2e = 1.44269504088896341f;
  const float C1 = 0.693359375f;
  const float C2 = -2.12194440e-4f;
  float n = rintf(x * log2e);
  float r = fmaf(-n, C1, x);
  r = fmaf(-n, C2, r);
  float p = 1.98412698412698413e-4f;          /* 1/7! */
  p = fmaf(p, r, 1.38888888888888889e-3f);    /* 1/6! */
  p = fmaf(p, r, 8.33333333333333333e-3f);    /* 1/5! */
  p = fmaf(p, r, 4.16666666666666667e-2f);    /* 1/4! */
  p = fmaf(p, r, 1.66666666666666667e-1f);    /* 1/3! */
  p = fmaf(p, r, 0.5f);                       /* 1/2! */
  p = fmaf(p, r, 1.0f);                       /* 1/1! */
  p = fmaf(p, r, 1.0f);                       /* 1/0! */
  int ni = (int)n; /* in [-126, 128] for the accepted range */
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  if (ni < -126) { p = p * u2f(0x00800000u) /* 2^-126 */; ni += 126; }
  return p * u2f((uint32_t)(ni + 127) << 23);
}

/* ------------------------------------------------------------------ */
/* Q8_0 block quantization -- Int8-gemm/gemm_kernels.cpp:25-58          */
/* ------------------------------------------------------------------ */
static inline int8_t sat_rne_i8(float v) {
  /* vcvtnq_s32_f32 (RNE, NaN -> 0, saturating), then vqmovn s32->s16->s8 */
  if (v != v) return 0;
  if (v >= 2147483520.0f) return 127;
  if (v <= -2147483648.0f) return -128;
  long r = lrintf(v); /* default rounding mode: nearest-even */
  if (r > 127) r = 127;
  if (r < -128) r = -128;
  return (int8_t)r;
}

static float block_q8_0_core(const float* x, int8_t* qs) {
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) {
    float a = fabsf(x[j]);
    if (a > amax) amax = a;
  }
  const float d = amax / 127.0f;
  const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  for (int j = 0; j < 32; ++j) qs[j] = sat_rne_i8(x[j] * id);
  return d;
}

void orc_quantize_block_q8_0(const float* x, float* d, int8_t* qs) {
  *d = block_q8_0_core(x, qs);
}

void orc_quantize_block_q8_0_f16d(const float* x, uint16_t* d_f16, int8_t* qs) {
  *d_f16 = orc_f32_to_f16(block_q8_0_core(x, qs));
}

void orc_quantize_act_q8_0(const uint16_t* x, int act_dtype, int64_t T,
                           int64_t H, int8_t* qs, float* d) {
  const int64_t nb = H / 32;
  float buf[32];
  for (int64_t t = 0; t < T; ++t)
    for (int64_t b = 0; b < nb; ++b) {
      for (int j = 0; j < 32; ++j) buf[j] = act_to_f32(x[t * H + b * 32 + j], act_dtype);
      orc_quantize_block_q8_0(buf, &d[t * nb + b], &qs[t * H + b * 32]);
    }
}

void orc_quantize_weight_q8_0(const float* w, int64_t N, int64_t K, int8_t* qs,
                              uint16_t* d_f16) {
  const int64_t nb = K / 32;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t b = 0; b < nb; ++b)
      orc_quantize_block_q8_0_f16d(w + n * K + b * 32, &d_f16[n * nb + b],
                                   qs + n * K + b * 32);
}

/* ------------------------------------------------------------------ */
/* Routing -- Int8-gemm/moe_common.cpp:146-216                          */
/* ------------------------------------------------------------------ */
int64_t orc_route(const int32_t* ids, int64_t T, int64_t K, int64_t E,
                  int32_t* counts, int32_t* starts, int32_t* token_map,
                  int32_t* scatter, int restrict_topk) {
  if (restrict_topk && !(K == 1 || K == 8 || K == 10)) return -1;
  for (int64_t e = 0; e < E; ++e) counts[e] = 0;
  for (int64_t i = 0; i < T * K; ++i) {
    int32_t e = ids[i];
    if (e >= 0 && e < E) counts[e]++;
  }
  starts[0] = 0;
  for (int64_t e = 0; e < E; ++e) starts[e + 1] = starts[e] + counts[e];
  int32_t* cur = (int32_t*)calloc((size_t)E, sizeof(int32_t));
  for (int64_t t = 0; t < T; ++t)
    for (int64_t k = 0; k < K; ++k) {
      int32_t e = ids[t * K + k];
      if (e >= 0 && e < E) {
        int32_t pos = starts[e] + cur[e]++;
        token_map[2 * pos] = (int32_t)t;
        token_map[2 * pos + 1] = (int32_t)k;
        scatter[t * K + k] = pos;
      } else {
        scatter[t * K + k] = -1;
      }
    }
  free(cur);
  return starts[E];
}

/* ------------------------------------------------------------------ */
/* Weight element access in the caller wire layout                    */
/* ------------------------------------------------------------------ */
/* Q4_0: element k of a row sits in u32[k/8] bits 4(k%8).. (value nibble-8);
 * Int8-gemm/gemm_kernels.cpp:542 reads sequential nibbles, and the generator
 * Int8-gemm/test/fused_moe_cpu_int4.py:58-71 decodes them in that order. */
static inline int wq(int qt, const void* w, int64_t row, int64_t K, int64_t k) {
  if (qt == 0) return ((const int8_t*)w)[row * K + k];
  uint32_t word = ((const uint32_t*)w)[row * (K / 8) + k / 8];
  return (int)((word >> (4 * (k % 8))) & 0xfu) - 8;
}

void orc_block_dots(int qt, const int8_t* a_qs, int64_t M, const void* w_qs,
                    int64_t N, int64_t K, int32_t* isum) {
  const int64_t nb = K / 32;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n)
      for (int64_t b = 0; b < nb; ++b) {
        int32_t s = 0;
        for (int i = 0; i < 32; ++i)
          s += (int32_t)a_qs[m * K + b * 32 + i] * wq(qt, w_qs, n, K, b * 32 + i);
        isum[(m * N + n) * nb + b] = s;
      }
}

/* One output of the block GEMM: c = sum_kb ((float)isum * dw) * da in kb
 * order (Int8-gemm/gemm_kernels.cpp:156-179 and 335-358: vmulq then
 * vmlaq_laneq; the fp32 value is kept in the order the micro-kernel walks
 * the k blocks). */
static float gemm_row_dot(int qt, const int8_t* a_qs, const float* a_d,
                          const void* w, const uint16_t* w_d, int scale_dtype,
                          int64_t row, int64_t K, int64_t kb0, int64_t nkb) {
  float c = 0.0f;
  const int64_t nb_row = K / 32;
  for (int64_t b = kb0; b < kb0 + nkb; ++b) {
    int32_t s = 0;
    for (int i = 0; i < 32; ++i)
      s += (int32_t)a_qs[b * 32 + i] * wq(qt, w, row, K, b * 32 + i);
    const float dw = act_to_f32(w_d[row * nb_row + b], scale_dtype);
    const float t1 = (float)s * dw;
    const float t2 = t1 * a_d[b];
    c = c + t2;
  }
  return c;
}

/* vec_simd.h:36-64: row[j] = up[j] * (g / (1 + exp(-g))) */
void orc_silu_and_mul(float* row, int64_t ish) {
  for (int64_t j = 0; j < ish; ++j) {
    const float g = row[j];
    const float eg = orc_expf(-g);
    const float denom = 1.0f + eg;
    const float sig = g / denom;
    row[j] = row[ish + j] * sig;
  }
}

/* ------------------------------------------------------------------ */
/* Fused forward, Q8_0 / Q4_0 -- Int8-gemm/q8_gemm.cpp:276-646          */
/* ------------------------------------------------------------------ */
int orc_moe_forward_q(int qt, int act_dtype, int scale_dtype,
                      const uint16_t* x, uint16_t* y, float* y_f32,
                      const float* topk_w, const int32_t* topk_ids,
                      const void* gate_up_qs, const uint16_t* gate_up_d,
                      const void* down_qs, const uint16_t* down_d,
                      int64_t T, int64_t H, int64_t E, int64_t I, int64_t tp,
                      int64_t K) {
  if (tp < 1 || H % 32 || I % tp || (I / tp) % 32) return -1;
  const int64_t Ish = I / tp;
  const int64_t n_ids = T * K;
  int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int32_t* starts = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
  int32_t* tmap = (int32_t*)malloc(sizeof(int32_t) * (size_t)(2 * n_ids + 2));
  int32_t* scat = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_ids + 1));
  int64_t total = orc_route(topk_ids, T, K, E, counts, starts, tmap, scat, 1);
  if (total < 0) { free(counts); free(starts); free(tmap); free(scat); return -1; }
  if (total == 0) { /* q8_gemm.cpp:328-333 */
    for (int64_t i = 0; i < T * H; ++i) { y[i] = 0; if (y_f32) y_f32[i] = 0.0f; }
    free(counts); free(starts); free(tmap); free(scat);
    return 0;
  }
  /* Stage A (q8_gemm.cpp:360-377) */
  int8_t* x_qs = (int8_t*)malloc((size_t)(T * H));
  float* x_d = (float*)malloc(sizeof(float) * (size_t)(T * H / 32));
  orc_quantize_act_q8_0(x, act_dtype, T, H, x_qs, x_d);

  float* y_part = (float*)calloc((size_t)(tp * T * H), sizeof(float));
  float* expert_out = (float*)malloc(sizeof(float) * (size_t)(total * H));
  float* inter = (float*)malloc(sizeof(float) * (size_t)(2 * Ish));
  float* act = (float*)malloc(sizeof(float) * (size_t)Ish);
  int8_t* a2_qs = (int8_t*)malloc((size_t)Ish);
  float* a2_d = (float*)malloc(sizeof(float) * (size_t)(Ish / 32));
  const int64_t wdiv = (qt == 1) ? 8 : 1;
  const int64_t Hb = H / 32, Ib = I / 32, Ishb = Ish / 32;

  for (int64_t s = 0; s < tp; ++s) {
    /* Stage B: every routed row, expert-sorted (tasks of M_BLOCK=32 rows do
     * not change the per-row arithmetic). */
    for (int64_t pos = 0; pos < total; ++pos) {
      const int64_t t = tmap[2 * pos];
      int64_t e = 0;
      while (starts[e + 1] <= pos) ++e;
      const int8_t* xq = x_qs + t * H;
      const float* xd = x_d + t * Hb;
      /* GEMM1 on the tp shard: rows [gate shard | up shard]
       * (moe_infer.cpp:143-176 / 218-250) */
      for (int64_t half = 0; half < 2; ++half)
        for (int64_t j = 0; j < Ish; ++j) {
          const int64_t row = e * 2 * I + half * I + s * Ish + j; /* wire row */
          const void* wbase = qt == 1 ? (const void*)((const uint32_t*)gate_up_qs)
                                      : (const void*)((const int8_t*)gate_up_qs);
          inter[half * Ish + j] =
              gemm_row_dot(qt, xq, xd, wbase, gate_up_d, scale_dtype, row, H, 0, Hb);
        }
      orc_silu_and_mul(inter, Ish);
      for (int64_t b = 0; b < Ishb; ++b)
        orc_quantize_block_q8_0(inter + b * 32, &a2_d[b], a2_qs + b * 32);
      /* GEMM2 on the shard: down columns [s*Ish, (s+1)*Ish) (moe_infer.cpp:178-205) */
      for (int64_t h = 0; h < H; ++h) {
        float c = 0.0f;
        const int64_t row = e * H + h;
        for (int64_t b = 0; b < Ishb; ++b) {
          const int64_t kb = s * Ishb + b;
          int32_t acc = 0;
          for (int i = 0; i < 32; ++i)
            acc += (int32_t)a2_qs[b * 32 + i] * wq(qt, down_qs, row, I, kb * 32 + i);
          const float dw = act_to_f32(down_d[row * Ib + kb], scale_dtype);
          const float t1 = (float)acc * dw;
          const float t2 = t1 * a2_d[b];
          c = c + t2;
        }
        expert_out[pos * H + h] = c;
      }
      (void)wdiv;
    }
    /* Stage C1 (q8_gemm.cpp:593-613) */
    float* yp = y_part + s * T * H;
    for (int64_t t = 0; t < T; ++t)
      for (int64_t k = 0; k < K; ++k) {
        const int32_t src = scat[t * K + k];
        if (src == -1) continue;
        const float w = topk_w[t * K + k];
        for (int64_t j = 0; j < H; ++j) {
          const float prod = w * expert_out[(int64_t)src * H + j];
          yp[t * H + j] = yp[t * H + j] + prod;
        }
      }
  }
  /* Stage C2 (q8_gemm.cpp:621-641) */
  for (int64_t t = 0; t < T; ++t)
    for (int64_t j = 0; j < H; ++j) {
      float acc = y_part[t * H + j];
      for (int64_t s = 1; s < tp; ++s) acc = acc + y_part[s * T * H + t * H + j];
      if (y_f32) y_f32[t * H + j] = acc;
      y[t * H + j] = f32_to_act(acc, act_dtype);
    }
  free(x_qs); free(x_d); free(y_part); free(expert_out); free(inter); free(act);
  free(a2_qs); free(a2_d); free(counts); free(starts); free(tmap); free(scat);
  return 0;
}

/* ------------------------------------------------------------------ */
/* W4A16 (AWQ-style) -- build-defined wire format                      */
/* ------------------------------------------------------------------ */
static const int AWQ_INV[8] = {0, 4, 1, 5, 2, 6, 3, 7}; /* column%8 -> slot */

static inline int awq_nib(const int32_t* packed, int64_t ncols, int64_t r, int64_t c) {
  uint32_t word = (uint32_t)packed[r * (ncols / 8) + c / 8];
  return (int)((word >> (4 * AWQ_INV[c % 8])) & 0xfu);
}

void orc_awq_dequant(const int32_t* qweight, const int32_t* qzeros,
                     const uint16_t* scales, int scale_dtype, int64_t K,
                     int64_t N, int64_t group, float* w) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      const int64_t g = k / group;
      const int q = awq_nib(qweight, N, k, n);
      const int z = awq_nib(qzeros, N, g, n);
      const float s = act_to_f32(scales[g * N + n], scale_dtype);
      w[n * K + k] = (float)(q - z) * s;
    }
}

int orc_moe_forward_w4a16(int act_dtype, int scale_dtype, const uint16_t* x,
                          uint16_t* y, float* y_f32, const float* topk_w,
                          const int32_t* topk_ids, const int32_t* w13_q,
                          const int32_t* w13_z, const uint16_t* w13_s,
                          const int32_t* w2_q, const int32_t* w2_z,
                          const uint16_t* w2_s, int64_t T, int64_t H,
                          int64_t E, int64_t I, int64_t K, int64_t group,
                          int nthreads) {
  if (group <= 0 || H % group || I % group || H % 8 || I % 8) return -1;
  (void)nthreads;
  const int64_t n_ids = T * K;
  int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int32_t* starts = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
  int32_t* tmap = (int32_t*)malloc(sizeof(int32_t) * (size_t)(2 * n_ids + 2));
  int32_t* scat = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_ids + 1));
  int64_t total = orc_route(topk_ids, T, K, E, counts, starts, tmap, scat, 0);
  float* xf = (float*)malloc(sizeof(float) * (size_t)(T * H));
  for (int64_t i = 0; i < T * H; ++i) xf[i] = act_to_f32(x[i], act_dtype);
  float* expert_out = (float*)malloc(sizeof(float) * (size_t)((total > 0 ? total : 1) * H));
  const int64_t N13 = 2 * I;

#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
  for (int64_t pos = 0; pos < total; ++pos) {
    const int64_t t = tmap[2 * pos];
    int64_t e = 0;
    while (starts[e + 1] <= pos) ++e;
    const int32_t* q13 = w13_q + e * H * (N13 / 8);
    const int32_t* z13 = w13_z + e * (H / group) * (N13 / 8);
    const uint16_t* s13 = w13_s + e * (H / group) * N13;
    const int32_t* q2 = w2_q + e * I * (H / 8);
    const int32_t* z2 = w2_z + e * (I / group) * (H / 8);
    const uint16_t* s2 = w2_s + e * (I / group) * H;
    const float* xr = xf + t * H;
    float* gu = (float*)malloc(sizeof(float) * (size_t)N13);
    for (int64_t n = 0; n < N13; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < H; ++k) {
        const int64_t g = k / group;
        const float w = (float)(awq_nib(q13, N13, k, n) - awq_nib(z13, N13, g, n)) *
                        act_to_f32(s13[g * N13 + n], scale_dtype);
        const float p = xr[k] * w;
        acc = acc + p;
      }
      gu[n] = acc;
    }
    orc_silu_and_mul(gu, I);
    for (int64_t h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int64_t k = 0; k < I; ++k) {
        const int64_t g = k / group;
        const float w = (float)(awq_nib(q2, H, k, h) - awq_nib(z2, H, g, h)) *
                        act_to_f32(s2[g * H + h], scale_dtype);
        const float p = gu[k] * w;
        acc = acc + p;
      }
      expert_out[pos * H + h] = acc;
    }
    free(gu);
  }
  for (int64_t t = 0; t < T; ++t)
    for (int64_t j = 0; j < H; ++j) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const int32_t src = scat[t * K + k];
        if (src == -1) continue;
        const float prod = topk_w[t * K + k] * expert_out[(int64_t)src * H + j];
        acc = acc + prod;
      }
      if (y_f32) y_f32[t * H + j] = acc;
      y[t * H + j] = f32_to_act(acc, act_dtype);
    }
  free(counts); free(starts); free(tmap); free(scat); free(xf); free(expert_out);
  return 0;
}

/* ------------------------------------------------------------------ */
/* Router top-k + softmax -- make_topk_from_logits_cpu                  */
/* (Int8-gemm/test/fused_moe_cpu.py:20-37)                              */
/* ------------------------------------------------------------------ */
/* Per token: the K largest of the E fp32 logits in descending order
 * (torch.topk(largest=True, sorted=True); equal logits: the lower expert id
 * first, a rule torch leaves open), then
 *   renormalize: w_k = exp(v_k - v_0) / sum_{j<K} exp(v_j - v_0)   (softmax
 *                of the K values; v_0 is their max), sum in k order;
 *   otherwise:   w_k = exp(v_k - v_0) / sum_{e<E} exp(x_e - v_0)  (softmax
 *                over all E gathered at the ids; v_0 is the max logit),
 *                sum in e order.
 * exp is orc_expf; NaN logits are not supported.  Returns -1 on bad sizes. */
int orc_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t K, int renormalize,
                     int32_t* ids, float* w) {
  if (T < 0 || E < 1 || K < 1 || K > E) return -1;
  unsigned char* taken = (unsigned char*)malloc((size_t)E);
  float* ex = (float*)malloc(sizeof(float) * (size_t)(E > K ? E : K));
  for (int64_t t = 0; t < T; ++t) {
    const float* x = logits + t * E;
    memset(taken, 0, (size_t)E);
    for (int64_t k = 0; k < K; ++k) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || x[e] > x[best]) best = e;   /* strict: ties keep the lower id */
      }
      taken[best] = 1;
      ids[t * K + k] = (int32_t)best;
    }
    const float m = x[ids[t * K]];
    float s = 0.0f;
    if (renormalize) {
      for (int64_t k = 0; k < K; ++k) {
        ex[k] = orc_expf(x[ids[t * K + k]] - m);
        s = s + ex[k];
      }
      for (int64_t k = 0; k < K; ++k) w[t * K + k] = ex[k] / s;
    } else {
      for (int64_t e = 0; e < E; ++e) {
        ex[e] = orc_expf(x[e] - m);
        s = s + ex[e];
      }
      for (int64_t k = 0; k < K; ++k) w[t * K + k] = ex[ids[t * K + k]] / s;
    }
  }
  free(taken);
  free(ex);
  return 0;
}
