// mi_moe_device.hpp -- device-side building blocks shared by the fused-MoE
// kernels (gfx950 / CDNA4, wave64).
//
// All fp32 arithmetic in this library is compiled with contraction off
// (see the pragma in each .hip file); explicit fmaf() is the only FMA.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimoe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kBlock = 256;            // 4 waves per workgroup

// ------------------------------------------------------------ conversions
// floor(i / d) for 0 <= i < 2^21 and d >= 1, given rd = 1.0f / d: (i + 0.5) / d
// lies at least 0.5 / d from an integer, far beyond the rounding of (i + 0.5) * rd.
// Replaces a runtime integer division (a ~15-instruction sequence) in index math.
__device__ __forceinline__ int div_small(int i, float rd) { return (int)(((float)i + 0.5f) * rd); }

__device__ __forceinline__ float bf16_to_f32(uint32_t b) {
  return __uint_as_float((b & 0xffffu) << 16);
}
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
  return (float)v;
}
template <int DT>
__device__ __forceinline__ float to_f32(uint32_t v) {
  return DT == 1 ? bf16_to_f32(v) : f16_to_f32(v);
}
// fp32 -> bf16 / fp16 bits, round to nearest even
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}
template <int DT>
__device__ __forceinline__ uint16_t from_f32(float f) {
  return DT == 1 ? f32_to_bf16(f) : f32_to_f16(f);
}

// exp(x): Cody & Waite (1980) reduction n = rint(x log2 e),
// r = (x - n*C1) - n*C2 with C1 = 355/512, then the degree-7 Taylor series of
// exp(r) in Horner form and a 2^n exponent-field scale.  Same operation
// sequence as the CPU checker so both round identically.
__device__ __forceinline__ float mi_expf(float x) {
  if (x != x) return x;
  if (x > 88.5f) return __uint_as_float(0x7f800000u);
  if (x < -87.0f) return 0.0f;
  const float log2e = 1.44269504088896341f;
  const float C1 = 0.693359375f;
  const float C2 = -2.12194440e-4f;
  float n = __builtin_rintf(x * log2e);
  float r = __builtin_fmaf(-n, C1, x);
  r = __builtin_fmaf(-n, C2, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) { p = p * 2.0f; ni -= 1; }
  if (ni < -126) { p = p * __uint_as_float(0x00800000u); ni += 126; }
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

// up * (g / (1 + exp(-g)))  -- the SiLU*mul of the reference (vec_simd.h:36-64)
__device__ __forceinline__ float silu_mul(float g, float up) {
  const float eg = mi_expf(-g);
  const float denom = 1.0f + eg;
  const float sig = g / denom;
  return up * sig;
}

// The same with the hardware exponential and reciprocal (v_exp_f32,
// v_rcp_f32: about 1 ulp each), for the W4A16 path whose output is rounded to
// 16 bits; the Q8_0 path keeps silu_mul, which its CPU checker reproduces.
__device__ __forceinline__ float silu_mul_fast(float g, float up) {
  const float eg = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return up * (g * __builtin_amdgcn_rcpf(1.0f + eg));
}

// ------------------------------------------------------------ Q8_0 block
// amax over 32 values, d = amax/127, id = 1/d, q = sat8(RNE(x*id)).
__device__ __forceinline__ int8_t q8_round(float v) {
  if (v != v) return 0;
  float r = __builtin_rintf(v);
  r = r > 127.0f ? 127.0f : r;
  r = r < -128.0f ? -128.0f : r;
  return (int8_t)(int)r;
}

// Scale of a Q8_0 block from its amax: d = amax / 127, *id = 1 / d (0 when
// d == 0).  Every Q8_0 quantization in this library goes through it.
__device__ __forceinline__ float q8_block_scale(float amax, float* id) {
  const float d = amax / 127.0f;
  *id = (d != 0.0f) ? 1.0f / d : 0.0f;
  return d;
}

// Q8_0 quantization of 32 fp32 values (quantize_block_q8_0,
// Int8-gemm/gemm_kernels.cpp:25-58): returns d, writes the 32 bytes to dst
// (16-byte aligned) and the sum of the q values to *qsum.  The one block
// quantizer of the activation paths: the standalone Stage-A kernel, the
// decode kernels' Stage A and the online weight quantization call it.
__device__ __forceinline__ float quant_block_q8_0(const float (&v)[32], int8_t* dst, int* qsum) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const float av = __builtin_fabsf(v[j]);
    amax = av > amax ? av : amax;
  }
  float id;
  const float d = q8_block_scale(amax, &id);
  int s = 0;
  uint32_t packed[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int8_t q = q8_round(v[4 * w + h] * id);
      s += q;
      word |= ((uint32_t)(uint8_t)q) << (8 * h);
    }
    packed[w] = word;
  }
  u32x4_t* o = reinterpret_cast<u32x4_t*>(dst);
  o[0] = u32x4_t{packed[0], packed[1], packed[2], packed[3]};
  o[1] = u32x4_t{packed[4], packed[5], packed[6], packed[7]};
  *qsum = s;
  return d;
}

// ------------------------------------------------------------ routing
// Stable counting sort of the routed (t,k) pairs by expert, the semantics of
// preprocess_moe_routing (Int8-gemm/moe_common.cpp:146-216): counts, exclusive
// starts, pair index i = t*K+k per expert-sorted position (the reference's
// token_map entry {t,k}), and scatter[i] = position or -1 for an id outside
// [0,E).  Also emits the ascending list of active
// experts.  Whole-workgroup routine (blockDim.x == 256), all arrays in LDS.
// Ranks are computed by wave 0 in 64-id chunks with a ballot match.
__device__ inline void route_lds(const int32_t* __restrict__ ids, int n, int K,
                                 int E, int* counts, int* starts, int* active,
                                 int* tok, int* scat, int* s_U) {
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += blockDim.x) counts[e] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += blockDim.x) {
    const int e = ids[i];
    scat[i] = e;   // the ranking below reads the ids from LDS (no second global read)
    if ((unsigned)e < (unsigned)E) atomicAdd(&counts[e], 1);
  }
  __syncthreads();
  if (tid < kWave) {
    const int lane = tid;
    const int per = (E + kWave - 1) / kWave;
    const int base = lane * per;
    int s = 0, a = 0;
    for (int i = 0; i < per; ++i) {
      const int e = base + i;
      if (e < E) { const int c = counts[e]; s += c; a += (c > 0); }
    }
    int sinc = s, ainc = a;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int v = __shfl_up(sinc, off);
      const int w = __shfl_up(ainc, off);
      if (lane >= off) { sinc += v; ainc += w; }
    }
    int sx = sinc - s, ax = ainc - a;
    for (int i = 0; i < per; ++i) {
      const int e = base + i;
      if (e < E) {
        const int c = counts[e];
        starts[e] = sx;
        if (c > 0) active[ax++] = e;
        sx += c;
        counts[e] = 0;  // becomes the running rank counter below
      }
    }
    if (lane == kWave - 1) { starts[E] = sinc; *s_U = ainc; }
    __builtin_amdgcn_wave_barrier();
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    for (int b0 = 0; b0 < n; b0 += kWave) {
      const int i = b0 + lane;
      const int e = (i < n) ? scat[i] : -1;
      const bool valid = (i < n) && ((unsigned)e < (unsigned)E);
      uint64_t m = __ballot(valid);
      for (int bit = 0; bit < nbits; ++bit) {
        const bool on = valid && ((e >> bit) & 1);
        const uint64_t bb = __ballot(on);
        m &= ((e >> bit) & 1) ? bb : ~bb;
      }
      int add = 0;
      if (valid) {
        const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
        const int pos = starts[e] + counts[e] + __popcll(m & lt);
        scat[i] = pos;
        tok[pos] = i;
        if (__ffsll((long long)m) - 1 == lane) add = __popcll(m);
      } else if (i < n) {
        scat[i] = -1;
      }
      __builtin_amdgcn_wave_barrier();
      if (add) counts[e] += add;
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();
}

}  // namespace mimoe
