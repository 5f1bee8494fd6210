// w4a16.hip -- W4A16 (AWQ-style int4, 16-bit activations) fused MoE layer for
// gfx950.  One launch does routing -> gate_up GEMV -> SiLU*mul -> down GEMV
// -> weighted combine -> cast, the dataflow of moe_forward_ptr_impl
// (Int8-gemm/q8_gemm.cpp:276-646) applied to the W4A16 format of the absent
// NPU grouped_gemv (README.md:19-30).
//
// Device weight layout ("tiles").  A tile is 16 output rows x 128 k (one
// quantization group) = 1 KiB, stored as 64 lanes x 16 bytes so that one
// global_load_dwordx4 per lane fetches it fully coalesced.  Lane l = 16*q + r
// holds row r, k in [32q, 32q+32) of the group as four u32 words; word i
// covers k = 32q + 8i + (0..7) with element 2p at bits 4p and element 2p+1
// at bits 4p+16.  (w >> 4p) & 0x000F000F | magic then yields the two 16-bit
// MFMA operand elements (2p, 2p+1) of v_mfma_f32_16x16x32_{bf16,f16} step i
// as (offset + q) exactly: offset 128 for bf16 (0x4300), 1024 for fp16
// (0x6400).  The offset and the zero point are removed per group with the
// column sums X of the activations (an MFMA against an all-ones operand):
//     y[n] += s[n,g] * (G[n] - (offset + z[n,g]) * X)
// gate_up tiles are ordered [expert][slice j of 16 rows][gate, up][group];
// down tiles [expert][16-row tile][group].  Per-(tile, group) metadata:
// 16 scales (2 B each) and 16 zero nibbles packed as four u16 (rows 4q..4q+3).
//
// Work decomposition: see mi_moe_sched.hpp (phase-1 launch: one workgroup
// per (expert, 16-row slice j of I) computing rows j*16.. of gate and up over
// all of H, the 4 waves splitting the groups, then an LDS reduction, SiLU*mul
// and act[pos][16j..16j+15]; phase-2 launch: one workgroup per (expert, hb)
// computing 64 rows of down (one 16-row tile per wave) over all of I, then
// the counted combine).
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
  static constexpr uint32_t ones = ACT == 1 ? 0x3f803f80u : 0x3c003c00u;
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

__device__ __forceinline__ u32x4_t ldg16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// Per lane: scales and zero-point terms of output rows 4q..4q+3 of a tile
// for one group.
template <int ACT, int SC>
__device__ __forceinline__ void load_meta(const uint16_t* s_base, const uint16_t* z_base,
                                          size_t tg, int q, float (&s)[4], float (&c)[4]) {
  const u32x2_t sv = *reinterpret_cast<const u32x2_t*>(s_base + tg * 16 + 4 * q);
  const uint32_t zv = z_base[tg * 4 + q];
  s[0] = to_f32<SC>(sv.x & 0xffffu);
  s[1] = to_f32<SC>(sv.x >> 16);
  s[2] = to_f32<SC>(sv.y & 0xffffu);
  s[3] = to_f32<SC>(sv.y >> 16);
#pragma unroll
  for (int v = 0; v < 4; ++v) c[v] = W4Consts<ACT>::offset + (float)((zv >> (4 * v)) & 0xfu);
}

// acc += s * (G - c * X), per output row of the lane
__device__ __forceinline__ void fold(f32x4_t& acc, const f32x4_t G, const f32x4_t X,
                                     const float (&s)[4], const float (&c)[4]) {
  acc.x = __builtin_fmaf(s[0], __builtin_fmaf(-c[0], X.x, G.x), acc.x);
  acc.y = __builtin_fmaf(s[1], __builtin_fmaf(-c[1], X.y, G.y), acc.y);
  acc.z = __builtin_fmaf(s[2], __builtin_fmaf(-c[2], X.z, G.z), acc.z);
  acc.w = __builtin_fmaf(s[3], __builtin_fmaf(-c[3], X.w, G.w), acc.w);
}

// ---------------------------------------------------------------- phase 1
template <int ACT, int SC>
__device__ void w4_phase1(const W4Args& a, const RouteView& rv, int ui, int j, float* red) {
  const SchedArgs& c = a.c;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int e = rv.active[ui];
  const int p0 = rv.starts[e], cnt = rv.starts[e + 1] - p0;
  const int G1 = c.H >> 7, NI1 = c.I >> 4;
  const int gpw = G1 >> 2, g0 = wave * gpw;
  const size_t tile_g = ((size_t)e * NI1 + j) * 2, tile_u = tile_g + 1;
  const char* wg_base = (const char*)a.w13 + (tile_g * G1) * 1024 + lane * 16;
  const char* wu_base = (const char*)a.w13 + (tile_u * G1) * 1024 + lane * 16;
  const u32x4_t ones = {W4Consts<ACT>::ones, W4Consts<ACT>::ones, W4Consts<ACT>::ones,
                        W4Consts<ACT>::ones};

  for (int cb0 = 0; cb0 < cnt; cb0 += kColsPerPass) {
    const int nb = min(4, (cnt - cb0 + 15) >> 4);
    int xoff[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int col = cb0 + 16 * b + r;
      xoff[b] = (b < nb && col < cnt) ? rv.tok[p0 + col] * c.H : -1;
    }
    f32x4_t accg[4], accu[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) { accg[b] = f32x4_t{0, 0, 0, 0}; accu[b] = f32x4_t{0, 0, 0, 0}; }

    for (int gc = 0; gc < gpw; gc += 4) {
      u32x4_t wgv[4], wuv[4];
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        if (gc + gi < gpw) {
          wgv[gi] = ldg16(wg_base + (size_t)(g0 + gc + gi) * 1024);
          wuv[gi] = ldg16(wu_base + (size_t)(g0 + gc + gi) * 1024);
        }
      }
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        if (gc + gi >= gpw) break;
        const int g = g0 + gc + gi;
        float sg[4], cg[4], su[4], cu[4];
        load_meta<ACT, SC>(a.w13_s, a.w13_z, tile_g * G1 + g, q, sg, cg);
        load_meta<ACT, SC>(a.w13_s, a.w13_z, tile_u * G1 + g, q, su, cu);
        u32x4_t Ag[4], Au[4];
        Ag[0] = deq4<ACT>(wgv[gi].x); Ag[1] = deq4<ACT>(wgv[gi].y);
        Ag[2] = deq4<ACT>(wgv[gi].z); Ag[3] = deq4<ACT>(wgv[gi].w);
        Au[0] = deq4<ACT>(wuv[gi].x); Au[1] = deq4<ACT>(wuv[gi].y);
        Au[2] = deq4<ACT>(wuv[gi].z); Au[3] = deq4<ACT>(wuv[gi].w);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (b >= nb) break;
          u32x4_t B[4];
          if (xoff[b] >= 0) {
            const uint16_t* xp = c.x + xoff[b] + 128 * g + 32 * q;
#pragma unroll
            for (int i = 0; i < 4; ++i) B[i] = ldg16(xp + 8 * i);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) B[i] = u32x4_t{0, 0, 0, 0};
          }
          f32x4_t X = {0, 0, 0, 0}, Gg = {0, 0, 0, 0}, Gu = {0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            X = mfma16<ACT>(ones, B[i], X);
            Gg = mfma16<ACT>(Ag[i], B[i], Gg);
            Gu = mfma16<ACT>(Au[i], B[i], Gu);
          }
          fold(accg[b], Gg, X, sg, cg);
          fold(accu[b], Gu, X, su, cu);
        }
      }
    }
    // cross-wave reduction of the K split: red[wave][gate/up][b][lane][4]
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b < nb) {
        *reinterpret_cast<f32x4_t*>(red + (((wave * 2 + 0) * 4 + b) * 64 + lane) * 4) = accg[b];
        *reinterpret_cast<f32x4_t*>(red + (((wave * 2 + 1) * 4 + b) * 64 + lane) * 4) = accu[b];
      }
    }
    __syncthreads();
    {
      const int b = tid >> 6;  // one (block, lane) per thread
      if (b < nb) {
        f32x4_t g = *reinterpret_cast<const f32x4_t*>(red + (((0 * 2 + 0) * 4 + b) * 64 + lane) * 4);
        f32x4_t u = *reinterpret_cast<const f32x4_t*>(red + (((0 * 2 + 1) * 4 + b) * 64 + lane) * 4);
#pragma unroll
        for (int w = 1; w < 4; ++w) {
          g += *reinterpret_cast<const f32x4_t*>(red + (((w * 2 + 0) * 4 + b) * 64 + lane) * 4);
          u += *reinterpret_cast<const f32x4_t*>(red + (((w * 2 + 1) * 4 + b) * 64 + lane) * 4);
        }
        const int col = cb0 + 16 * b + r;
        if (col < cnt) {
          const uint32_t h0 = from_f32<ACT>(silu_mul(g.x, u.x));
          const uint32_t h1 = from_f32<ACT>(silu_mul(g.y, u.y));
          const uint32_t h2 = from_f32<ACT>(silu_mul(g.z, u.z));
          const uint32_t h3 = from_f32<ACT>(silu_mul(g.w, u.w));
          u32x2_t pk = {h0 | (h1 << 16), h2 | (h3 << 16)};
          *reinterpret_cast<u32x2_t*>(a.act + (size_t)(p0 + col) * c.I + 16 * j + 4 * q) = pk;
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- phase 2
template <int ACT, int SC>
__device__ void w4_phase2(const W4Args& a, const RouteView& rv, int ui, int hb, int* s_list,
                          int* s_nlist) {
  const SchedArgs& c = a.c;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int e = rv.active[ui];
  const int p0 = rv.starts[e], cnt = rv.starts[e + 1] - p0;
  const int G2 = c.I >> 7, NT = c.H >> 4;
  const int nt = 4 * hb + wave;
  const size_t tile = (size_t)e * NT + nt;
  const char* w_base = (const char*)a.w2 + (tile * G2) * 1024 + lane * 16;
  const u32x4_t ones = {W4Consts<ACT>::ones, W4Consts<ACT>::ones, W4Consts<ACT>::ones,
                        W4Consts<ACT>::ones};

  for (int cb0 = 0; cb0 < cnt; cb0 += kColsPerPass) {
    const int nb = min(4, (cnt - cb0 + 15) >> 4);
    int aoff[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int col = cb0 + 16 * b + r;
      aoff[b] = (b < nb && col < cnt) ? (p0 + col) * c.I : -1;
    }
    f32x4_t acc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[b] = f32x4_t{0, 0, 0, 0};

    for (int gc = 0; gc < G2; gc += 4) {
      u32x4_t wv[4];
#pragma unroll
      for (int gi = 0; gi < 4; ++gi)
        if (gc + gi < G2) wv[gi] = ldg16(w_base + (size_t)(gc + gi) * 1024);
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        if (gc + gi >= G2) break;
        const int g = gc + gi;
        float s[4], cz[4];
        load_meta<ACT, SC>(a.w2_s, a.w2_z, tile * G2 + g, q, s, cz);
        u32x4_t A[4];
        A[0] = deq4<ACT>(wv[gi].x); A[1] = deq4<ACT>(wv[gi].y);
        A[2] = deq4<ACT>(wv[gi].z); A[3] = deq4<ACT>(wv[gi].w);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (b >= nb) break;
          u32x4_t B[4];
          if (aoff[b] >= 0) {
            const uint16_t* ap = a.act + (size_t)aoff[b] + 128 * g + 32 * q;
#pragma unroll
            for (int i = 0; i < 4; ++i) B[i] = ldg16(ap + 8 * i);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) B[i] = u32x4_t{0, 0, 0, 0};
          }
          f32x4_t X = {0, 0, 0, 0}, G = {0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            X = mfma16<ACT>(ones, B[i], X);
            G = mfma16<ACT>(A[i], B[i], G);
          }
          fold(acc[b], G, X, s, cz);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int col = cb0 + 16 * b + r;
      if (b < nb && col < cnt)
        *reinterpret_cast<f32x4_t*>(c.eout + (size_t)(p0 + col) * c.H + 16 * nt + 4 * q) = acc[b];
    }
  }
  combine_hb<ACT>(c, rv, p0, cnt, hb, s_list, s_nlist);
}

// ---------------------------------------------------------------- kernels
constexpr size_t kW4RedBytes = (size_t)4 * 2 * 4 * 64 * 4 * sizeof(float);  // 32 KiB

template <int ACT, int SC>
__global__ __launch_bounds__(kBlock) void w4a16_phase1_kernel(W4Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_U;
  float* red = reinterpret_cast<float*>(smem);
  const RouteView rv = sched_route(a.c, reinterpret_cast<int*>(smem + kW4RedBytes), &s_U);
  if (blockIdx.x == 0) zero_unrouted<ACT>(a.c, rv);
  const int NI1 = a.c.I >> 4;
  const int ui = blockIdx.x / NI1;
  if (ui >= rv.U) return;  // uniform across the workgroup
  w4_phase1<ACT, SC>(a, rv, ui, blockIdx.x % NI1, red);
}

template <int ACT, int SC>
__global__ __launch_bounds__(kBlock) void w4a16_phase2_kernel(W4Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_U, s_nlist;
  __shared__ int s_list[kBlock];
  const RouteView rv = sched_route(a.c, reinterpret_cast<int*>(smem), &s_U);
  const int NI2 = a.c.H >> 6;
  const int ui = blockIdx.x / NI2;
  if (ui >= rv.U) return;
  w4_phase2<ACT, SC>(a, rv, ui, blockIdx.x % NI2, s_list, &s_nlist);
}

// ---------------------------------------------------------------- repack
// AWQ wire -> tiles.  One thread per output u32 word.
//   src qweight [E][Kdim][N/8] (int32), column n, slot AWQ_INV[n%8]
//   tiles per expert NT; tile ti covers rows row0(ti) .. +16, groups Kdim/128
// gate_up (interleave=1): ti = 2*j + which, row0 = which*I + 16*j
// down    (interleave=0): ti = nt,          row0 = 16*nt
__device__ __forceinline__ int awq_slot(int col) {
  return ((col & 1) << 2) | ((col >> 1) & 3);  // {0,4,1,5,2,6,3,7}
}
__device__ __forceinline__ int tile_row0(int ti, int interleave, int I) {
  return interleave ? ((ti & 1) * I + 16 * (ti >> 1)) : 16 * ti;
}

__global__ void awq_repack_qweight(const int32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                   int E, int Kdim, int N, int NT, int interleave, int I) {
  const int G = Kdim >> 7;
  const size_t total = (size_t)E * NT * G * 256;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int wi = idx & 3;
    const int lane = (idx >> 2) & 63;
    size_t t = idx >> 8;
    const int g = t % G; t /= G;
    const int ti = t % NT;
    const int e = (int)(t / NT);
    const int qq = lane >> 4, r = lane & 15;
    const int n = tile_row0(ti, interleave, I) + r;
    const int k0 = 128 * g + 32 * qq + 8 * wi;
    const int sh = 4 * awq_slot(n & 7);
    const int32_t* col = src + (size_t)e * Kdim * (N / 8) + (n >> 3);
    uint32_t word = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = k0 + 2 * p + h;
        const uint32_t nib = ((uint32_t)col[(size_t)k * (N / 8)] >> sh) & 0xfu;
        word |= nib << (4 * p + 16 * h);
      }
    }
    dst[idx] = word;
  }
}

// scales [E][G][N] -> [tile][g][16];  qzeros [E][G][N/8] -> [tile][g][4] u16
__global__ void awq_repack_meta(const uint16_t* __restrict__ scales, const int32_t* __restrict__ qzeros,
                                uint16_t* __restrict__ s_dst, uint16_t* __restrict__ z_dst, int E,
                                int Kdim, int N, int NT, int interleave, int I) {
  const int G = Kdim >> 7;
  const size_t total = (size_t)E * NT * G * 16;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int r = idx & 15;
    size_t t = idx >> 4;
    const int g = t % G; t /= G;
    const int ti = t % NT;
    const int e = (int)(t / NT);
    const int n = tile_row0(ti, interleave, I) + r;
    s_dst[idx] = scales[((size_t)e * G + g) * N + n];
    if ((r & 3) == 0) {
      uint32_t zq = 0;
      for (int v = 0; v < 4; ++v) {
        const int nn = n + v;
        const uint32_t w = (uint32_t)qzeros[((size_t)e * G + g) * (N / 8) + (nn >> 3)];
        zq |= ((w >> (4 * awq_slot(nn & 7))) & 0xfu) << (4 * v);
      }
      z_dst[(idx >> 4) * 4 + (r >> 2)] = (uint16_t)zq;
    }
  }
}

// ---------------------------------------------------------------- launchers
#define W4_INST(ACT, SC)                                                   \
  template __global__ void w4a16_phase1_kernel<ACT, SC>(W4Args);          \
  template __global__ void w4a16_phase2_kernel<ACT, SC>(W4Args);
W4_INST(0, 0)
W4_INST(0, 1)
W4_INST(1, 0)
W4_INST(1, 1)

template <int ACT, int SC>
static hipError_t launch_w4_t(const W4Args& a, int grid1, int grid2, hipStream_t st) {
  const size_t route = a.c.route_global ? 0 : route_lds_ints(a.c.E, a.c.n) * sizeof(int);
  hipLaunchKernelGGL((w4a16_phase1_kernel<ACT, SC>), dim3(grid1), dim3(kBlock), kW4RedBytes + route, st, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((w4a16_phase2_kernel<ACT, SC>), dim3(grid2), dim3(kBlock), route, st, a);
  return hipGetLastError();
}

hipError_t launch_w4a16(const W4Args& a, int act, int sc, int grid1, int grid2, hipStream_t st) {
  if (act == 1 && sc == 1) return launch_w4_t<1, 1>(a, grid1, grid2, st);
  if (act == 1) return launch_w4_t<1, 0>(a, grid1, grid2, st);
  if (sc == 1) return launch_w4_t<0, 1>(a, grid1, grid2, st);
  return launch_w4_t<0, 0>(a, grid1, grid2, st);
}

hipError_t launch_awq_repack(const int32_t* qw, const int32_t* qz, const uint16_t* sc, void* w_dst,
                             uint16_t* s_dst, uint16_t* z_dst, int E, int Kdim, int N, int NT,
                             int interleave, int I, hipStream_t st) {
  const int G = Kdim >> 7;
  size_t total = (size_t)E * NT * G * 256;
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(awq_repack_qweight, dim3(grid), dim3(256), 0, st, qw, (uint32_t*)w_dst, E,
                     Kdim, N, NT, interleave, I);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  total = (size_t)E * NT * G * 16;
  grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(awq_repack_meta, dim3(grid), dim3(256), 0, st, sc, qz, s_dst, z_dst, E, Kdim,
                     N, NT, interleave, I);
  return hipGetLastError();
}

}  // namespace mimoe
