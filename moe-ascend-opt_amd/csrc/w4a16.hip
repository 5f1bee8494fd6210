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
// Work decomposition (one persistent launch, tickets from an atomic counter):
//   phase 1 item (expert, j): rows j*16.. of gate and up, all H; 4 waves split
//     the groups; LDS reduction; SiLU*mul; write act[pos][16j..16j+15].
//   phase 2 item (expert, hb): 64 rows of down (one 16-row tile per wave),
//     all I; waits for the expert's phase-1 items (bounded spin), writes
//     eout[pos][64hb..]; the last arriving expert of a token does the combine
//     y[t] = cast(sum_k w[t,k] * eout[scatter[t,k]]) in k order
//     (Int8-gemm/q8_gemm.cpp:593-641).
// Tickets are taken in order, so every phase-1 item a phase-2 item waits on is
// already held by a running workgroup that never waits: no deadlock.
#pragma clang fp contract(off)
#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"

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

struct RouteView {
  const int* starts;
  const int* active;
  const int* tok;
  const int* scat;
  int U;
};

__device__ __forceinline__ int nvalid_of(const RouteView& rv, int t, int K) {
  int c = 0;
  for (int k = 0; k < K; ++k) c += rv.scat[t * K + k] >= 0;
  return c;
}

// ---------------------------------------------------------------- phase 1
template <int ACT, int SC>
__device__ void w4_phase1(const W4Args& a, const RouteView& rv, int ui, int j, float* red) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int e = rv.active[ui];
  const int p0 = rv.starts[e], cnt = rv.starts[e + 1] - p0;
  const int G1 = a.H >> 7, NI1 = a.I >> 4;
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
      xoff[b] = (b < nb && col < cnt) ? rv.tok[p0 + col] * a.H : -1;
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
            const uint16_t* xp = a.x + xoff[b] + 128 * g + 32 * q;
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
          *reinterpret_cast<u32x2_t*>(a.act + (size_t)(p0 + col) * a.I + 16 * j + 4 * q) = pk;
        }
      }
    }
    __syncthreads();
  }
  // every wave publishes its act stores (L2 write-back), then one arrival
  fence_release();
  __syncthreads();
  if (tid == 0)
    __hip_atomic_fetch_add(a.done1 + e, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- phase 2
template <int ACT, int SC>
__device__ void w4_phase2(const W4Args& a, const RouteView& rv, int ui, int hb, int* s_list,
                          int* s_nlist) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4, r = lane & 15;
  const int e = rv.active[ui];
  const int p0 = rv.starts[e], cnt = rv.starts[e + 1] - p0;
  const int G2 = a.I >> 7, NI1 = a.I >> 4, NI2 = a.H >> 6, NT = a.H >> 4;
  const int nt = 4 * hb + wave;
  const size_t tile = (size_t)e * NT + nt;
  const char* w_base = (const char*)a.w2 + (tile * G2) * 1024 + lane * 16;
  const u32x4_t ones = {W4Consts<ACT>::ones, W4Consts<ACT>::ones, W4Consts<ACT>::ones,
                        W4Consts<ACT>::ones};

  // Issue the first weight loads before waiting on the expert's activations.
  u32x4_t wpre[4];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi)
    if (gi < G2) wpre[gi] = ldg16(w_base + (size_t)gi * 1024);

  if (tid == 0) {
    uint32_t spins = 0;
    while (ld_acquire_relaxed(a.done1 + e) < (uint32_t)NI1) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kSpinLimit) {
        __hip_atomic_store(a.ctl + CTL_ERROR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
  fence_acquire();

  for (int cb0 = 0; cb0 < cnt; cb0 += kColsPerPass) {
    const int nb = min(4, (cnt - cb0 + 15) >> 4);
    int aoff[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int col = cb0 + 16 * b + r;
      aoff[b] = (b < nb && col < cnt) ? (p0 + col) * a.I : -1;
    }
    f32x4_t acc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[b] = f32x4_t{0, 0, 0, 0};

    for (int gc = 0; gc < G2; gc += 4) {
      u32x4_t wv[4];
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        if (gc + gi < G2) wv[gi] = (gc == 0 && cb0 == 0) ? wpre[gi] : ldg16(w_base + (size_t)(gc + gi) * 1024);
      }
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        if (gc + gi >= G2) break;
        const int g = gc + gi;
        float s[4], c[4];
        load_meta<ACT, SC>(a.w2_s, a.w2_z, tile * G2 + g, q, s, c);
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
          fold(acc[b], G, X, s, c);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int col = cb0 + 16 * b + r;
      if (b < nb && col < cnt)
        *reinterpret_cast<f32x4_t*>(a.eout + (size_t)(p0 + col) * a.H + 16 * nt + 4 * q) = acc[b];
    }
  }
  fence_release();
  __syncthreads();

  // Combine: count arrivals per (token, hb); the last expert of a token sums
  // eout over k in order and casts.
  for (int c0 = 0; c0 < cnt; c0 += kBlock) {
    if (tid == 0) *s_nlist = 0;
    __syncthreads();
    const int c = c0 + tid;
    if (c < cnt) {
      const int t = rv.tok[p0 + c];
      const uint32_t old = __hip_atomic_fetch_add(a.cnt2 + (size_t)t * NI2 + hb, 1u,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((int)old + 1 == nvalid_of(rv, t, a.K)) s_list[atomicAdd(s_nlist, 1)] = t;
    }
    __syncthreads();
    const int nl = *s_nlist;
    if (nl > 0) {
      fence_acquire();
      for (int li = wave; li < nl; li += 4) {
        const int t = s_list[li];
        const int h = 64 * hb + lane;
        float acc = 0.0f;
        for (int k = 0; k < a.K; ++k) {
          const int pos = rv.scat[t * a.K + k];
          if (pos < 0) continue;
          const float prod = a.tw[t * a.K + k] * a.eout[(size_t)pos * a.H + h];
          acc = acc + prod;
        }
        a.y[(size_t)t * a.H + h] = from_f32<ACT>(acc);
        if (lane == 0) a.cnt2[(size_t)t * NI2 + hb] = 0u;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- kernel
template <int ACT, int SC>
__global__ __launch_bounds__(kBlock) void w4a16_fused_kernel(W4Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_ticket, s_U, s_nlist;
  __shared__ int s_list[kBlock];
  float* red = reinterpret_cast<float*>(smem);                  // 32 KiB
  int* rl = reinterpret_cast<int*>(smem + 4 * 2 * 4 * 64 * 4 * 4);
  const int tid = threadIdx.x;

  RouteView rv;
  if (!a.route_global) {
    int* counts = rl;
    int* starts = counts + a.E;
    int* active = starts + a.E + 1;
    int* tok = active + a.E;
    int* scat = tok + a.n;
    route_lds(a.ids, a.n, a.K, a.E, counts, starts, active, tok, scat, &s_U);
    rv.starts = starts; rv.active = active; rv.tok = tok; rv.scat = scat; rv.U = s_U;
  } else {
    rv.starts = a.rg.starts; rv.active = a.rg.active; rv.tok = a.rg.tok; rv.scat = a.rg.scat;
    rv.U = *a.rg.U;
  }
  const int NI1 = a.I >> 4, NI2 = a.H >> 6;
  const int total1 = rv.U * NI1, total = rv.U * (NI1 + NI2);

  for (;;) {
    if (tid == 0) s_ticket = (int)atomicAdd(a.ctl + CTL_TICKET, 1u);
    __syncthreads();
    const int tk = s_ticket;
    __syncthreads();
    if (tk == 0) {
      // tokens without any valid expert id get y = 0 (Int8-gemm/q8_gemm.cpp:329-332, 599-611)
      for (int t = tid >> 6; t < a.T; t += 4) {
        if (nvalid_of(rv, t, a.K) == 0)
          for (int h = tid & 63; h < a.H; h += 64) a.y[(size_t)t * a.H + h] = 0;
      }
    }
    if (tk >= total) break;
    if (tk < total1) {
      w4_phase1<ACT, SC>(a, rv, tk / NI1, tk % NI1, red);
    } else {
      const int t2 = tk - total1;
      w4_phase2<ACT, SC>(a, rv, t2 / NI2, t2 % NI2, s_list, &s_nlist);
    }
  }
  // The last workgroup out resets the per-call counters for the next launch.
  if (tid == 0) {
    fence_release();
    const uint32_t old = atomicAdd(a.ctl + CTL_EXIT, 1u);
    if (old == gridDim.x - 1) {
      fence_acquire();
      for (int e = 0; e < a.E; ++e) a.done1[e] = 0u;
      a.ctl[CTL_TICKET] = 0u;
      a.ctl[CTL_EXIT] = 0u;
      fence_release();
    }
  }
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
#define W4_INST(ACT, SC) template __global__ void w4a16_fused_kernel<ACT, SC>(W4Args);
W4_INST(0, 0)
W4_INST(0, 1)
W4_INST(1, 0)
W4_INST(1, 1)

size_t w4a16_lds_bytes(const W4Args& a) {
  size_t red = (size_t)4 * 2 * 4 * 64 * 4 * sizeof(float);
  size_t route = a.route_global ? 0 : (size_t)(3 * a.E + 1 + 2 * a.n) * sizeof(int);
  return red + route;
}

hipError_t launch_w4a16_fused(const W4Args& a, int act, int sc, int grid, hipStream_t st) {
  const size_t lds = w4a16_lds_bytes(a);
  if (act == 1 && sc == 1) hipLaunchKernelGGL((w4a16_fused_kernel<1, 1>), dim3(grid), dim3(kBlock), lds, st, a);
  else if (act == 1) hipLaunchKernelGGL((w4a16_fused_kernel<1, 0>), dim3(grid), dim3(kBlock), lds, st, a);
  else if (sc == 1) hipLaunchKernelGGL((w4a16_fused_kernel<0, 1>), dim3(grid), dim3(kBlock), lds, st, a);
  else hipLaunchKernelGGL((w4a16_fused_kernel<0, 0>), dim3(grid), dim3(kBlock), lds, st, a);
  return hipGetLastError();
}

int w4a16_max_blocks_per_cu(int act, int sc, size_t lds) {
  int nb = 0;
  hipError_t err;
  if (act == 1 && sc == 1) err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, w4a16_fused_kernel<1, 1>, kBlock, lds);
  else if (act == 1) err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, w4a16_fused_kernel<1, 0>, kBlock, lds);
  else if (sc == 1) err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, w4a16_fused_kernel<0, 1>, kBlock, lds);
  else err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, w4a16_fused_kernel<0, 0>, kBlock, lds);
  if (err != hipSuccess || nb < 1) nb = 1;
  return nb;
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
