// common_kernels.hip -- routing and Q8_0 activation quantization kernels used
// by every weight format (and exposed alone through the C ABI for checking).
#pragma clang fp contract(off)
#include <algorithm>

#include "mi_moe_device.hpp"
#include "mi_moe_internal.hpp"

namespace mimoe {

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / kWave;

// Routing: the stable counting sort of preprocess_moe_routing
// (Int8-gemm/moe_common.cpp:146-216) for any number of (t,k) pairs, plus, with
// tiles_out, the row tiles of the grouped GEMMs: each active expert's sorted
// rows in chunks of kGemmRows, listed heaviest first (route_finish).
//   n <= kRouteMultiMin: one workgroup (route_global_kernel);
//   above: route_count_kernel (a histogram per chunk of kRouteChunk ids),
//   route_scan_kernel (totals, starts, tiles, and per-chunk base offsets),
//   route_scatter_kernel (stable ranks per chunk).
// Inside a workgroup each wave owns a contiguous segment of ids; per-wave
// per-expert counts are prefix-summed across waves (and, across workgroups,
// seeded with the chunk's base offsets), so ranks stay in (t,k) order.

// Lanes of this wave holding the same valid expert id as this lane.
__device__ __forceinline__ uint64_t route_match(int e, bool valid, int nbits) {
  uint64_t m = __ballot(valid);
  for (int bit = 0; bit < nbits; ++bit) {
    const uint64_t bb = __ballot(valid && ((e >> bit) & 1));
    m &= ((e >> bit) & 1) ? bb : ~bb;
  }
  return m;
}

// Row-tile classes by MFMA sub-tiles: class 0 holds 49-64 rows (4 sub-tiles
// of 16), ..., class 3 holds 1-16 rows.  A W4A16 grouped-GEMM workgroup's time
// grows with its tile's sub-tiles, so with lpt the tile list is ordered
// heaviest class first (longest-processing-time first): the heavy tiles start
// in the first round of workgroups instead of forming the tail of the launch
// (Zipf-routed T = 512, same box: 138.2-138.7 -> 129.9-130.1 us per layer).
// The int8 GEMMs keep each expert's tiles together (lpt = 0): there the
// workgroups of one weight slice and consecutive tiles share an XCD and read
// the slice through its L2 (with lpt, Q4_0 T = 4096 was 2.7% slower).
constexpr int kTileClasses = kGemmRows / 16;
static_assert(kTileClasses == 4, "four 16-row sub-tile classes");
__device__ __forceinline__ int tile_class(int rows) { return kTileClasses - ((rows + 15) >> 4); }

// Wave 0: per-expert totals counts[E] (LDS) -> counts_out, starts_out, the
// active list, U and the row tiles; counts[] becomes the starts.  Tiles are
// listed by class (lpt: heaviest first; otherwise one class), within a class
// by expert, then by row.
__device__ void route_finish(int* counts, int E, int lane, int32_t* counts_out, int32_t* starts_out,
                             int32_t* active_out, int32_t* U_out, int32_t* tiles_out, int32_t* ntiles_out,
                             int lpt) {
  const int per = (E + kWave - 1) / kWave;
  const int base = lane * per;
  // rows, active experts and row tiles per class of this lane's experts
  int s = 0, a = 0, t0 = 0, t1 = 0, t2 = 0, t3 = 0;
  for (int i = 0; i < per; ++i) {
    const int e = base + i;
    if (e < E) {
      const int c = counts[e], rem = c % kGemmRows, k = lpt ? tile_class(rem) : 0;
      s += c; a += (c > 0); t0 += c / kGemmRows;
      if (rem) { t0 += k == 0; t1 += k == 1; t2 += k == 2; t3 += k == 3; }
    }
  }
  int sinc = s, ainc = a, i0 = t0, i1 = t1, i2 = t2, i3 = t3;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(sinc, off), w = __shfl_up(ainc, off);
    const int u0 = __shfl_up(i0, off), u1 = __shfl_up(i1, off), u2 = __shfl_up(i2, off), u3 = __shfl_up(i3, off);
    if (lane >= off) { sinc += v; ainc += w; i0 += u0; i1 += u1; i2 += u2; i3 += u3; }
  }
  const int n0 = __shfl(i0, kWave - 1), n1 = __shfl(i1, kWave - 1), n2 = __shfl(i2, kWave - 1),
            n3 = __shfl(i3, kWave - 1);
  // next free position of each class for this lane's tiles
  int x0 = i0 - t0, x1 = n0 + i1 - t1, x2 = n0 + n1 + i2 - t2, x3 = n0 + n1 + n2 + i3 - t3;
  int sx = sinc - s, ax = ainc - a;
  for (int i = 0; i < per; ++i) {
    const int e = base + i;
    if (e < E) {
      const int c = counts[e];
      counts_out[e] = c;
      starts_out[e] = sx;
      counts[e] = sx;
      if (c > 0) active_out[ax++] = e;
      if (tiles_out)
        for (int r0 = 0; r0 < c; r0 += kGemmRows) {
          const int rows = min(kGemmRows, c - r0), k = lpt ? tile_class(rows) : 0;
          const int tx = k == 0 ? x0++ : k == 1 ? x1++ : k == 2 ? x2++ : x3++;
          *reinterpret_cast<int4*>(tiles_out + 4 * tx) = int4{e, sx + r0, rows, 0};
        }
      sx += c;
    }
  }
  if (lane == kWave - 1) {
    starts_out[E] = sinc;
    *U_out = ainc;
    if (ntiles_out) *ntiles_out = n0 + n1 + n2 + n3;
  }
}

__device__ __forceinline__ int route_bits(int E) {
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  return nbits;
}

// A wave's ids (up to kRouteSegIter batches of 64) and their match masks,
// kept in registers between the counting and the ranking pass.
constexpr int kRouteSegIter = 4;
struct RouteSeg {
  int e[kRouteSegIter];
  uint64_t m[kRouteSegIter];
};

// Counting pass over ids[lo, hi) (hi - lo <= 64 * kRouteSegIter): per-expert
// counts added into mine[E], ids and masks kept in seg.
__device__ __forceinline__ void route_seg_count(const int32_t* __restrict__ ids, int lo, int hi, int E, int nbits,
                                                int lane, int* mine, RouteSeg& seg) {
  // every batch's ids are loaded before the first is used: one memory round
  // trip for the segment, not one per batch
  int ev[kRouteSegIter];
#pragma unroll
  for (int it = 0; it < kRouteSegIter; ++it) {
    const int i = lo + 64 * it + lane;
    ev[it] = i < hi ? ids[i] : -1;
  }
#pragma unroll
  for (int it = 0; it < kRouteSegIter; ++it) {
    const int i = lo + 64 * it + lane;
    int e = -1;
    uint64_t m = 0;
    if (lo + 64 * it < hi) {   // uniform
      e = ev[it];
      const bool valid = (i < hi) && ((unsigned)e < (unsigned)E);
      m = route_match(e, valid, nbits);
      if (!valid) e = -1;
      if (valid && __ffsll((long long)m) - 1 == lane) mine[e] += __popcll(m);
      __builtin_amdgcn_wave_barrier();
    }
    seg.e[it] = e;
    seg.m[it] = m;
  }
}

// Ranking pass: pos = base[e] (if base) + mine[e] (this wave's running
// offset) + rank within the batch; scat[i] = pos and tok[pos] = the token
// (tok_div) or pair index, scat[i] = -1 for an invalid id.
__device__ __forceinline__ void route_seg_rank(int lo, int hi, int K, const int* base, int lane, int* mine,
                                               const RouteSeg& seg, int32_t* tok, int32_t* scat, int tok_div) {
  const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
#pragma unroll
  for (int it = 0; it < kRouteSegIter; ++it) {
    if (lo + 64 * it >= hi) break;   // uniform
    const int i = lo + 64 * it + lane, e = seg.e[it];
    const uint64_t m = seg.m[it];
    int add = 0;
    if (e >= 0) {
      const int pos = (base ? base[e] : 0) + mine[e] + __popcll(m & lt);
      scat[i] = pos;
      tok[pos] = tok_div ? i / K : i;
      if (__ffsll((long long)m) - 1 == lane) add = __popcll(m);
    } else if (i < hi) {
      scat[i] = -1;
    }
    __builtin_amdgcn_wave_barrier();
    if (add) mine[e] += add;
    __builtin_amdgcn_wave_barrier();
  }
}

// One workgroup for n <= kRouteMultiMin ids: each wave counts its segment
// (ids kept in registers), the per-wave counts give the totals and the
// exclusive prefix over waves, then the segments are ranked.
// LDS: (kRouteWaves + 1) * E ints (E <= 512).
static_assert(kRouteMultiMin <= kRouteThreads * kRouteSegIter, "a wave segment fits kRouteSegIter batches");
__device__ __forceinline__ void route_global_body(const int32_t* __restrict__ ids, int n, int K, int E,
                                                  int32_t* counts_out, int32_t* starts_out, int32_t* active_out,
                                                  int32_t* tok, int32_t* scat, int32_t* U_out, int tok_div,
                                                  int32_t* tiles_out, int32_t* ntiles_out, int* lds, int lpt) {
  int* counts = lds;            // [E]: totals, then the starts
  int* cw = lds + E;            // [kRouteWaves][E]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) cw[i] = 0;
  __syncthreads();
  const int nbits = route_bits(E);
  const int segw = ((n + kRouteWaves - 1) / kRouteWaves + kWave - 1) / kWave * kWave;
  const int lo = wave * segw, hi = min(n, lo + segw);
  int* mine = cw + wave * E;
  RouteSeg seg;
  route_seg_count(ids, lo, hi, E, nbits, lane, mine, seg);
  __syncthreads();
  for (int e = tid; e < E; e += kRouteThreads) {   // exclusive prefix over waves; totals
    int run = 0;
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = cw[w * E + e];
      cw[w * E + e] = run;
      run += c;
    }
    counts[e] = run;
  }
  __syncthreads();
  if (tid < kWave)
    route_finish(counts, E, lane, counts_out, starts_out, active_out, U_out, tiles_out, ntiles_out, lpt);
  __syncthreads();
  route_seg_rank(lo, hi, K, counts, lane, mine, seg, tok, scat, tok_div);
}

__global__ __launch_bounds__(kRouteThreads) void route_global_kernel(
    const int32_t* __restrict__ ids, int n, int K, int E, int32_t* counts_out,
    int32_t* starts_out, int32_t* active_out, int32_t* tok, int32_t* scat, int32_t* U_out,
    int tok_div, int32_t* tiles_out, int32_t* ntiles_out, int lpt) {
  extern __shared__ int lds[];
  route_global_body(ids, n, K, E, counts_out, starts_out, active_out, tok, scat, U_out, tok_div, tiles_out,
                    ntiles_out, lds, lpt);
}

// Multi-workgroup routing, step 1: the expert histogram of one chunk of ids.
constexpr int kRouteCountThreads = 256;
static_assert(kRouteChunk % kRouteCountThreads == 0, "a count thread takes a whole number of ids");
__global__ __launch_bounds__(kRouteCountThreads) void route_count_kernel(const int32_t* __restrict__ ids, int n,
                                                                         int E, int32_t* chunk_counts) {
  extern __shared__ int hist[];   // [E]
  const int tid = threadIdx.x, c = blockIdx.x;
  for (int e = tid; e < E; e += kRouteCountThreads) hist[e] = 0;
  __syncthreads();
  const int lo = c * kRouteChunk, hi = min(n, lo + kRouteChunk);
  constexpr int kPer = kRouteChunk / kRouteCountThreads;   // ids per thread, all loaded before use
  int ev[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = lo + tid + j * kRouteCountThreads;
    ev[j] = i < hi ? ids[i] : -1;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if ((unsigned)ev[j] < (unsigned)E) atomicAdd(&hist[ev[j]], 1);
  __syncthreads();
  for (int e = tid; e < E; e += kRouteCountThreads) chunk_counts[(size_t)c * E + e] = hist[e];
}

// Step 2 (one workgroup): totals over the C chunks, the outputs of
// route_finish, and chunk_counts[c][e] replaced by the sorted position of
// chunk c's first row of expert e.
__global__ __launch_bounds__(kRouteThreads) void route_scan_kernel(int32_t* chunk_counts, int C, int E,
                                                                   int32_t* counts_out, int32_t* starts_out,
                                                                   int32_t* active_out, int32_t* U_out,
                                                                   int32_t* tiles_out, int32_t* ntiles_out,
                                                                   int lpt) {
  extern __shared__ int counts[];   // [E]
  const int tid = threadIdx.x, lane = tid & 63;
  // chunk counts in batches of 8 loads issued together (one round trip per batch)
  constexpr int kB = 8;
  for (int e = tid; e < E; e += kRouteThreads) {
    int s = 0;
    for (int c0 = 0; c0 < C; c0 += kB) {
      int v[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) v[j] = c0 + j < C ? chunk_counts[(size_t)(c0 + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < kB; ++j) s += v[j];
    }
    counts[e] = s;
  }
  __syncthreads();
  if (tid < kWave)
    route_finish(counts, E, lane, counts_out, starts_out, active_out, U_out, tiles_out, ntiles_out, lpt);
  __syncthreads();
  for (int e = tid; e < E; e += kRouteThreads) {
    int run = counts[e];
    for (int c0 = 0; c0 < C; c0 += kB) {
      int v[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) v[j] = c0 + j < C ? chunk_counts[(size_t)(c0 + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < kB; ++j)
        if (c0 + j < C) {
          chunk_counts[(size_t)(c0 + j) * E + e] = run;
          run += v[j];
        }
    }
  }
}

// Step 3: stable ranks of one chunk, each wave kRouteChunk / kRouteWaves ids.
// LDS: kRouteWaves * E ints.
__global__ __launch_bounds__(kRouteThreads) void route_scatter_kernel(const int32_t* __restrict__ ids, int n,
                                                                      int K, int E, const int32_t* chunk_base,
                                                                      int32_t* tok, int32_t* scat, int tok_div) {
  extern __shared__ int cw[];   // [kRouteWaves][E]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = blockIdx.x;
  for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) cw[i] = 0;
  __syncthreads();
  const int nbits = route_bits(E);
  constexpr int segw = kRouteChunk / kRouteWaves;
  static_assert(segw <= 64 * kRouteSegIter, "a wave segment fits kRouteSegIter batches");
  const int lo = min(n, c * kRouteChunk + wave * segw), hi = min(n, lo + segw);
  int* mine = cw + wave * E;
  RouteSeg seg;
  route_seg_count(ids, lo, hi, E, nbits, lane, mine, seg);
  __syncthreads();
  for (int e = tid; e < E; e += kRouteThreads) {
    int run = chunk_base[(size_t)c * E + e];
    for (int w = 0; w < kRouteWaves; ++w) {
      const int v = cw[w * E + e];
      cw[w * E + e] = run;
      run += v;
    }
  }
  __syncthreads();
  route_seg_rank(lo, hi, K, nullptr, lane, mine, seg, tok, scat, tok_div);
}

// tok_div = 0: tok[] holds pair indices t*K+k (fused kernels); 1: token ids.
// lpt: row tiles heaviest first (route_finish).
hipError_t launch_route_global(const int32_t* ids, int n, int K, int E, const RouteGlobal& rg,
                               hipStream_t st, int tok_div, int lpt) {
  if (n > kRouteMultiMin) {
    if (!rg.chunk) return hipErrorInvalidValue;   // the chunked routing needs its scratch
    const int C = (n + kRouteChunk - 1) / kRouteChunk;
    hipLaunchKernelGGL(route_count_kernel, dim3(C), dim3(kRouteCountThreads), (size_t)E * sizeof(int), st, ids,
                       n, E, rg.chunk);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(kRouteThreads), (size_t)E * sizeof(int), st, rg.chunk,
                       C, E, rg.counts, rg.starts, rg.active, rg.U, rg.tiles, rg.ntiles, lpt);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(route_scatter_kernel, dim3(C), dim3(kRouteThreads), (size_t)kRouteWaves * E * sizeof(int),
                       st, ids, n, K, E, rg.chunk, rg.tok, rg.scat, tok_div);
    return hipGetLastError();
  }
  const size_t lds = (size_t)(kRouteWaves + 1) * E * sizeof(int);
  hipLaunchKernelGGL(route_global_kernel, dim3(1), dim3(kRouteThreads), lds, st, ids, n, K, E,
                     rg.counts, rg.starts, rg.active, rg.tok, rg.scat, rg.U, tok_div, rg.tiles,
                     rg.ntiles, lpt);
  return hipGetLastError();
}

// Stage C1 + C2 of Int8-gemm/q8_gemm.cpp:593-641 (tp = 1): y[t,h] =
// cast(sum_k w[t,k] * eout[t*K+k, h]) over the valid ids in k order; a token
// without a valid id gets 0.  E16: the rows hold activation-dtype values (the
// W4A16 sorted path; one thread per (t, 8 consecutive h)), else fp32 (one
// thread per (t, 4 consecutive h)): 16-byte row loads either way.
template <int ACT, bool E16>
__global__ void combine_kernel(const float* __restrict__ eout, const float* __restrict__ tw,
                               const int32_t* __restrict__ ids, uint16_t* __restrict__ y, int T,
                               int K, int E, int H) {
  constexpr int V = E16 ? 8 : 4;
  const int HV = H / V;
  const int64_t total = (int64_t)T * HV;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(idx / HV), h = (int)(idx - (int64_t)t * HV) * V;
    float acc[V];
#pragma unroll
    for (int q = 0; q < V; ++q) acc[q] = 0.0f;
    // 8 pairs at a time: their ids, weights and rows are loaded together (the
    // row of a pair with an invalid id is read but not used), then added in k
    // order
    constexpr int kB = 8;
    for (int k0 = 0; k0 < K; k0 += kB) {
      int ev[kB];
      float wv[kB];
      u32x4_t rv[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int i = t * K + min(k0 + j, K - 1);
        ev[j] = k0 + j < K ? ids[i] : -1;
        wv[j] = tw[i];
        const size_t off = (size_t)i * H + h;
        rv[j] = E16 ? *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(eout) + off)
                    : *reinterpret_cast<const u32x4_t*>(eout + off);
      }
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        if ((unsigned)ev[j] >= (unsigned)E) continue;
        const uint32_t u[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
        float vv[V];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (E16) {
            vv[2 * q] = to_f32<ACT>(u[q]);
            vv[2 * q + 1] = to_f32<ACT>(u[q] >> 16);
          } else {
            vv[q] = __uint_as_float(u[q]);
          }
        }
#pragma unroll
        for (int q = 0; q < V; ++q) {
          const float prod = wv[j] * vv[q];
          acc[q] = acc[q] + prod;
        }
      }
    }
    uint32_t o[V / 2];
#pragma unroll
    for (int q = 0; q < V / 2; ++q)
      o[q] = from_f32<ACT>(acc[2 * q]) | ((uint32_t)from_f32<ACT>(acc[2 * q + 1]) << 16);
    if constexpr (E16)
      *reinterpret_cast<u32x4_t*>(y + (size_t)t * H + h) = u32x4_t{o[0], o[1], o[2], o[3]};
    else
      *reinterpret_cast<u32x2_t*>(y + (size_t)t * H + h) = u32x2_t{o[0], o[1]};
  }
}

// eout16 requires H % 8 == 0 (the W4A16 layouts have H % 128 == 0).
hipError_t launch_combine(const float* eout, const float* tw, const int32_t* ids, void* y, int T,
                          int K, int E, int H, int act, hipStream_t st, bool eout16) {
  const int64_t total = (int64_t)T * (H / (eout16 ? 8 : 4));
  if (total == 0) return hipSuccess;
  int64_t grid = (total + 255) / 256;
  if (grid > 65536) grid = 65536;
  auto kern = act == 1 ? (eout16 ? combine_kernel<1, true> : combine_kernel<1, false>)
                       : (eout16 ? combine_kernel<0, true> : combine_kernel<0, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, st, eout, tw, ids, (uint16_t*)y, T, K, E, H);
  return hipGetLastError();
}

// Stage A: one thread per 32-element block, through quant_block_q8_0 (the
// block quantizer of the decode kernels too): amax, d = amax/127, id = 1/d (0
// if d == 0), q = sat8(RNE(x*id)) (Int8-gemm/gemm_kernels.cpp:37-57); d stays
// fp32 (Int8-gemm/q8_gemm.cpp:371-375).
template <int ACT>
__device__ __forceinline__ void quant_act_blocks(const uint16_t* __restrict__ x, int64_t b0, int64_t stride,
                                                 int64_t nblk, int8_t* __restrict__ qs, float* __restrict__ d) {
  for (int64_t b = b0; b < nblk; b += stride) {
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(x + b * 32);
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4_t w = src[c];
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        v[8 * c + 2 * h] = to_f32<ACT>(ws[h] & 0xffffu);
        v[8 * c + 2 * h + 1] = to_f32<ACT>(ws[h] >> 16);
      }
    }
    int qsum;
    d[b] = quant_block_q8_0(v, qs + b * 32, &qsum);
  }
}

template <int ACT>
__global__ void quant_act_q8_0_kernel(const uint16_t* __restrict__ x, int64_t nblk,
                                      int8_t* __restrict__ qs, float* __restrict__ d) {
  quant_act_blocks<ACT>(x, (int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x, nblk,
                        qs, d);
}

// The single-workgroup routing and Stage A in one launch (the two are
// independent): workgroup 0 routes, the others quantize.
template <int ACT>
__global__ __launch_bounds__(kRouteThreads) void route_quant_kernel(
    const int32_t* __restrict__ ids, int n, int K, int E, int32_t* counts_out, int32_t* starts_out,
    int32_t* active_out, int32_t* tok, int32_t* scat, int32_t* U_out, int tok_div, int32_t* tiles_out,
    int32_t* ntiles_out, const uint16_t* __restrict__ x, int64_t nblk, int8_t* __restrict__ qs,
    float* __restrict__ d) {
  extern __shared__ int lds[];
  if (blockIdx.x == 0) {   // uniform
    route_global_body(ids, n, K, E, counts_out, starts_out, active_out, tok, scat, U_out, tok_div, tiles_out,
                      ntiles_out, lds, 0);
    return;
  }
  quant_act_blocks<ACT>(x, (int64_t)(blockIdx.x - 1) * kRouteThreads + threadIdx.x,
                        (int64_t)(gridDim.x - 1) * kRouteThreads, nblk, qs, d);
}


hipError_t launch_quant_act(const void* x, int act, int64_t T, int64_t H, int8_t* qs, float* d,
                            hipStream_t st) {
  const int64_t nblk = T * (H / 32);
  if (nblk == 0) return hipSuccess;
  int64_t grid = (nblk + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (act == 1)
    hipLaunchKernelGGL(quant_act_q8_0_kernel<1>, dim3((unsigned)grid), dim3(256), 0, st,
                       (const uint16_t*)x, nblk, qs, d);
  else
    hipLaunchKernelGGL(quant_act_q8_0_kernel<0>, dim3((unsigned)grid), dim3(256), 0, st,
                       (const uint16_t*)x, nblk, qs, d);
  return hipGetLastError();
}

// Stage A (Q8_0 of the T hidden rows) and the routing of the sorted path; one
// launch when the routing is a single workgroup.
hipError_t launch_quant_route(const void* x, int act, int64_t T, int64_t H, int8_t* qs, float* d,
                              const int32_t* ids, int n, int K, int E, const RouteGlobal& rg, hipStream_t st,
                              int tok_div) {
  const int64_t nblk = T * (H / 32);
  if (n > kRouteMultiMin || nblk == 0) {
    hipError_t err = launch_quant_act(x, act, T, H, qs, d, st);
    if (err != hipSuccess) return err;
    return launch_route_global(ids, n, K, E, rg, st, tok_div, 0);
  }
  const int64_t gq = std::min<int64_t>((nblk + kRouteThreads - 1) / kRouteThreads, 1024);
  const size_t lds = (size_t)(kRouteWaves + 1) * E * sizeof(int);
  auto kern = act == 1 ? route_quant_kernel<1> : route_quant_kernel<0>;
  hipLaunchKernelGGL(kern, dim3((unsigned)(1 + gq)), dim3(kRouteThreads), lds, st, ids, n, K, E, rg.counts,
                     rg.starts, rg.active, rg.tok, rg.scat, rg.U, tok_div, rg.tiles, rg.ntiles, (const uint16_t*)x,
                     nblk, qs, d);
  return hipGetLastError();
}

// Router top-k + softmax (make_topk_from_logits_cpu,
// Int8-gemm/test/fused_moe_cpu.py:20-37): one wave per token.  Lane l holds
// logits l, l+64, ... (E <= kTopkMaxE).  K rounds of a wave arg-max (the
// larger logit, then the lower id: a total order, so every lane agrees; DPP
// inside rows, readlane across them);
// lane k keeps pick k.  Softmax over the K picks (renorm) or over all E
// gathered at the picks, with mi_expf and the sum taken in k (or e) order by
// lane 0 through LDS, w = e / s: the arithmetic of orc_topk_softmax.
constexpr int kTopkWaves = 4;
constexpr int kTopkMaxE = 512;
constexpr int kTopkMaxK = 64;

// (v, i) beats (bv, bi): the larger logit, then the lower id
__device__ __forceinline__ bool topk_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int CTRL>
__device__ __forceinline__ void topk_dpp_step(float& bv, int& bi) {
  const float ov = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(bv), CTRL, 0xf, 0xf, false));
  const int oi = __builtin_amdgcn_mov_dpp(bi, CTRL, 0xf, 0xf, false);
  if (topk_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
}

// Wave arg-max of (bv, bi) under topk_better; the result in every lane.
// Inside each 16-lane row: row_mirror (i <-> 15-i), row_half_mirror
// (i <-> 7-i in each half), quad_perm [2,3,0,1] and [1,0,3,2] leave every
// lane with the row's best; then the four rows through readlane.
__device__ __forceinline__ void topk_wave_argmax(float& bv, int& bi) {
  topk_dpp_step<0x140>(bv, bi);   // row_mirror
  topk_dpp_step<0x141>(bv, bi);   // row_half_mirror
  topk_dpp_step<0x4e>(bv, bi);    // quad_perm [2,3,0,1]
  topk_dpp_step<0xb1>(bv, bi);    // quad_perm [1,0,3,2]
  float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
  int ri = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
  for (int row = 1; row < 4; ++row) {
    const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 16 * row));
    const int i = __builtin_amdgcn_readlane(bi, 16 * row);
    if (topk_better(v, i, rv, ri)) { rv = v; ri = i; }
  }
  bv = rv;
  bi = ri;
}
template <int LDT>  // logits: 0 fp16, 1 bf16, 2 fp32
__global__ __launch_bounds__(kTopkWaves * kWave) void topk_softmax_kernel(const void* __restrict__ logits,
                                                                          int T, int E, int K, int renorm,
                                                                          int32_t* __restrict__ ids_out,
                                                                          float* __restrict__ w_out) {
  __shared__ float ex[kTopkWaves][kTopkMaxE];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * kTopkWaves + wave;
  if (t >= T) return;   // whole wave; no workgroup barrier follows
  constexpr int NJ = kTopkMaxE / kWave;
  float v[NJ];
  bool live[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = lane + kWave * j;
    live[j] = e < E;
    const size_t off = (size_t)t * E + (live[j] ? e : 0);
    if constexpr (LDT == 2) v[j] = reinterpret_cast<const float*>(logits)[off];
    else v[j] = to_f32<LDT>(reinterpret_cast<const uint16_t*>(logits)[off]);
  }
  float myv = 0.0f;
  int myid = 0;
  for (int k = 0; k < K; ++k) {
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;   // no candidate: loses to any real one
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (live[j] && (bi == 0x7fffffff || v[j] > bv)) { bv = v[j]; bi = lane + kWave * j; }
    topk_wave_argmax(bv, bi);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (bi == lane + kWave * j) live[j] = false;
    if (lane == k) { myv = bv; myid = bi; }
  }
  const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myv), 0));
  float* exw = ex[wave];
  float e_k = 0.0f;
  if (renorm) {
    if (lane < K) {
      e_k = mi_expf(myv - m);
      exw[lane] = e_k;
    }
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = lane + kWave * j;
      if (e < E) exw[e] = mi_expf(v[j] - m);
    }
  }
  __builtin_amdgcn_wave_barrier();
  float s = 0.0f;
  if (lane == 0) {
    const int cnt = renorm ? K : E;
    for (int i = 0; i < cnt; ++i) s = s + exw[i];
  }
  s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
  if (lane < K) {
    if (!renorm) e_k = exw[myid];
    ids_out[(size_t)t * K + lane] = myid;
    w_out[(size_t)t * K + lane] = e_k / s;
  }
}

hipError_t launch_topk_softmax(const void* logits, int ldt, int T, int E, int K, int renorm, int32_t* ids,
                               float* w, hipStream_t st) {
  if (T == 0) return hipSuccess;
  const dim3 grid((T + kTopkWaves - 1) / kTopkWaves), block(kTopkWaves * kWave);
  if (ldt == 2)
    hipLaunchKernelGGL(topk_softmax_kernel<2>, grid, block, 0, st, logits, T, E, K, renorm, ids, w);
  else if (ldt == 1)
    hipLaunchKernelGGL(topk_softmax_kernel<1>, grid, block, 0, st, logits, T, E, K, renorm, ids, w);
  else
    hipLaunchKernelGGL(topk_softmax_kernel<0>, grid, block, 0, st, logits, T, E, K, renorm, ids, w);
  return hipGetLastError();
}

}  // namespace mimoe
