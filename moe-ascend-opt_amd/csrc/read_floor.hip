// read_floor.hip -- read-only floors of the W4A16 decode layer (Qwen3 shape:
// H=2048, I=768, E=128, top-8, AWQ int4 group 128) on one GPU: kernels that
// only read the bytes a layer call must read (the distinct routed experts'
// gate_up block of 1,634,304 B and down block of 817,152 B each), from 16
// rotated weight copies, replayed from a HIP graph of 256 calls per batch
// size, like the headline benchmark.  Three layouts:
//  * "grid": the shipped one-launch kernel's grid -- 512-thread workgroups,
//    gate_up items per (pair, block of S slices of 16 rows of I; a pair
//    serves its expert iff it is the expert's first pair), then down items per
//    (token, RT 16-row tiles of H) that read the tiles of the token's 8
//    experts -- each workgroup reading only, with no hand-over;
//  * "grid2": the same items as two launches (gate_up, then down);
//  * "chunk": the best plain streaming form measured: 256-thread workgroups
//    each reading one 16 KB chunk of a distinct expert, 4 loads per thread in
//    flight, one launch.
// Each workgroup XORs what it read into a value it stores only if it equals a
// constant, so the loads cannot be dropped.  Prints one JSON line.
// Built by nanovllm_moe/build.py into nanovllm_moe/mimoe_read_floor; run by
// `python3 bench.py --read-floor`.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CK(x)                                                                       \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) {                                                         \
      std::fprintf(stderr, "%s: %s (line %d)\n", #x, hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                 \
    }                                                                               \
  } while (0)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int H = 2048, I = 768, E = 128, K = 8, NSETS = 16, NCALL = 256, NROUTE = 32;
constexpr size_t W13 = 1634304, W2 = 817152, EB = W13 + W2;
constexpr int NI1 = I / 16;            // gate_up slices of 16 rows
constexpr int NT = H / 16;             // down tiles of 16 rows
constexpr size_t SLICE = W13 / NI1;    // 34,048 B: a slice's gate and up rows with their scales and zeros
constexpr size_t TILE = W2 / NT;       // 6,384 B: a down tile over all of I with its metadata

__device__ __forceinline__ u32x4 ld(const char* p) { return *reinterpret_cast<const u32x4*>(p); }

// Read n bytes from p with the workgroup (16-byte loads, all issued before use).
template <int NTHR>
__device__ __forceinline__ u32x4 read_block(const char* p, size_t n) {
  u32x4 acc = {0, 0, 0, 0};
  constexpr int kBatch = 8;
  for (size_t o0 = 0; o0 < n; o0 += (size_t)NTHR * 16 * kBatch) {
    u32x4 v[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const size_t o = o0 + ((size_t)b * NTHR + threadIdx.x) * 16;
      v[b] = o + 16 <= n ? ld(p + o) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) acc ^= v[b];
  }
  return acc;
}

// Is pair i the first pair of its expert among ids[0, n)?  (every thread)
__device__ __forceinline__ bool first_pair(const int* ids, int n, int i, int& e) {
  e = ids[i];
  for (int j = 0; j < i; ++j)
    if (ids[j] == e) return false;
  return true;
}

// gate_up items [0, n1): (pair, slice block of S slices); down items after:
// (token, RT tiles) reading the tiles of the token's K experts.
template <int S, int RT>
__global__ __launch_bounds__(512) void grid_kernel(const char* base, const int* ids, int n, int n1, int role,
                                                   unsigned* out) {
  const int b = blockIdx.x + (role == 2 ? n1 : 0);
  const int njs = NI1 / S;
  u32x4 acc = {0, 0, 0, 0};
  if (b < n1) {
    const int item = b / njs, js = b - item * njs;
    int e;
    if (!first_pair(ids, n, item, e)) return;
    acc = read_block<512>(base + (size_t)e * EB + (size_t)js * S * SLICE, S * SLICE);
  } else {
    const int d = b - n1, nt = NT / RT, t = d / nt, tile0 = (d - t * nt) * RT;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = ids[t * K + wave];   // wave k reads expert k's RT tiles
    const char* p = base + (size_t)e * EB + W13 + (size_t)tile0 * TILE;
    constexpr int kLoads = (int)((RT * TILE + 1023) / 1024);   // all of the wave's loads in flight together
    u32x4 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const size_t o = (size_t)i * 1024 + (size_t)lane * 16;
      v[i] = o + 16 <= RT * TILE ? ld(p + o) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) acc ^= v[i];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) out[b] = 1;
}

// 16 KB chunk c of distinct expert slot u (elist: the call's distinct experts).
__global__ __launch_bounds__(256) void chunk_kernel(const char* base, const int* elist, const int* nu, int cpe,
                                                    unsigned* out) {
  const int u = blockIdx.x / cpe, c = blockIdx.x - u * cpe;
  if (u >= *nu) return;
  const char* p = base + (size_t)elist[u] * EB + (size_t)c * 16384;
  u32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = ld(p + ((size_t)i * 256 + threadIdx.x) * 16);
  const u32x4 acc = v[0] ^ v[1] ^ v[2] ^ v[3];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) out[blockIdx.x] = 1;
}

unsigned rng_state = 12345u;
unsigned rnd() {
  rng_state = rng_state * 1664525u + 1013904223u;
  return rng_state >> 8;
}

}  // namespace

int main() {
  char* w = nullptr;
  CK(hipMalloc(&w, (size_t)NSETS * E * EB));
  CK(hipMemset(w, 1, (size_t)NSETS * E * EB));
  unsigned* out = nullptr;
  CK(hipMalloc(&out, 1 << 20));
  hipStream_t st;
  CK(hipStreamCreate(&st));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  std::printf("{\"workload\": \"read-only floors of the W4A16 decode layer, Qwen3 shape (H=2048, I=768, E=128, "
              "top-8), 16 weight copies rotated, HIP-graph replay of %d calls\", \"per_batch\": {", NCALL);
  const int batches[] = {1, 2, 4, 8};
  for (int bi = 0; bi < 4; ++bi) {
    const int T = batches[bi], n = T * K;
    // routings: uniform top-8 of 128 per token
    std::vector<int> ids((size_t)NROUTE * n), elist((size_t)NROUTE * 64, 0), nu(NROUTE);
    double meanU = 0;
    for (int r = 0; r < NROUTE; ++r) {
      std::vector<int> all;
      for (int t = 0; t < T; ++t) {
        std::vector<int> perm(E);
        for (int i = 0; i < E; ++i) perm[i] = i;
        for (int i = E - 1; i > 0; --i) std::swap(perm[i], perm[rnd() % (unsigned)(i + 1)]);
        for (int k = 0; k < K; ++k) {
          ids[(size_t)r * n + t * K + k] = perm[k];
          all.push_back(perm[k]);
        }
      }
      std::sort(all.begin(), all.end());
      all.erase(std::unique(all.begin(), all.end()), all.end());
      nu[r] = (int)all.size();
      std::copy(all.begin(), all.end(), elist.begin() + (size_t)r * 64);
      meanU += (double)all.size() / NROUTE;
    }
    int *d_ids, *d_el, *d_nu;
    CK(hipMalloc(&d_ids, ids.size() * 4));
    CK(hipMalloc(&d_el, elist.size() * 4));
    CK(hipMalloc(&d_nu, nu.size() * 4));
    CK(hipMemcpy(d_ids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_el, elist.data(), elist.size() * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_nu, nu.data(), nu.size() * 4, hipMemcpyHostToDevice));
    // the shipped kernel's geometry: 8-wave slices at <= 8 pairs, else 2 slices of
    // 4 waves; down items of 1 or 2 tiles by its slot rule (2 workgroups per CU)
    const int S = n <= 8 ? 1 : 2, njs = NI1 / S, n1 = n * njs;
    int cus = 0;
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const long slots = 2L * cus, tiles = (long)T * NT;
    const int RT = (S == 2 && (tiles > slots || (n1 + tiles > slots && n1 + tiles / 2 <= slots))) ? 2 : 1;
    const int n2 = T * NT / RT;
    const double bytes = meanU * (double)EB;
    std::printf("%s\"%d\": {\"mean_unique_experts\": %.2f, \"bytes_per_call\": %.0f, \"grid\": \"%d + %d "
                "workgroups of 512, S=%d, RT=%d\"", bi ? ", " : "", T, meanU, bytes, n1, n2, S, RT);
    const char* names[] = {"one_launch_grid", "two_launch_grid", "one_launch_chunk16k"};
    for (int v = 0; v < 3; ++v) {
      hipGraph_t g;
      hipGraphExec_t ge;
      CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
      for (int i = 0; i < NCALL; ++i) {
        const int r = i % NROUTE;
        const char* base = w + (size_t)(i % NSETS) * E * EB;
        const int* di = d_ids + (size_t)r * n;
        if (v < 2) {
          auto k = S == 1 ? grid_kernel<1, 1> : (RT == 2 ? grid_kernel<2, 2> : grid_kernel<2, 1>);
          if (v == 0) {
            hipLaunchKernelGGL(k, dim3(n1 + n2), dim3(512), 0, st, base, di, n, n1, 0, out);
          } else {
            hipLaunchKernelGGL(k, dim3(n1), dim3(512), 0, st, base, di, n, n1, 1, out);
            hipLaunchKernelGGL(k, dim3(n2), dim3(512), 0, st, base, di, n, n1, 2, out);
          }
        } else {
          const int cpe = (int)(EB / 16384);   // the last 10,240 B of an expert are not read (0.4%)
          hipLaunchKernelGGL(chunk_kernel, dim3(std::min(n, E) * cpe), dim3(256), 0, st, base, d_el + (size_t)r * 64,
                             d_nu + r, cpe, out);
        }
      }
      CK(hipStreamEndCapture(st, &g));
      CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
      CK(hipGraphLaunch(ge, st));
      CK(hipStreamSynchronize(st));
      float best = 1e30f;
      for (int rep = 0; rep < 3; ++rep) {
        CK(hipEventRecord(e0, st));
        CK(hipGraphLaunch(ge, st));
        CK(hipEventRecord(e1, st));
        CK(hipStreamSynchronize(st));
        float ms = 0;
        CK(hipEventElapsedTime(&ms, e0, e1));
        best = std::min(best, ms);
      }
      const double us = best * 1e3 / NCALL;
      std::printf(", \"%s_us\": %.2f, \"%s_frac\": %.4f", names[v], us, names[v], bytes / (us * 1e-6) / 8e12);
      CK(hipGraphExecDestroy(ge));
      CK(hipGraphDestroy(g));
    }
    std::printf("}");
    std::fflush(stdout);
    CK(hipFree(d_ids));
    CK(hipFree(d_el));
    CK(hipFree(d_nu));
  }
  std::printf("}}\n");
  return 0;
}
