// mi_moe_internal.hpp -- structures shared by the kernels and the C-ABI host
// code of libmimoe.so.  Not part of the public ABI (include/mi_moe.h is).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimoe {

// Routing done inside the fused kernel (LDS) up to this many (t,k) pairs;
// beyond it a separate routing kernel writes the arrays to the workspace.
constexpr int kRouteLdsMax = 1024;
// Tokens per pass of the integer path (activations staged in LDS).
constexpr int kQTokPerPass = 8;

// Routing arrays written by the standalone routing kernel (global path).
struct RouteGlobal {
  int32_t* counts;   // [E]
  int32_t* starts;   // [E+1]
  int32_t* active;   // [E]
  int32_t* tok;      // [n]
  int32_t* scat;     // [n]
  int32_t* U;        // [1]
  int32_t* tiles;    // [n/kGemmRows + E][4]: expert, first sorted row, rows (<= kGemmRows), 0; or null
  int32_t* ntiles;   // [1]
  int32_t* chunk;    // [ceil(n / kRouteChunk)][E] scratch of the multi-workgroup routing, or null
};

// Routing: one workgroup up to kRouteMultiMin pairs, three launches over
// chunks of kRouteChunk ids above.
constexpr int kRouteChunk = 2048;
constexpr int kRouteMultiMin = 4096;
__host__ __device__ constexpr int route_chunks(int n) { return (n + kRouteChunk - 1) / kRouteChunk; }

// Row tile of the grouped GEMMs of the sorted path: routed rows of one expert.
constexpr int kGemmRows = 64;
// Q8_0 / Q4_0: above this many routed pairs the int8 grouped GEMMs run
constexpr int kQGemmMinPairs = 64;
// Q8_0 / Q4_0 lane-per-row gate_up: up to this many routed pairs the work
// items are pairs routed by one ballot per wave (grid = pairs x slices).
constexpr int kQBallotMaxPairs = 64;
__host__ __device__ inline int64_t gemm_tiles_max(int64_t n, int E) {
  return n / kGemmRows + (n < E ? n : E);
}

// Error reporting and shape rules shared by the C-ABI translation units:
// api_fail records msg as the thread's last error and returns code;
// check_dims applies the handle shape rules of mi_moe_create.
int api_fail(int code, const char* msg);
int check_dims(int64_t E, int64_t H, int64_t I, int quant_type);

// Arguments every fused kernel shares (routing, schedule, combine).
struct SchedArgs {
  const uint16_t* x;       // [T,H] act dtype bits
  uint16_t* y;             // [T,H]
  const float* tw;         // [T,K]
  const int32_t* ids;      // [T,K]
  int T, K, E, H, I, n;
  int route_global;
  RouteGlobal rg;
  float* eout;             // [n, H] per-pair expert outputs (row i = t*K+k)
};

// W4A16 fused kernels (w4a16.hip).
struct W4Args {
  SchedArgs c;
  const void* w13;             // uint4 tiles [e][I/16][gate,up][H/128][64 lanes][16 B]
  const unsigned char* w13_m;  // metadata blocks of 80*(H/128) bytes per (e, I/16 slice)
  const void* w2;              // [e][H/64][4][I/128][64 lanes][16 B]
  const unsigned char* w2_m;   // metadata sections of w2_meta_sec_bytes(I/128) per (e, H/64 quad, row tile)
  uint16_t* act;               // [n, I] SiLU*mul activations (act dtype), row = pair
  int p1_cols;                 // phase-1 token columns per pass (rows staged in LDS)
  int sdt;                     // scale dtype: 1 bf16, 0 fp16
  int x_all;                   // phase 1 copies the hidden rows of all T tokens at start
};

// Bytes of the w2 metadata of one 16-row tile: G2 = I/128 groups of 16 u16
// scales and 8 bytes of zero nibbles, rounded up to 16 bytes.
__host__ __device__ inline int w2_meta_sec_bytes(int G2) { return (40 * G2 + 15) & ~15; }
constexpr size_t kMaxLds = 65536;   // dynamic LDS a kernel launch may ask for

// The decode down kernel runs a wave per routed expert of a token.
constexpr int kDownMaxK = 8;

// LDS bytes of the W4A16 decode kernels.
// Phase-1 cross-wave reduction buffer of one slice: [NW waves][gate,up][64][4] f32.
__host__ __device__ constexpr int p1_red_bytes(int NW) { return NW * 2 * 64 * 4 * 4; }
__host__ __device__ inline size_t w4_p1_lds_bytes(int H, int xrows, int slices, int NW = 4) {
  return (size_t)slices * (p1_red_bytes(NW) + 80 * (H >> 7)) + (size_t)xrows * H * 2;
}
// W4A16 decode gate_up: up to this many routed pairs the K split is 8 waves.
constexpr int kW4WideMaxPairs = 8;
// Waves of a W4A16 decode gate_up workgroup for n routed pairs at hidden size H.
// (8 only where its larger reduction buffer leaves room for one hidden row).
inline int w4_p1_waves(int64_t n, int H) {
  return (n <= kW4WideMaxPairs && (H / 128) % 8 == 0 && w4_p1_lds_bytes(H, 1, 1, 8) <= kMaxLds) ? 8 : 4;
}
__host__ __device__ inline size_t w4_down_token_lds_bytes(int I, int K, int RT) {
  return (size_t)K * I * 2 + (size_t)K * RT * w2_meta_sec_bytes(I >> 7) + (size_t)K * 16 * RT * 4 + (size_t)K * 4;
}

// Launch geometry of the W4A16 kernels (see w4a16_plan).
struct W4Plan {
  int nb1, s1;    // phase 1: groups per load batch, 16-row slices per workgroup
  int nb2, rt2;   // down: groups per load batch, 16-row tiles per wave
};

// Q8_0 / Q4_0 fused kernel (qint.hip).
struct QArgs {
  SchedArgs c;
  const void* w13;         // [E][I/32 tiles][H/32 blocks][chunks][64 lanes][16 B]
  const uint16_t* w13_d;   // [E][I/32][H/32][64]
  const void* w2;          // [E][H/64 tiles][I/32 blocks][chunks][64][16 B]
  const uint16_t* w2_d;    // [E][H/64][I/32][64]
  int8_t* act_q;           // [n, I] intermediate Q8_0 bytes, row = pair
  float* act_d;            // [n, I/32] intermediate Q8_0 scales
  const int8_t* xq;        // [T, H] Q8_0 activations (grouped GEMM path)
  const float* xd;         // [T, H/32]
};

}  // namespace mimoe
