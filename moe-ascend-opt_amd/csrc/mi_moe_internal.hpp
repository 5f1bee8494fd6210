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
// Q8_0 / Q4_0: up to this many routed pairs the lane-per-row kernels run,
// above it the int8 grouped GEMMs (the measured crossover on the H=2048,
// E=128, I=512/768 layers, top-8 and top-10: a Q4_0 weight byte holds two
// values, so its lane-per-row dots stay ahead of the GEMMs' per-block VALU
// scaling to more pairs than Q8_0's).
inline int q_lpr_max_pairs(int quant) { return quant == 1 ? 160 : 96; }
// Q8_0 / Q4_0 lane-per-row gate_up: up to this many routed pairs the work
// items are pairs routed by ballots over all ids (one per 64 ids; grid =
// pairs x slices).
constexpr int kQBallotMaxPairs = 192;
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
  unsigned long long* tact;    // one-launch decode: tagged act units (tagged_act_bytes(I))
};

// Bytes of the w2 metadata of one 16-row tile: G2 = I/128 groups of 16 u16
// scales and 8 bytes of zero nibbles, rounded up to 16 bytes.
__host__ __device__ inline int w2_meta_sec_bytes(int G2) { return (40 * G2 + 15) & ~15; }
// LDS a launch may ask for without opting in (hipFuncSetAttribute), and the
// most a workgroup may use on the current device
// (hipDeviceAttributeMaxSharedMemoryPerBlock, queried once per device; 64 KB
// if the query fails).  Path choices test the layer's LDS needs against the
// latter.
constexpr size_t kMaxLds = 65536;
size_t device_max_lds();

// The decode down kernel runs a wave per routed expert of a token.
constexpr int kDownMaxK = 16;

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

// One-launch W4A16 decode kernel (w4a16_fused.hip): 8-wave workgroups; gate_up
// items take 8 / NW slices of 16 rows of I with NW waves splitting H each, down
// items a wave per routed expert (top-k <= 8).
constexpr int kW4FusedWaves = 8;
// The one-launch kernel serves the whole decode path (up to 64 routed pairs,
// top-k <= 8); the two-launch kernels serve top-k 9-16.
constexpr int kW4FusedMaxPairs = 64;
// Its hand-over buffer (per handle, and the head of the no-alloc scratch):
// u64 units [64 pairs][I/2] of (dispatch tag << 32 | two act values), then
// one u64 that records a wait that gave up.  A unit is valid for a call iff
// it carries that dispatch's tag, so the buffer is never cleared; it starts
// zeroed (no dispatch has tag 0).  The one-launch kernel serves I <= kTagActMaxI.
constexpr int kTagActMaxI = 4096;
__host__ __device__ constexpr size_t tagged_act_bytes(int I) { return (size_t)64 * I * 4 + 64; }
// red [2][S][...] (double-buffered: a unit's sums while the previous unit's
// epilogue reads its own) | metadata [S][80*G1] | hidden rows
inline size_t w4_fused_gate_up_lds_bytes(int H, int xrows, int NW) {
  return (size_t)(kW4FusedWaves / NW) * (2 * p1_red_bytes(NW) + 80 * (H >> 7)) + (size_t)xrows * H * 2;
}
// act rows [8][I] | w2 metadata [8][RT][SEC] | outputs [8][16 RT] f32 |
// state [8] | routing weights [8] f32
inline size_t w4_fused_down_lds_bytes(int I, int RT) {
  return (size_t)kW4FusedWaves * ((size_t)I * 2 + (size_t)RT * (w2_meta_sec_bytes(I >> 7) + 16 * 4) + 8);
}
struct W4FusedPlan {
  int ok;          // the one-launch kernel serves the call
  int nw, njs;     // gate_up: waves splitting H per slice (8 or 4), slice blocks per item
  int nb1, nb2;    // load batches (groups) of the gate_up and down roles
  int rt;          // 16-row tiles of H per down item (1 or 2)
  int ngu;         // gate_up workgroups (each takes every ngu-th item)
  size_t lds;
};

// W4A16 decode path: both kernels fit in `lds` bytes (phase 1 with one token
// column per pass).
inline bool w4_decode_fits(int H, int I, int K, size_t lds) {
  return w4_p1_lds_bytes(H, 1, 1, 4) <= lds && w4_down_token_lds_bytes(I, K, 1) <= lds;
}

// W4A16 grouped GEMMs (sorted path): 64-row tiles staged with a 272-byte row
// stride (256 B of a 128-group + 16 B that spread the rows over the LDS
// banks), double-buffered, with the row sums and pair indices; gate_up takes
// kGemm13Blocks blocks of 4 slices, down kGemm2Quads quads of 64 rows of H,
// and each stages the workgroup's metadata for all of K.
constexpr int kGemmRowStride = 272;
constexpr int kGemmABytes = kGemmRows * kGemmRowStride;
constexpr size_t kGemmLds = 2 * (size_t)kGemmABytes + 3 * kGemmRows * sizeof(float);
constexpr int kGemm13Blocks = 2;
constexpr int kGemm2Quads = 4;
inline size_t w4_gemm13_lds_bytes(int H) { return kGemmLds + (size_t)4 * kGemm13Blocks * 80 * (H >> 7); }
inline size_t w4_gemm2_lds_bytes(int I) { return kGemmLds + (size_t)kGemm2Quads * 4 * w2_meta_sec_bytes(I >> 7); }
inline bool w4_sorted_fits(int H, int I, size_t lds) {
  return (H / 64) % kGemm2Quads == 0 && (I / 64) % kGemm13Blocks == 0 && w4_gemm13_lds_bytes(H) <= lds &&
         w4_gemm2_lds_bytes(I) <= lds;
}

// Launch geometry of the W4A16 kernels (see w4a16_plan).
struct W4Plan {
  int nb1, s1;    // phase 1: groups per load batch, 16-row slices per workgroup
  int nb2, rt2;   // down: groups per load batch, 16-row tiles per wave
};

// Q8_0 / Q4_0 lane-per-row kernels: LDS of the phase kernels for a K range
// of Kmax (kQTokPerPass tokens' activation bytes, scales and byte sums, and
// the cross-wave partials of up to kQDecWavesMax waves), plus the routing
// arrays when they live in LDS; the token-major down kernel's LDS: act bytes
// [K][I] | act d [K][I/32] | act byte sums [K][I/32] | quarter partials
// [K][64] | outputs [K][16] | valid [K].
constexpr int kQDecWavesMax = 8;
__host__ __device__ inline size_t q_stage_bytes(int Kmax) {
  return (size_t)kQTokPerPass * Kmax + (size_t)kQTokPerPass * (Kmax / 32) * 8 +
         (size_t)kQDecWavesMax * kQTokPerPass * 64 * 4;
}
__host__ __device__ inline size_t q_down_token_lds_bytes(int I, int K) {
  return (size_t)K * I + (size_t)K * (I / 32) * 8 + (size_t)K * 64 * 4 + (size_t)K * 16 * 4 + (size_t)K * 4;
}
__host__ __device__ inline size_t route_lds_ints(int E, int n) { return (size_t)3 * E + 1 + 2 * (size_t)n; }
// LDS of the routing arrays of the lane-per-row kernels for n routed pairs
// (at least the ballot path's 64-entry pair list).
inline size_t q_route_lds_bytes(int E, int n) {
  const size_t r = n > kRouteLdsMax ? 0 : route_lds_ints(E, n) * sizeof(int);
  return r < 64 * sizeof(int) ? 64 * sizeof(int) : r;
}
// The lane-per-row path fits for n routed pairs (token_down: the down
// projection token-major, the combine fused; else expert-major phase 2).
inline bool q_lpr_fits(int H, int I, int E, int n, int K, bool token_down, size_t lds) {
  const size_t route = q_route_lds_bytes(E, n);
  if (q_stage_bytes(H) + route > lds) return false;
  return token_down ? q_down_token_lds_bytes(I, K) <= lds : q_stage_bytes(I) + route <= lds;
}
// The int8 grouped GEMMs (any n) need H and I multiples of 128.
inline bool q_gemm_ok(int H, int I) { return H % 128 == 0 && I % 128 == 0; }

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
  unsigned long long* tact;   // tagged intermediate units of the one-launch decode kernel
};

// One-launch Q8_0 / Q4_0 decode kernel (qint.hip): 8-wave workgroups, gate_up
// items (pair, 32-row slice of I) for calls of up to kQDecWideMaxPairs routed
// pairs, down items (token, 16-row tile of H) with a wave per routed expert
// (top-k <= 8).  The intermediate Q8_0 row of a pair travels as q_tag_units(I)
// tagged units in the hand-over buffer: I/4 units of 4 bytes, then I/32 units
// of the blocks' fp32 scales (within tagged_act_bytes(I), whose last unit
// records a wait that gave up).
constexpr int kQFusedWaves = 8;
constexpr int kQFusedMaxPairs = 12;
__host__ __device__ constexpr int q_tag_units(int I) { return I / 4 + I / 32; }
// The gate_up workgroups split K in two; the first half's gate and up sums
// travel as units [pair][I/32 slices][64 rows] after the rows of
// kQFusedMaxPairs pairs, below the timeout unit (64 * I/2).
__host__ __device__ constexpr size_t q_part_unit0(int I) { return (size_t)kQFusedMaxPairs * q_tag_units(I); }
static_assert(q_part_unit0(32) + (size_t)kQFusedMaxPairs * 2 * 32 <= (size_t)32 * 32, "Q units fit the buffer");
static_assert(q_part_unit0(kTagActMaxI) + (size_t)kQFusedMaxPairs * 2 * kTagActMaxI <= (size_t)32 * kTagActMaxI,
              "Q units fit the buffer");
// LDS of a down item: act bytes [8][I] | act d [8][I/32] | act byte sums
// [8][I/32] | quarter partials [8][64] | outputs [8][16] | state [8] |
// routing weights [8].
__host__ __device__ inline size_t q_fused_down_lds_bytes(int I) {
  return (size_t)kQFusedWaves * (I + (I / 32) * 8 + 64 * 4 + 16 * 4 + 8);
}

}  // namespace mimoe
