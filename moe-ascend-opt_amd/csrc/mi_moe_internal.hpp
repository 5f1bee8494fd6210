// mi_moe_internal.hpp -- structures shared by the kernels and the C-ABI host
// code of libmimoe.so.  Not part of the public ABI (include/mi_moe.h is).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimoe {

// Routing done inside the fused kernel (LDS) up to this many (t,k) pairs;
// beyond it a separate routing kernel writes the arrays to the workspace.
constexpr int kRouteLdsMax = 1024;
// Columns (routed rows of one expert) handled per register pass (W4A16).
constexpr int kColsPerPass = 64;
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
};

// Arguments every fused kernel shares (routing, schedule, combine).
struct SchedArgs {
  const uint16_t* x;       // [T,H] act dtype bits
  uint16_t* y;             // [T,H]
  const float* tw;         // [T,K]
  const int32_t* ids;      // [T,K]
  int T, K, E, H, I, n;
  int route_global;
  RouteGlobal rg;
  uint32_t* cnt2;          // [T * (H/64)] combine arrivals
  float* eout;             // [n, H] per-(t,k) expert outputs
};

// W4A16 fused kernel (w4a16.hip).
struct W4Args {
  SchedArgs c;
  const void* w13;         // uint4 tiles
  const uint16_t* w13_s;   // [tile][g][16]
  const uint16_t* w13_z;   // [tile][g][4]  (u16 per row quartet)
  const void* w2;
  const uint16_t* w2_s;
  const uint16_t* w2_z;
  uint16_t* act;           // [n, I] SiLU*mul activations (act dtype)
};

// Q8_0 / Q4_0 fused kernel (qint.hip).
struct QArgs {
  SchedArgs c;
  const void* w13;         // [E][I/32 tiles][H/32 blocks][chunks][64 lanes][16 B]
  const uint16_t* w13_d;   // [E][I/32][H/32][64]
  const void* w2;          // [E][H/64 tiles][I/32 blocks][chunks][64][16 B]
  const uint16_t* w2_d;    // [E][H/64][I/32][64]
  int8_t* act_q;           // [n, I] intermediate Q8_0 bytes
  float* act_d;            // [n, I/32] intermediate Q8_0 scales
};

}  // namespace mimoe
