// mi_moe_internal.hpp -- structures shared by the kernels and the C-ABI host
// code of libmimoe.so.  Not part of the public ABI (include/mi_moe.h is).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimoe {

// Routing done inside the fused kernel (LDS) up to this many (t,k) pairs;
// beyond it a separate routing kernel writes the arrays to the workspace.
constexpr int kRouteLdsMax = 1024;
// Columns (routed rows of one expert) handled per register pass.
constexpr int kColsPerPass = 64;

// Workspace control words (uint32 indices into Workspace::ctl).
enum { CTL_TICKET = 0, CTL_EXIT = 1, CTL_ERROR = 2, CTL_WORDS = 8 };

// Routing arrays written by the standalone routing kernel (global path).
struct RouteGlobal {
  int32_t* counts;   // [E]
  int32_t* starts;   // [E+1]
  int32_t* active;   // [E]
  int32_t* tok;      // [n]
  int32_t* scat;     // [n]
  int32_t* U;        // [1]
};

// Arguments of the fused W4A16 kernel (passed by value).
struct W4Args {
  const uint16_t* x;       // [T,H] act dtype bits
  uint16_t* y;             // [T,H]
  const float* tw;         // [T,K]
  const int32_t* ids;      // [T,K]
  int T, K, E, H, I, n;
  int route_global;
  RouteGlobal rg;
  // weights (device tile layout, see w4a16 kernels)
  const void* w13;         // uint4 tiles
  const uint16_t* w13_s;   // [tile][g][16]
  const uint16_t* w13_z;   // [tile][g][4]  (u16 per row quartet)
  const void* w2;
  const uint16_t* w2_s;
  const uint16_t* w2_z;
  // workspace
  uint32_t* ctl;           // control words
  uint32_t* done1;         // [E] phase-1 completions per expert
  uint32_t* cnt2;          // [T * (H/64)] combine arrivals
  uint16_t* act;           // [n, I] SiLU*mul activations (act dtype)
  float* eout;             // [n, H] per-(t,k) expert outputs
};

}  // namespace mimoe
