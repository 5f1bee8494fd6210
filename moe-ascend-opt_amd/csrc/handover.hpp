// handover.hpp -- the in-launch hand-over of the one-launch decode kernels
// (w4a16_fused.hip, qint.hip): producer workgroups write 8-byte units
// (dispatch tag << 32 | 32-bit payload) with agent-scope coherent stores
// (global_store ... sc1: written through, never left dirty in one XCD's L2),
// consumer workgroups placed after every producer in the grid poll them with
// agent-scope coherent loads.  A unit is valid for a call iff it carries that
// dispatch's tag: nothing is cleared between calls, there are no atomics, no
// flags and no L2 write-back or invalidate, and a producer never waits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimoe {

constexpr int kSpinMax = 1 << 18;   // polls of one wait (each at least one memory round trip)

__device__ __forceinline__ unsigned long long load_agent(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void store_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The AQL packet index of this dispatch (llvm.amdgcn.dispatch.id: SGPRs the
// command processor fills at launch).
extern "C" __device__ unsigned long long mimoe_llvm_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

// 32-bit tag of this dispatch: the packet index plus a multiple of the
// queue's address (odd, so never 0, the value of a cleared unit).  A unit
// written by an earlier dispatch on the same queue matches only after 2^31
// more dispatches.
__device__ __forceinline__ unsigned dispatch_tag32() {
  const unsigned long long q = (unsigned long long)(uintptr_t)__builtin_amdgcn_queue_ptr();
  return ((unsigned)mimoe_llvm_dispatch_id() * 2u + (unsigned)(q >> 12) * 0x9E3779B2u) | 1u;
}

}  // namespace mimoe
