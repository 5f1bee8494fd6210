// w4a16_device.hpp -- device helpers shared by the W4A16 kernels
// (w4a16.hip: two-launch decode, grouped GEMMs, repack; w4a16_fused.hip: the
// one-launch decode kernel): the MFMA wrapper, the int4 dequantization, the
// zero/scale fold, direct-to-LDS staging and the wait/barrier primitives.
#pragma once
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
  static constexpr uint32_t one2 = ACT == 1 ? 0x3f803f80u : 0x3c003c00u;
};

// 8 nibbles of a word -> 8 values (magic + nibble): value pair p holds the
// nibbles at bits 4p and 16 + 4p.  The mask and the magic are made opaque
// (empty asm, no instruction) so they sit in an SGPR and a VGPR and each pair
// is one v_and_or_b32: VOP3 on gfx9 takes no literal, so with the constants
// visible the compiler emits a separate and and or.
template <int ACT>
__device__ __forceinline__ u32x4_t deq4(uint32_t w) {
  uint32_t m = 0x000f000fu, c = W4Consts<ACT>::magic;
  asm("" : "+s"(m));
  asm("" : "+v"(c));
  u32x4_t a;
  a.x = (w & m) | c;
  a.y = ((w >> 4) & m) | c;
  a.z = ((w >> 8) & m) | c;
  a.w = ((w >> 12) & m) | c;
  return a;
}

template <int ACT>
__device__ __forceinline__ u32x4_t ones4() {
  const uint32_t o = W4Consts<ACT>::one2;
  return u32x4_t{o, o, o, o};
}

__device__ __forceinline__ u32x4_t ldg16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ u32x4_t lds16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ u32x4_t zero4() { return u32x4_t{0, 0, 0, 0}; }

__device__ __forceinline__ uint64_t bits_range(int lo, int count) {
  const uint64_t m = count >= 64 ? ~0ull : ((1ull << count) - 1);
  return m << lo;
}

// Scale bits -> fp32 with the scale dtype fixed at compile time (1 bf16, 0 fp16).
template <int SDT>
__device__ __forceinline__ float scale_of(uint32_t bits) {
  if constexpr (SDT == 1) return bf16_to_f32(bits);
  else return f16_to_f32(bits);
}

// acc[t] += s * (G[t] - c * X[t]) for the lane's 4 token columns
__device__ __forceinline__ void fold(f32x4_t& acc, const f32x4_t G, const f32x4_t X, float s,
                                     float c) {
  acc.x = __builtin_fmaf(s, __builtin_fmaf(-c, X.x, G.x), acc.x);
  acc.y = __builtin_fmaf(s, __builtin_fmaf(-c, X.y, G.y), acc.y);
  acc.z = __builtin_fmaf(s, __builtin_fmaf(-c, X.z, G.z), acc.z);
  acc.w = __builtin_fmaf(s, __builtin_fmaf(-c, X.w, G.w), acc.w);
}

// Copy nitems 16-byte items into LDS (contiguous from dst, 16-byte aligned)
// with direct-to-LDS loads (global_load_lds_dwordx4): wave instruction s moves
// items 64s..64s+63, lane l landing at dst + 1024s + 16l; instructions are
// dealt round-robin to the nwaves waves of the workgroup.  src(k) is evaluated by every lane of a
// participating wave (it may shuffle).  The caller waits for vmcnt and
// barriers before reading the copy.
template <class Src>
__device__ __forceinline__ void stage_lds(unsigned char* dst, int nitems, int wave, int nwaves,
                                          int lane, Src src) {
  for (int s = wave; s * 64 < nitems; s += nwaves) {   // uniform per wave
    const int k = s * 64 + lane;
    const void* p = src(k < nitems ? k : nitems - 1);
    if (k < nitems) __builtin_amdgcn_global_load_lds(p, dst + s * 1024, 16, 0, 0);
  }
}

// Wait until at most N vector-memory loads of this wave are outstanding, then
// barrier.  With the direct-to-LDS copies issued before the N weight loads
// (vector loads complete in order), this waits for the copies only; the
// weights are waited for one by one where they are used.
template <int N>
__device__ __forceinline__ void wait_copies_and_sync() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
  // a bare barrier: __syncthreads() would add fences that wait for every load
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Keeps the compiler from moving memory operations across this point (the
// weight loads must be issued after the direct-to-LDS copies).
__device__ __forceinline__ void issue_order_fence() { asm volatile("" ::: "memory"); }

// Zero point of a (16 row x 128 k) group of one w2 row tile: a metadata
// section holds scales u16 [g2][r], then zeros [g2][r/2] (row r in nibble r&1).
__device__ __forceinline__ float w2_zero(const unsigned char* sec, int G2, int g2, int r) {
  return (float)((sec[32 * G2 + 8 * g2 + (r >> 1)] >> (4 * (r & 1))) & 0xfu);
}

}  // namespace mimoe
