// host_experts.hpp -- the host (CPU) half of the hybrid offload executor:
// experts whose weights stay in host memory ("cold" experts) run here, on a
// fixed pool of host threads, from the wire-format bytes the caller stored.
//
// Arithmetic per format (the reference CPU algorithm for Q8_0 / Q4_0,
// Int8-gemm/q8_gemm.cpp:276-646, with tp = 1):
//   Q8_0 / Q4_0  x rows -> Q8_0 blocks (fp32 d); gate_up rows c += (isum*dw)*da
//                over the 32-blocks in order; SiLU(gate)*up; the intermediate
//                -> Q8_0; down rows likewise; weighted sum over k in order.
//   W4A16        fp32: y = sum_g s[g,n] * (sum_{k in g} x_k q_kn - z[g,n] sum_{k in g} x_k)
//                per 128-group, SiLU(gate)*up in fp32, down likewise.
// No HIP calls: this file is plain C++ and runs inside a stream host callback.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "worker_pool.hpp"

#include <atomic>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace mimoe_host {

// A fixed set of worker threads.  run(n, f) calls f(i) for every i in [0, n)
// on the workers and the calling thread and returns when all calls are done.
// One run at a time per pool.
using Pool = mimoe_pool::WorkerPool;

// Number of weight arrays of a format (Q8_0 / Q4_0: gate_up_qs, gate_up_d,
// down_qs, down_d; W4A16: w13_q, w13_z, w13_s, w2_q, w2_z, w2_s) and the
// bytes one expert takes in array idx of the wire layout.
int num_arrays(int quant);
size_t expert_bytes(int quant, int64_t H, int64_t I, int idx);

// Wire-format weights of the cold experts: arr[a] holds array a of cold
// expert c at c * expert_bytes(quant, H, I, a) (W4A16: the two qweight
// arrays are released once prepare_host_layouts has copied them).
struct ColdSet {
  int quant = 0;        // 0 Q8_0, 1 Q4_0, 2 W4A16 (group 128)
  int scale_dtype = 0;  // 0 fp16, 1 bf16
  int64_t E = 0, H = 0, I = 0, Ec = 0;
  std::vector<int32_t> cold_of;   // [E]: cold index of expert e, or -1
  std::vector<uint8_t> arr[6];
  // W4A16 (prepare_host_layouts; empty unless H % 128 == I % 128 == 0):
  // the qweight arrays again in 128-column blocks, each block's k rows one
  // contiguous run of 64-byte rows, bq13 [Ec][2I/128][H][16] and
  // bq2 [Ec][H/128][I][16] words, so that a task streams one run.
  std::vector<int32_t> bq13, bq2;
  // And gate_up in the k-pair order of the AVX512-BF16 kernel (also empty
  // when the host lacks the instructions):
  //   pq [Ec][2I/64][H/2][16] u32 (64-column blocks, each one contiguous
  //      run): word (b, kp, i) holds, for s = 0..3, the nibble of
  //      (k = 2kp, n = 64b + 4i + s) at bits 4s and of (k = 2kp + 1, same n)
  //      at bits 16 + 4s;
  //   pz [Ec][H/128][2I] zero nibbles and ps [Ec][H/128][2I] scale bits, in
  //      lane order: column n = 64b + 4i + s at index 64b + 16s + i.
  std::vector<uint32_t> pq;
  std::vector<uint8_t> pz;
  std::vector<uint16_t> ps;
};

// Fills the block-major and k-pair copies of a W4A16 ColdSet from its wire
// arrays (all six stored), then releases arr[0] and arr[3]; a no-op for
// other formats.
void prepare_host_layouts(ColdSet& cs);

// y_part [T,H] fp32: per token, the sum over k in ascending order of
// topk_w[t,k] * expert(x[t]) over the pairs whose id is a cold expert (rows
// of tokens without such a pair are 0).  x [T,H] fp16/bf16 bits (act_dtype
// 0/1).  Returns the number of cold pairs.
int64_t forward(const ColdSet& cs, Pool& pool, const uint16_t* x, int act_dtype, const int32_t* ids,
                const float* topk_w, int64_t T, int64_t K, float* y_part);

}  // namespace mimoe_host
