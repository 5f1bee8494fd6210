// cpu_moe.hpp -- host (CPU) engine of the Q8_0 / Q4_0 fused MoE layer: the
// reference CPU algorithm (moe_forward_ptr_impl, Int8-gemm/q8_gemm.cpp:276-646)
// on x86 cores with VNNI / AVX2 int8 dot products, tp shards over NUMA nodes.
// Plain C++ (no HIP); bound by the mi_moe_cpu_* entry points of the C ABI.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "worker_pool.hpp"

#include <atomic>
#include <condition_variable>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

namespace mimoe_cpu {

// fp16 (dt 0) / bf16 (dt 1) bits -> fp32, exact
float half_to_f32(uint16_t v, int dt);
// Router top-k + softmax on host cores: the device kernel's picks (strictly
// larger logit first, equal logits the lower id) and weights (float exp of the
// Cody-Waite routine the device uses, summed in float in pick / expert order),
// bit-equal to the device kernel for non-NaN logits.
void topk_softmax(const float* logits, int64_t T, int64_t E, int64_t K, int renormalize, int32_t* ids,
                  float* w);

// Q8_0 of n values (n % 32 == 0) into q, q ^ 0x80, block scales d and int32
// block sums s: a hidden row of fp16 / bf16 bits (Stage A), or SiLU(gate) * up
// (the intermediate).  simd picks the AVX2 + FMA form (same bytes and scales).
void quant_hidden_row(bool simd, const uint16_t* x, int64_t n, int dt, int8_t* q, uint8_t* qb, float* d, int32_t* s);
void quant_act_row(bool simd, const float* gate, const float* up, int64_t n, int8_t* q, uint8_t* qb, float* d,
                   int32_t* s);

// Row helpers of the W4A16 host executor, AVX2 + FMA where the host has it
// (the scalar forms give the same bits): out = up * SiLU(gate) with the exp
// of the device code; sums of 128-element groups (a fixed lane tree);
// fp16 / bf16 bits -> fp32.
bool host_simd();
void silu_mul_row(const float* gate, const float* up, int64_t n, float* out);
void group_sums_128(const float* a, int64_t ngroups, float* sums);
void half_row_to_f32(const uint16_t* x, int64_t n, int dt, float* out);

enum class Isa : int { kScalar = 0, kAvx2 = 1, kAvxVnni = 2, kAvx512Vnni = 3 };
Isa detect_isa();               // the widest form the host runs
bool isa_supported(Isa i);
const char* isa_name(Isa i);

constexpr int kNR = 16;       // weight rows per panel
constexpr int kMBlock = 32;   // routed rows per task (M_BLOCK, Int8-gemm/q8_gemm.cpp:335)

// One weight matrix (N rows x K, N % 16 == 0, K % 32 == 0) in 16-row panels.
struct PackedMat {
  int qt = 0;
  int64_t N = 0, K = 0, blk = 0;
  std::vector<uint8_t> qs;   // [N/16][K/32][blk]
  std::vector<float> d;      // [N/16][K/32][16]
  std::vector<int32_t> ws;   // Q8_0: [N/16][K/32][16] = 128 * sum of the block's weights
  void init(int qt, int64_t N, int64_t K);
  void set_row(int64_t n, const int8_t* w, const float* dw);   // values (Q4_0: n - 8) and block scales
};

// The host's CPUs as used: affinity size, NUMA nodes among them, and the
// CPUs chosen (at most max_threads, whole nodes first) grouped by node.
struct Topology {
  int affinity_cpus = 0, affinity_nodes = 0;
  std::vector<int> node_ids;
  std::vector<std::vector<int>> node_cpus;
};
Topology host_topology(int max_threads);

// A pool of threads pinned to the given CPUs; run(n, f) calls f(i) for
// i < n on the workers and the caller, dynamically.  One run at a time.
class NodePool {
 public:
  explicit NodePool(const std::vector<int>& cpus);
  NodePool(const NodePool&) = delete;
  NodePool& operator=(const NodePool&) = delete;
  int size() const { return pool_->size(); }
  void run(int64_t n, const std::function<void(int64_t)>& f) { pool_->run(n, f); }
  void pin(int i);   // pin the calling thread to CPU i of the pool

 private:
  std::vector<int> cpus_;
  std::unique_ptr<mimoe_pool::WorkerPool> pool_;
};

class Engine {
 public:
  // max_threads 0: every CPU of the affinity mask; tp 0: one shard per NUMA
  // node holding chosen CPUs.
  Engine(int64_t E, int64_t H, int64_t I, int quant, int max_threads, int tp);
  // The reference's NUMA layout (Int8-gemm/moe_infer.cpp:25-36,
  // numa_threadpool.h:498-504): tp shards (0: one per NUMA node of the
  // affinity mask), shard s on node s with threads_per_node of its CPUs (0:
  // all).  With fewer nodes than tp the affinity CPUs are split into tp
  // groups in order, each cut to threads_per_node.
  struct NumaLayout {};
  Engine(int64_t E, int64_t H, int64_t I, int quant, NumaLayout, int tp, int threads_per_node);
  ~Engine();
  bool shape_ok() const;
  // wire layout of store_quantized_weights_repack (Int8-gemm/moe_infer.cpp:96-282)
  void store(const void* gate_up_qs, const uint16_t* gate_up_d, const void* down_qs, const uint16_t* down_d,
             int scale_dtype);
  // one projection (0 gate [I,H], 1 up [I,H], 2 down [H,I]) of expert e, fp32 values
  void quantize_and_store(int64_t e, int proj, const float* w);
  // y [T,H] in act_dtype; or, with y_f32, the fp32 sums before the cast
  // (Stage C2 without its rounding) into y_f32 and y unused.  Calls on one
  // engine run one at a time (its buffers and pools are shared).
  int forward(const uint16_t* x, uint16_t* y, const float* topk_w, const int32_t* topk_ids, int64_t T, int64_t K,
              int act_dtype, float* y_f32 = nullptr);
  bool loaded() const { return loaded_; }
  int threads() const { return threads_; }
  int tp() const { return tp_; }
  Isa isa() const { return isa_; }
  void set_isa(Isa i) { isa_ = i; }
  // Largest number of parts a task is cut into: 2 (default) is the
  // reference's split (two parts when tasks * 2 <= threads); more lets few
  // routed experts keep every thread busy (same results).
  void set_split_max(int p) { split_max_ = p < 2 ? 2 : p; }
  double last_ms() const { return last_ms_; }
  const Topology& topology() const { return topo_; }
  int64_t E() const { return E_; }
  int64_t H() const { return H_; }
  int64_t I() const { return I_; }
  int quant() const { return qt_; }

 private:
  struct Shard {
    std::vector<PackedMat> w13, w2;   // per expert: [gate shard | up shard] rows x H; H rows x shard
  };
  // Per-shard buffers of a call, kept between calls (they only grow), so a
  // call allocates no large blocks: Stage A rows, gate_up outputs, the
  // intermediate's Q8_0, the expert outputs.
  struct Scratch {
    std::vector<int8_t> xq, aq;
    std::vector<uint8_t> xb, ab;
    std::vector<float> xd, ad, inter, eout;
    std::vector<int32_t> xs, as;
    std::vector<int8_t> ga;       // routed rows of the Stage-A activations, sorted order
    std::vector<uint8_t> gab;
    std::vector<float> gad;
    std::vector<int32_t> gas;
  };
  int64_t E_, H_, I_;
  int qt_;
  Isa isa_;
  Topology topo_;
  int tp_ = 1, threads_ = 1;
  std::vector<std::unique_ptr<NodePool>> pools_;
  std::vector<Shard> shards_;
  std::vector<Scratch> scratch_;
  std::vector<float> part_;   // [tp][T][H] shard partials
  std::mutex call_mu_;        // forward calls, one at a time
  bool loaded_ = false;
  int split_max_ = 2;
  double last_ms_ = -1.0;
};

}  // namespace mimoe_cpu
