/*
 * mi_moe.h -- C ABI of the MI355X fused-MoE expert library (libmimoe.so).
 *
 * Plain C: opaque handle, raw device pointers, sizes, an int status and a
 * thread-local error string.  No torch types cross this boundary.  Each entry
 * point names the reference interface it replaces (paths relative to the
 * reference checkout).
 *
 * Streams are passed as void* (a hipStream_t; NULL = the default stream).
 * All data pointers given to mi_moe_forward* must be device memory on the
 * device the handle was created on.  Loader entry points accept either host
 * or device memory (flag src_on_device).
 */
#ifndef MI_MOE_H
#define MI_MOE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MI_MOE_OK 0
#define MI_MOE_EINVAL 1      /* bad argument / shape / dtype */
#define MI_MOE_ENOTLOADED 2  /* forward before weights were stored */
#define MI_MOE_EUNSUPPORTED 3
#define MI_MOE_EHIP 4        /* a HIP runtime call failed */
#define MI_MOE_EDEVICE 5     /* a kernel reported an error (e.g. bounded wait expired) */

/* quant types: 0/1 as Int8-gemm/quant_traits.h:7-10 (Python ints 0/1); 2 is
 * the W4A16 AWQ-style format of the absent NPU grouped_gemv path. */
#define MI_MOE_Q8_0 0
#define MI_MOE_Q4_0 1
#define MI_MOE_W4A16 2

/* dtype codes for activations and scales (and router logits, which may also
 * be MI_MOE_F32) */
#define MI_MOE_F16 0
#define MI_MOE_BF16 1
#define MI_MOE_F32 2

typedef struct mi_moe_handle mi_moe_handle;

/* Thread-local message for the last non-zero status of this thread. */
const char* mi_moe_last_error(void);

/* Library/ABI version (major*10000 + minor*100 + patch). */
int mi_moe_version(void);

/* Create a handle for E experts, hidden H, intermediate I.
 * Replaces MoEInfer::MoEInfer (Int8-gemm/moe_infer.cpp:18-75) and the
 * TorchBind constructor MoEInfer(E,H,I,quant_type)
 * (Int8-gemm/nanovllm_ops.cpp:28-30,353).  Requires H%32==0, I%32==0
 * (W4A16: H%512==0, I%128==0).  Allocates nothing on the device until weights
 * are stored; uses the current HIP device. */
int mi_moe_create(int64_t num_experts, int64_t hidden, int64_t intermediate,
                  int quant_type, mi_moe_handle** out);

/* Free all device memory of the handle.  Replaces MoEInfer::~MoEInfer
 * (Int8-gemm/moe_infer.cpp:77-84). */
int mi_moe_destroy(mi_moe_handle* h);

/* Shape / type queries (Int8-gemm/nanovllm_ops.cpp:376-391). */
int mi_moe_get_info(const mi_moe_handle* h, int64_t* num_experts,
                    int64_t* hidden, int64_t* intermediate, int* quant_type,
                    int* scale_dtype);

/* Pre-quantized Q8_0 / Q4_0 weights in the caller wire layout -> device
 * layout owned by the handle.  Replaces MoEInfer::store_quantized_weights_repack
 * (Int8-gemm/moe_infer.cpp:96-282), bound as store_quantized_repack
 * (Int8-gemm/nanovllm_ops.cpp:366-371).
 *   Q8_0: gate_up_qs int8 [E,2I,H], down_qs int8 [E,H,I]
 *   Q4_0: gate_up_qs u32 [E,2I,H/8], down_qs u32 [E,H,I/8]
 *   gate_up_d [E,2I,H/32], down_d [E,H,I/32]: fp16 or bf16 (scale_dtype). */
int mi_moe_store_quantized(mi_moe_handle* h, const void* gate_up_qs,
                           const void* gate_up_d, const void* down_qs,
                           const void* down_d, int scale_dtype,
                           int src_on_device, void* stream);

/* Online Q8_0 weight quantization of one projection of one expert.
 * Replaces MoEInfer::quantize_and_store_expert (Int8-gemm/moe_infer.cpp:
 * 284-360; rule of quantize_weight_only, Int8-gemm/q8_gemm.cpp:197-260).
 * proj: 0 = gate_proj [I,H], 1 = up_proj [I,H], 2 = down_proj [H,I];
 * w_dtype: 0 fp16, 1 bf16, 2 fp32.  Q8_0 handles only (the reference rejects
 * Q4_0, Int8-gemm/nanovllm_ops.cpp:359-363).  Scales are stored as fp16. */
int mi_moe_quantize_and_store_expert(mi_moe_handle* h, int64_t expert,
                                     int proj, const void* w, int w_dtype,
                                     int src_on_device, void* stream);

/* W4A16 AWQ-layout weights -> device layout.  No reference counterpart in
 * the checkout: the W4A16 grouped_gemv loader lives in the absent
 * sgl-kernel-npu submodule (README.md:19-30,152).  Layout (AWQ, as
 * nanovllm_moe/formats.py writes it; nibble slot {0,4,1,5,2,6,3,7}[n%8] of
 * each int32): w13_* [E,H,2I/8], [E,H/g,2I/8], [E,H/g,2I] with w13 = gate||up
 * along N; w2_* [E,I,H/8], [E,I/g,H/8], [E,I/g,H].  group must be 128. */
int mi_moe_store_awq(mi_moe_handle* h, const int32_t* w13_qweight,
                     const int32_t* w13_qzeros, const void* w13_scales,
                     const int32_t* w2_qweight, const int32_t* w2_qzeros,
                     const void* w2_scales, int64_t group, int scale_dtype,
                     int src_on_device, void* stream);

/* The fused MoE layer: y[t] = sum_k topk_w[t,k] * Expert_{ids[t,k]}(x[t]).
 * Replaces MoEInfer::ExecuteFn (Int8-gemm/moe_infer.h:51-61) /
 * execute_on_cpu_routed_from_pointers (Int8-gemm/moe_infer.cpp:430-456) and
 * the op body of moe_forward (Int8-gemm/nanovllm_ops.cpp:219-236).
 *   x, y      [T,H] fp16 or bf16 (act_dtype), device
 *   topk_w    [T,K] fp32, device
 *   topk_ids  [T,K] int32, device; ids outside [0,E) are dropped
 *             (Int8-gemm/moe_common.cpp:158,175-181); a token with no valid
 *             id gets y = 0.
 * Stream-ordered and asynchronous.  Calls that overlap on one handle race on
 * its workspace (the reference is likewise not re-entrant).
 * Graph capture: a call can be captured into a HIP graph once the handle's
 * workspace holds it (an earlier call of at least its size, or
 * mi_moe_reserve); decode calls (T*K <= 64, top-k <= 8) need no workspace at
 * all.  Once a call on the handle has been captured, workspace that a later,
 * larger call outgrows is kept until mi_moe_destroy instead of being freed,
 * so captured graphs stay valid through eager calls of any size.  A graph
 * must not outlive its handle. */
int mi_moe_forward(mi_moe_handle* h, const void* x, void* y,
                   const float* topk_w, const int32_t* topk_ids, int64_t T,
                   int64_t K, int act_dtype, void* stream);

/* Size of the device array that holds the workspace of
 * mi_moe_forward_noalloc: 32 MiB per GPU. */
#define MI_MOE_NOALLOC_SCRATCH_BYTES (32u << 20)

/* mi_moe_forward without device memory allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as mi_moe_forward, but the call's
 * workspace (routing arrays, intermediate activations, per-pair outputs) is
 * carved from a static device array of MI_MOE_NOALLOC_SCRATCH_BYTES that each
 * GPU holds from the library's load until the process ends, instead of the
 * handle's grown buffers; it calls no hipMalloc / hipFree and records no
 * timing events.  A call whose workspace exceeds the array returns
 * MI_MOE_EINVAL (decode sizes need well under 1 MiB; at H=2048, I=768 the
 * limit is about 3,000 routed pairs, where the per-pair fp32 outputs
 * dominate).  Every call on a GPU shares that GPU's array and the array keeps
 * the last call's contents (nothing in it has to start at zero): calls that
 * overlap on one GPU, on any handles or streams, race. */
int mi_moe_forward_noalloc(mi_moe_handle* h, const void* x, void* y,
                           const float* topk_w, const int32_t* topk_ids,
                           int64_t T, int64_t K, int act_dtype, void* stream);

/* Wall time of the last timed mi_moe_forward on the handle, in ms, measured
 * with HIP events around its launches (synchronizes on the end event).
 * Replaces MoEInfer::get_last_run_time_ms (Int8-gemm/moe_infer.h:23,
 * Int8-gemm/moe_infer.cpp:439-455).  Timing is off by default (see
 * mi_moe_set_timing); returns a negative value if it is off or no timed call
 * was made. */
double mi_moe_get_last_run_time_ms(mi_moe_handle* h);

/* Enable (1) / disable (0) the per-call HIP-event timing.  Default 0: a
 * forward records no events unless a caller asks for timing, so serving calls
 * pay nothing for it. */
int mi_moe_set_timing(mi_moe_handle* h, int enable);

/* Grow the handle's device workspace to hold a call of T tokens at top_k K
 * (synchronizes `stream` if it grows), so that later calls up to that size
 * allocate nothing and can be captured into a HIP graph.  Replaces the buffer
 * preallocation of MoEGraphContext's constructor
 * (Int8-gemm/nanovllm_ops.cpp:160-201), which sizes the graph-mode op's
 * staging for num_tokens x top_k. */
int mi_moe_reserve(mi_moe_handle* h, int64_t T, int64_t K, void* stream);

/* Per-launch-phase times of the last timed mi_moe_forward, in ms: calls with
 * two launch phases (the W4A16 sorted path and the top-k 9-16 decode path)
 * fill ms[0] = routing + gate_up (+SiLU) launch(es), ms[1] = down (+combine)
 * launch(es) and return 2; the one-launch W4A16 decode kernel and the integer
 * path return 1 (whole call).  mi_moe_forward_noalloc leaves the record of the
 * last timed call unchanged.
 * Synchronizes on the end event.  No counterpart in the reference (its timer
 * covers the whole op); it is the measurement hook behind the per-kernel
 * roofline figures. */
int mi_moe_get_last_phase_times_ms(mi_moe_handle* h, double* ms, int max_phases);

/* Stage A activation quantization alone: x [T,H] fp16/bf16 -> x_qs [T,H]
 * int8, x_d [T,H/32] fp32, with quant_block_q8_0, the device block
 * quantizer the decode kernels' Stage A also calls.  Replaces Stage A of moe_forward_ptr_impl
 * (Int8-gemm/q8_gemm.cpp:360-377; quantize_block_q8_0,
 * Int8-gemm/gemm_kernels.cpp:25-58). */
int mi_moe_quantize_act_q8_0(const void* x, int act_dtype, int64_t T,
                             int64_t H, int8_t* x_qs, float* x_d, void* stream);

/* Routing alone: ids [T,K] -> counts [E], starts [E+1], token_map [T*K]
 * (token id per expert-sorted position; entries past starts[E] unspecified),
 * scatter [T*K] (position or -1).  Replaces preprocess_moe_routing
 * (Int8-gemm/moe_common.cpp:146-216); any top_k >= 1 is accepted. */
int mi_moe_route(const int32_t* topk_ids, int64_t T, int64_t K, int64_t E,
                 int32_t* counts, int32_t* starts, int32_t* token_map,
                 int32_t* scatter, void* stream);

/* Per-32-block int32 dot products of the handle's stored weights against
 * quantized activations, computed by the device block-dot routine of the
 * fused kernels: isum[m][n][kb] for expert e, proj 0 = gate_up [2I rows, K=H],
 * 1 = down [H rows, K=I]; a_qs [M,K] int8 device; isum [M,N,K/32] int32
 * device.  Q8_0 / Q4_0 handles only.  Exposes the inner product of
 * gemm_q{8,4}_0_microkernel (Int8-gemm/gemm_kernels.cpp:102-133,262-309) for
 * bit-exact checking. */
int mi_moe_block_dots(mi_moe_handle* h, int64_t expert, int proj,
                      const int8_t* a_qs, int64_t M, int32_t* isum,
                      void* stream);

/* The same block dots through the int8-MFMA block routine of the grouped
 * GEMMs (the path of Q8_0 / Q4_0 calls above 96 / 160 routed pairs), for bit-exact
 * checking of its two exact rewrites: acc[m][n][kb] int32 = the MFMA result
 * less its 1.5*2^23 bias (Q8_0: isum; Q4_0: 16*isum, the nibbles enter as
 * bytes 16*(n-8)), prod[m][n][kb] fp32 = the first scaled product the GEMMs
 * form from that result read as a float (Q8_0: round(isum*dw); Q4_0:
 * 16*round(isum*dw)).  Shapes as mi_moe_block_dots; needs H and I multiples
 * of 128; a_qs 8-byte aligned.  Counterpart of the integer block dot and the
 * first product of its per-block scaling, (float)isum*dw
 * (Int8-gemm/gemm_kernels.cpp:102-179, 262-358). */
int mi_moe_block_dots_mfma(mi_moe_handle* h, int64_t expert, int proj,
                           const int8_t* a_qs, int64_t M, int32_t* acc,
                           float* prod, void* stream);

/* Router top-k + softmax: logits [T,E] (fp16, bf16 or fp32, device) ->
 * topk_ids [T,K] int32 and topk_w [T,K] fp32 (device), the K largest logits
 * of each token in descending order (equal logits: the lower expert id first)
 * with weights softmax over the K values (renormalize != 0) or the softmax
 * over all E gathered at the ids.  Replaces make_topk_from_logits_cpu
 * (Int8-gemm/test/fused_moe_cpu.py:20-37), the step the reference harness
 * runs before moe_forward.  E <= 512, 1 <= K <= min(E, 64).  Stream-ordered. */
int mi_moe_topk_softmax(const void* logits, int logits_dtype, int64_t T,
                        int64_t E, int64_t K, int renormalize,
                        int32_t* topk_ids, float* topk_w, void* stream);

/* mi_moe_topk_softmax on host memory and host cores: fp32 logits [T,E] ->
 * topk_ids [T,K], topk_w [T,K].  The same picks and weights as the device
 * kernel, bit for bit (non-NaN logits).  Replaces make_topk_from_logits_cpu
 * (Int8-gemm/test/fused_moe_cpu.py:20-37) for the CPU dispatch key. */
int mi_moe_cpu_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t K,
                            int renormalize, int32_t* topk_ids, float* topk_w);

/* Router top-k + softmax followed by mi_moe_forward on the same stream:
 * router_logits [T,E] with E the handle's expert count.  The picks go to
 * topk_ids_out / topk_w_out ([T,K], device) when both are given, else to a
 * buffer the handle owns (grown on demand; growth synchronizes the stream).
 * The reference composes make_topk_from_logits_cpu
 * (Int8-gemm/test/fused_moe_cpu.py:20-37) with moe_forward
 * (Int8-gemm/nanovllm_ops.cpp:219-236) in Python; here it is one call.  The
 * handle's timer (mi_moe_get_last_run_time_ms) covers the forward only. */
int mi_moe_forward_logits(mi_moe_handle* h, const void* x, void* y,
                          const void* router_logits, int logits_dtype,
                          int64_t T, int64_t K, int renormalize,
                          int act_dtype, int32_t* topk_ids_out,
                          float* topk_w_out, void* stream);

/* ------------------------------------------------------------------------
 * Host (CPU) engine of the Q8_0 / Q4_0 layer: the reference's CPU algorithm
 * (moe_forward_ptr_impl, Int8-gemm/q8_gemm.cpp:276-646) on x86 cores.  It is
 * the CPU dispatch key of nanovllm::moe_forward (the reference's only key,
 * Int8-gemm/nanovllm_ops.cpp:410-412) and the CPU baseline of the benchmark.
 * Stage A Q8_0 activations, tasks of 32 routed rows of one expert (2 threads
 * per task -- gate / up rows, then halves of the down rows -- when there are
 * at most half as many tasks as threads), exact int32 block dots, the
 * reference's per-block scaling order, Q8_0 intermediate, combine in k order,
 * tp shards of I over the NUMA nodes of the threads (partials summed in shard
 * order).  All pointers are host memory; calls are synchronous.  The
 * MoEInfer counterpart for this path is Int8-gemm/moe_infer.cpp:18-84. */
typedef struct mi_moe_cpu mi_moe_cpu;

/* Instruction sets of the int8 dot products (mi_moe_cpu_get_info's isa). */
#define MI_MOE_ISA_SCALAR 0
#define MI_MOE_ISA_AVX2 1
#define MI_MOE_ISA_AVX_VNNI 2
#define MI_MOE_ISA_AVX512_VNNI 3

/* num_threads 0: every CPU of the process affinity mask, else at most that
 * many (whole NUMA nodes first); tp 0: one shard per NUMA node holding
 * threads, else exactly tp shards (I/tp a multiple of 32).  quant_type 0 / 1. */
int mi_moe_cpu_create(int64_t num_experts, int64_t hidden, int64_t intermediate,
                      int quant_type, int num_threads, int tp, mi_moe_cpu** out);

/* The reference's NUMA layout: tp shards, shard s on NUMA node s with
 * threads_per_node of its CPUs (0: all of them, as when
 * NANOVLLM_TP_THREADS_PER_NODE is unset); tp 0 = one shard per NUMA node of
 * the affinity mask.  On a host with fewer nodes than tp the affinity CPUs
 * are split into tp groups in order (the reference refuses tp > nodes).
 * Replaces the tp_size / threads-per-node setup of MoEInfer
 * (Int8-gemm/moe_infer.cpp:25-36, Int8-gemm/numa_threadpool.h:498-504);
 * the CPU dispatch key calls it when NANOVLLM_TP_SIZE or
 * NANOVLLM_TP_THREADS_PER_NODE is set. */
int mi_moe_cpu_create_numa(int64_t num_experts, int64_t hidden, int64_t intermediate,
                           int quant_type, int tp, int threads_per_node, mi_moe_cpu** out);
int mi_moe_cpu_destroy(mi_moe_cpu* c);

/* Wire layout as mi_moe_store_quantized (store_quantized_weights_repack,
 * Int8-gemm/moe_infer.cpp:96-282), host memory; each shard's threads repack
 * their shard (first touch places it on their node). */
int mi_moe_cpu_store_quantized(mi_moe_cpu* c, const void* gate_up_qs,
                               const void* gate_up_d, const void* down_qs,
                               const void* down_d, int scale_dtype);

/* Online Q8_0 of one projection (as mi_moe_quantize_and_store_expert;
 * Int8-gemm/moe_infer.cpp:284-360), host memory; Q8_0 only. */
int mi_moe_cpu_quantize_and_store_expert(mi_moe_cpu* c, int64_t expert, int proj,
                                         const void* w, int w_dtype);

/* The fused layer on host memory: arguments as mi_moe_forward (ids outside
 * [0,E) dropped; a token with no valid id gets zeros).  Replaces
 * MoEInfer::execute_on_cpu_routed_from_pointers (Int8-gemm/moe_infer.cpp:
 * 430-456); wall time of the call in mi_moe_cpu_get_info's last_ms.  Calls
 * on one handle run one at a time (its buffers and thread pools are shared;
 * the reference's process-wide pool, moe_common.cpp:57-111, is not locked). */
int mi_moe_cpu_forward(mi_moe_cpu* c, const void* x, void* y, const float* topk_w,
                       const int32_t* topk_ids, int64_t T, int64_t K, int act_dtype);

/* Threads, shards, instruction set (MI_MOE_ISA_*), CPUs and NUMA nodes of the
 * affinity mask, and the last forward's wall time in ms.  Any output may be
 * NULL. */
int mi_moe_cpu_get_info(mi_moe_cpu* c, int* threads, int* tp, int* isa,
                        int* affinity_cpus, int* affinity_nodes, double* last_ms);

/* Run the dots with another instruction set the host supports (results are
 * the same bit for bit; for testing each form).  MI_MOE_EUNSUPPORTED if the
 * host lacks it. */
int mi_moe_cpu_set_isa(mi_moe_cpu* c, int isa);

/* Name of an MI_MOE_ISA_* value. */
const char* mi_moe_cpu_isa_name(int isa);

/* ------------------------------------------------------------------------
 * Hybrid CPU-offload executor.  The reference's NPU op runs the whole layer
 * in a host callback between device->host and host->device copies
 * (moe_forward_npu_stream, Int8-gemm/nanovllm_ops.cpp:244-305); its roadmap
 * keeps hot experts in device memory and runs cold ones on the CPU
 * (README.md:124-134).  Here experts with host_mask[e] != 0 ("cold") keep
 * their wire-format weights in host memory and run on a pool of host
 * threads; the others are stored compacted in a device handle, so device
 * memory holds only them.  A forward overlaps the two halves (see
 * mi_moe_hybrid_forward). */
typedef struct mi_moe_hybrid mi_moe_hybrid;

/* num_threads host threads (0: the CPUs of the affinity mask but one, at most
 * 16; the calling thread counts as one of them).  Shape rules
 * as mi_moe_create.  Without a HIP device only an all-cold handle can be made
 * (usable through mi_moe_hybrid_host_forward). */
int mi_moe_hybrid_create(int64_t num_experts, int64_t hidden, int64_t intermediate,
                         int quant_type, const uint8_t* host_mask, int num_threads,
                         mi_moe_hybrid** out);

int mi_moe_hybrid_destroy(mi_moe_hybrid* hh);

/* Same arrays and layouts as mi_moe_store_quantized / mi_moe_store_awq,
 * covering all E experts; each expert's slices go to the device handle or to
 * host memory according to the mask. */
int mi_moe_hybrid_store_quantized(mi_moe_hybrid* hh, const void* gate_up_qs,
                                  const void* gate_up_d, const void* down_qs,
                                  const void* down_d, int scale_dtype,
                                  int src_on_device, void* stream);
int mi_moe_hybrid_store_awq(mi_moe_hybrid* hh, const int32_t* w13_qweight,
                            const int32_t* w13_qzeros, const void* w13_scales,
                            const int32_t* w2_qweight, const int32_t* w2_qzeros,
                            const void* w2_scales, int64_t group, int scale_dtype,
                            int src_on_device, void* stream);

/* The fused MoE layer over all E experts, arguments as mi_moe_forward (device
 * pointers, stream-ordered).  On `stream`: the ids of cold experts are
 * remapped to -1, a kernel writes x, ids and topk_w into pinned host memory
 * and the device handle runs the hot ones into y; meanwhile a side stream of
 * the handle runs the cold experts in a stream host callback into a pinned
 * fp32 partial, which a device kernel then reads: y = round(y_hot + y_cold), with
 * y_hot already rounded to the activation dtype.  Calls that overlap on one handle race, as for
 * mi_moe_forward.  Growing the staging buffers synchronizes the streams; a
 * call can be captured into a HIP graph once a call of at least its size has
 * been made (under capture a call that would grow returns MI_MOE_EINVAL), and
 * the graph must not outlive the handle.  A captured call's host callback
 * reads the staging buffers the graph captured (staging outgrown after a
 * capture is kept until destroy), and its arguments belong to the graph (a
 * HIP user object: freed with the graph).  If a host pass fails (out of host
 * memory) its partial is filled with NaN, so that call's y is NaN, and the
 * next mi_moe_hybrid_forward on the handle returns MI_MOE_EDEVICE. */
int mi_moe_hybrid_forward(mi_moe_hybrid* hh, const void* x, void* y,
                          const float* topk_w, const int32_t* topk_ids,
                          int64_t T, int64_t K, int act_dtype, void* stream);

/* The cold experts' partial alone, synchronously, on host memory: y_part
 * [T,H] fp32 = per token, sum over k in order of topk_w * expert(x) over the
 * pairs routed to cold experts (0 elsewhere).  x_host [T,H] fp16/bf16. */
int mi_moe_hybrid_host_forward(mi_moe_hybrid* hh, const void* x_host,
                               const float* topk_w_host,
                               const int32_t* topk_ids_host, int64_t T,
                               int64_t K, int act_dtype, float* y_part_host);

/* Expert split, host weight bytes, and the last host pass: its duration and
 * routed pairs, and the delay from the mi_moe_hybrid_forward call to the start
 * of its host callback (ms; valid once that call's stream has been
 * synchronized).  Any output pointer may be NULL. */
int mi_moe_hybrid_get_stats(mi_moe_hybrid* hh, int64_t* device_experts,
                            int64_t* host_experts, int64_t* host_weight_bytes,
                            double* last_host_ms, int64_t* last_host_pairs,
                            double* last_queue_ms);

#ifdef __cplusplus
}
#endif
#endif
