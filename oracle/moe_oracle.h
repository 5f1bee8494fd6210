/*
 * moe_oracle.h -- CPU restatement of the reference fused-MoE algorithm.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the MI355X
 * kernels: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path (libmimoe.so, the torch shim) never
 * links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference checkout, Int8-gemm/...).  Numeric conventions:
 *   - fp16 / bf16 values travel as raw uint16_t bits.
 *   - All fp32 arithmetic is written operation by operation and the library is
 *     compiled with -ffp-contract=off, so no multiply-add is fused unless an
 *     explicit fmaf() appears.
 *   - dtype codes: 0 = fp16, 1 = bf16 (matches include/mi_moe.h).
 *   - quant codes: 0 = Q8_0, 1 = Q4_0 (Int8-gemm/quant_traits.h:7-10),
 *     2 = W4A16 (AWQ-style int4, build-defined; the reference's W4A16 kernel
 *     lives in an absent submodule).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (RNE), exact widenings ---- */
float orc_f16_to_f32(uint16_t h);
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_f16(float f);
uint16_t orc_f32_to_bf16(float f);

/* exp(x) by Cody-Waite range reduction + degree-7 Taylor polynomial (Horner,
 * fmaf).  Same operation sequence as the device function in the HIP library. */
float orc_expf(float x);

/* Q8_0 block quantizer, 32 floats -> fp32 scale + 32 int8.
 * Int8-gemm/gemm_kernels.cpp:25-58 (amax, d=amax/127, id=1/d, RNE, saturate). */
void orc_quantize_block_q8_0(const float* x, float* d, int8_t* qs);

/* Same rule, scale stored as fp16 bits (quantize_weight_only,
 * Int8-gemm/q8_gemm.cpp:197-260; q uses the fp32 id of the unrounded d). */
void orc_quantize_block_q8_0_f16d(const float* x, uint16_t* d_f16, int8_t* qs);

/* Stage A activation quantization: x [T,H] fp16/bf16 -> qs [T,H] int8,
 * d [T,H/32] fp32.  Int8-gemm/q8_gemm.cpp:360-377. */
void orc_quantize_act_q8_0(const uint16_t* x, int act_dtype, int64_t T,
                           int64_t H, int8_t* qs, float* d);

/* quantize_weight_only: w [N,K] fp32 -> qs [N,K] int8, d [N,K/32] fp16 bits.
 * Int8-gemm/q8_gemm.cpp:219-260. */
void orc_quantize_weight_q8_0(const float* w, int64_t N, int64_t K,
                              int8_t* qs, uint16_t* d_f16);

/* Routing preprocessing, Int8-gemm/moe_common.cpp:146-216.
 * ids [T,K] -> counts [E], starts [E+1], token_map [2*n_valid] as (t,k)
 * pairs in expert-sorted order, scatter [T*K] (position or -1).
 * Returns n_valid, or -1 for an unsupported top_k (reference throws). */
int64_t orc_route(const int32_t* ids, int64_t T, int64_t K, int64_t E,
                  int32_t* counts, int32_t* starts, int32_t* token_map,
                  int32_t* scatter, int restrict_topk);

/* Per-32-block exact int32 dots for one weight matrix in WIRE layout:
 * isum[m][n][kb] = sum_{i<32} a_qs[m][32kb+i] * w(n, 32kb+i)
 * with w = int8 (Q8_0) or nibble-8 (Q4_0, element k in u32[k/8] bits 4(k%8)).
 * Int8-gemm/gemm_kernels.cpp:102-133 (Q8_0), 262-309 (Q4_0). */
void orc_block_dots(int qt, const int8_t* a_qs, int64_t M, const void* w_qs,
                    int64_t N, int64_t K, int32_t* isum);

/* silu_and_mul on one [2*ish] fp32 row, in place into the first ish entries:
 * row[j] = up[j] * (g / (1 + exp(-g))).  Int8-gemm/vec_simd.h:36-64. */
void orc_silu_and_mul(float* row, int64_t ish);

/* Full Q8_0 / Q4_0 fused-MoE forward, weights in the caller WIRE layout of
 * store_quantized_repack (Int8-gemm/moe_infer.cpp:96-282):
 *   Q8_0: gate_up_qs int8 [E,2I,H], down_qs int8 [E,H,I]
 *   Q4_0: gate_up_qs u32 [E,2I,H/8], down_qs u32 [E,H,I/8]
 *   gate_up_d [E,2I,H/32], down_d [E,H,I/32] as fp16/bf16 bits (scale_dtype)
 * Restates moe_forward_ptr_impl, Int8-gemm/q8_gemm.cpp:276-646, including the
 * tp-shard split of I (Int8-gemm/moe_infer.cpp:143-205) and the C2 reduction
 * order.  y [T,H] in act_dtype bits; y_f32 (optional) receives the fp32 value
 * before the cast.  Returns 0, or -1 for an unsupported top_k / shape. */
int orc_moe_forward_q(int qt, int act_dtype, int scale_dtype,
                      const uint16_t* x, uint16_t* y, float* y_f32,
                      const float* topk_w, const int32_t* topk_ids,
                      const void* gate_up_qs, const uint16_t* gate_up_d,
                      const void* down_qs, const uint16_t* down_d,
                      int64_t T, int64_t H, int64_t E, int64_t I, int64_t tp,
                      int64_t K);

/* W4A16 AWQ-style weight dequantization of one expert projection:
 * qweight int32 [K, N/8], qzeros int32 [K/g, N/8], scales [K/g, N] (bits) ->
 * w fp32 [N, K] (row n = output).  Nibble slot s of a packed word holds
 * column 8*j + AWQ_ORDER[s], AWQ_ORDER = {0,2,4,6,1,3,5,7}. */
void orc_awq_dequant(const int32_t* qweight, const int32_t* qzeros,
                     const uint16_t* scales, int scale_dtype, int64_t K,
                     int64_t N, int64_t group, float* w);

/* W4A16 fused-MoE forward in fp32 (dequant (q-z)*s, fp32 accumulation in k
 * order, fp32 SiLU*mul, fp32 combine in k order, final cast).  Weights:
 *   w13_q int32 [E,H,2I/8], w13_z int32 [E,H/g,2I/8], w13_s [E,H/g,2I]
 *   w2_q  int32 [E,I,H/8],  w2_z  int32 [E,I/g,H/8],  w2_s  [E,I/g,H]
 * Columns [0,I) of w13 are gate_proj, [I,2I) are up_proj.
 * The dataflow (dispatch -> gate_up -> SiLU*mul -> down -> weighted combine
 * in k order -> cast) follows Int8-gemm/q8_gemm.cpp:276-646 with the
 * dequantized weights of the absent W4A16 kernel (README.md:19-30). */
int orc_moe_forward_w4a16(int act_dtype, int scale_dtype, const uint16_t* x,
                          uint16_t* y, float* y_f32, const float* topk_w,
                          const int32_t* topk_ids, const int32_t* w13_q,
                          const int32_t* w13_z, const uint16_t* w13_s,
                          const int32_t* w2_q, const int32_t* w2_z,
                          const uint16_t* w2_s, int64_t T, int64_t H,
                          int64_t E, int64_t I, int64_t K, int64_t group,
                          int nthreads);

/* Router top-k + softmax (Int8-gemm/test/fused_moe_cpu.py:20-37). */
int orc_topk_softmax(const float* logits, int64_t T, int64_t E, int64_t K,
                     int renormalize, int32_t* ids, float* w);

#ifdef __cplusplus
}
#endif
#endif
