/*
 * marlin_mi355x.h -- C ABI of the MI355X (gfx950) Marlin mixed-precision GEMM library.
 *
 * Every entry point takes plain device pointers, element counts and a HIP stream, and
 * launches asynchronously on that stream.  No entry point synchronises the host.
 * Each entry point replaces one torch op of the reference extension; the comment above it
 * cites the reference host function whose validation contract and semantics it keeps.
 *
 * Return value: MARLIN_STATUS_OK, or an error code with a message available from
 * marlin_get_last_error() (thread-local).  Messages for argument errors reuse the
 * reference's TORCH_CHECK wording where the condition is the same.
 *
 * Tensor arguments are passed as (pointer, dtype, numel) where the reference passes a
 * tensor.  An absent optional tensor is (NULL, any dtype, 0).  All tensors are contiguous
 * row-major unless a stride argument says otherwise.
 */
#ifndef MARLIN_MI355X_H_
#define MARLIN_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without including HIP headers. */
typedef struct ihipStream_t* marlin_stream_t;

typedef enum {
  MARLIN_STATUS_OK = 0,
  MARLIN_STATUS_INVALID_ARGUMENT = 1, /* a validation check failed (TORCH_CHECK in the reference) */
  MARLIN_STATUS_NOT_SUPPORTED = 2,    /* legal upstream, not implemented on this build */
  MARLIN_STATUS_HIP_ERROR = 3,        /* a HIP runtime call or kernel launch failed */
} marlin_status_t;

/* Element types of the tensors crossing the boundary (torch dtype equivalents). */
typedef enum {
  MARLIN_DTYPE_FLOAT16 = 0,
  MARLIN_DTYPE_BFLOAT16 = 1,
  MARLIN_DTYPE_FLOAT32 = 2,
  MARLIN_DTYPE_FLOAT8_E4M3FN = 3,
  MARLIN_DTYPE_FLOAT8_E8M0FNU = 4,
  MARLIN_DTYPE_INT32 = 5,
  MARLIN_DTYPE_INT64 = 6,
  MARLIN_DTYPE_UINT8 = 7,
  MARLIN_DTYPE_INT8 = 8,
  MARLIN_DTYPE_UINT32 = 9,
} marlin_dtype_t;

/* Message of the last failed call on this thread ("" if none). */
const char* marlin_get_last_error(void);

/* ABI version of this header; bumped on incompatible changes. */
int marlin_abi_version(void);
#define MARLIN_MI355X_ABI_VERSION 2

/*
 * Weight repack: GPTQ layout [size_k / (32/num_bits), size_n] int32 (values packed LSB-first
 * along K) -> kernel layout, int32 [size_k/16, size_n*16/(32/num_bits)].
 * Replaces torch.ops._C.gptq_marlin_repack
 * (reference csrc/quantization/marlin/gptq_marlin_repack.cu:399-469).
 * perm: optional act-order row permutation (perm_numel == size_k) or NULL/0.
 * is_a_8bit: the reference's 8-bit-activation layout instead
 * (gptq_marlin_repack.cu:225-335): 32 x 32 (k x n) tiles, k tiles outer; within a tile the
 * words of thread th (0..31) and n8 slice s (0..3) are the B fragment of an m16n8k32 8-bit
 * tensor-core MMA for column 16*(s/2) + 8*(s%2) + th/4, rows 4*(th%4) + {0..3} and the same
 * rows + 16 (4-bit: word th*4 + s, nibble i = row 4*(th%4) + i/2 + 16*(i%2); 8-bit: words
 * th*8 + 2*s + h, byte i = row 4*(th%4) + 16*h + i).  Not with perm (the reference rejects
 * that combination).  The GEMM itself rejects 8-bit activations, as the reference's does.
 */
marlin_status_t marlin_gptq_marlin_repack(const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                          const int32_t* perm, int64_t perm_numel,
                                          int64_t size_k, int64_t size_n, int64_t num_bits,
                                          int is_a_8bit, int32_t* out, int64_t out_numel,
                                          marlin_stream_t stream);

/*
 * Weight repack: AWQ layout [size_k, size_n / (32/num_bits)] int32 (values packed along N
 * in AWQ interleave order) -> the same kernel layout as marlin_gptq_marlin_repack.
 * Replaces torch.ops._C.awq_marlin_repack
 * (reference csrc/quantization/marlin/awq_marlin_repack.cu:300-381).
 * is_a_8bit: the 8-bit-activation layout of marlin_gptq_marlin_repack
 * (awq_marlin_repack.cu:165-270).
 */
marlin_status_t marlin_awq_marlin_repack(const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                         int64_t size_k, int64_t size_n, int64_t num_bits,
                                         int is_a_8bit, int32_t* out, int64_t out_numel,
                                         marlin_stream_t stream);

/*
 * W4A8-FP8 weight preprocess: every 4-bit code v of qweight becomes v - z when v >= z, else
 * 15 - v, with z = 8 (qzeros NULL: GPTQ-style weights, any shape with numel * 8 % 256 == 0)
 * or the code's AWQ zero point (qweight [size_k, size_n/8] int32, qzeros
 * [size_k/group_size, size_n/8] int32: same word column and nibble, row k / group_size;
 * size_k % 32 == 0, group_size % 8 == 0).  out may equal qweight (in place).
 * Replaces torch.ops._C.marlin_int4_fp8_preprocess
 * (reference csrc/quantization/marlin/marlin_int4_fp8_preprocess.cu:5-97).
 */
marlin_status_t marlin_int4_fp8_preprocess(const int32_t* qweight, int64_t qweight_rows,
                                           int64_t qweight_cols, const int32_t* qzeros,
                                           int64_t qzeros_rows, int64_t qzeros_cols, int32_t* out,
                                           marlin_stream_t stream);

/*
 * Dense mixed-precision GEMM: C[M,N] = A[M,K] . dequant(B)[K,N] (+ bias), fp32 accumulation.
 * Replaces torch.ops._C.marlin_gemm (reference csrc/quantization/marlin/marlin.cu:83-506).
 *   a         : [size_m, size_k] fp16 or bf16, row stride a_row_stride elements (%8 == 0).
 *   c         : [size_m, size_n] output, dtype of a, contiguous; overwritten (not accumulated).
 *   b_q_weight: repacked weights (marlin_*_repack output).
 *   b_bias    : optional [size_n], dtype of a, in marlin_permute_bias order.
 *   b_scales  : [num_groups, size_n]; dtype of a for integer types, float8_e4m3fn
 *               (NVFP4, S0E5M3-processed) or float8_e8m0fnu (MXFP4) for float4_e2m1f.
 *   a_scales_numel: must be 0 (8-bit activations are not supported, as in the reference).
 *   global_scale: NVFP4 only, fp32 numel 1.
 *   b_zeros   : uint4/uint8 only (and required there): float zero points [num_groups, size_n]
 *               in the dtype of a with is_zp_float = 1, or integer zero points packed along N
 *               as int32 [num_groups, size_n / (32/bits)] (column n in bits
 *               [bits*(n % (32/bits)), ...)) with is_zp_float = 0; the latter dequantizes to
 *               the single rounding of (q - z) * s.  The SM70 reference rejects packed integer
 *               zero points (marlin.cu:336-339); upstream marlin takes them.
 *   g_idx, perm: act-order, both [size_k] int32 or both absent: perm = argsort(original g_idx),
 *               g_idx the sorted group index (marlin_sort_g_idx), the weights repacked with
 *               perm.  Every group must hold group_size rows (GPTQ act-order), i.e.
 *               g_idx[j] == j / group_size; columns that break it come out NaN.  A is gathered
 *               by perm into a library staging buffer before the GEMM.  Integer weight types
 *               and is_k_full = 1 only.  The reference rejects
 *               act-order (marlin.cu:95-102); upstream marlin takes it.
 *   workspace : accepted for ABI fidelity and ignored, as in the reference (marlin.cu:103);
 *               split-K scratch is owned by the library per (device, stream).
 *   b_type_id : vllm ScalarType id (uint4, uint4b8, uint8, uint8b128, float8_e4m3fn,
 *               float4_e2m1f).
 *   is_k_full, use_atomic_add, use_fp32_reduce: accepted and ignored, as in the reference.
 */
marlin_status_t marlin_gemm(const void* a, marlin_dtype_t a_dtype, int64_t a_row_stride,
                            void* c, const int32_t* b_q_weight, int64_t b_q_weight_numel,
                            const void* b_bias, int64_t b_bias_numel,
                            const void* b_scales, marlin_dtype_t b_scales_dtype,
                            int64_t b_scales_numel, int64_t num_groups,
                            int64_t a_scales_numel,
                            const float* global_scale, int64_t global_scale_numel,
                            const void* b_zeros, marlin_dtype_t b_zeros_dtype,
                            int64_t b_zeros_numel, const int32_t* g_idx, int64_t g_idx_numel,
                            const int32_t* perm, int64_t perm_numel, void* workspace,
                            int64_t workspace_bytes, int64_t b_type_id, int64_t size_m,
                            int64_t size_n, int64_t size_k, int is_k_full, int use_atomic_add,
                            int use_fp32_reduce, int is_zp_float, marlin_stream_t stream);

/*
 * marlin_gemm for callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  No counterpart in the reference.
 * Same arguments, checks and results as marlin_gemm (minus the ignored workspace and
 * reduction flags), but it calls no hipMalloc / hipFree / allocating library routine: the
 * split-K partial sums and arrival counters live in a static device array of fixed size,
 * one per GPU, held until the process ends.  A call whose plan splits K and needs more than
 * MARLIN_NO_ALLOC_MAX_PARTIALS partial sums (size_m * size_n) or MARLIN_NO_ALLOC_MAX_COUNTERS
 * counters returns MARLIN_STATUS_INVALID_ARGUMENT.  The first call on a device clears the
 * array with one fill kernel on `stream`.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, or host threads) race.  Act-order
 * (g_idx_numel or perm_numel non-zero) and packed integer zero points return
 * MARLIN_STATUS_NOT_SUPPORTED: their staging buffers would need an allocation.
 */
#define MARLIN_NO_ALLOC_MAX_PARTIALS 2097152
#define MARLIN_NO_ALLOC_MAX_COUNTERS 65536
marlin_status_t marlin_gemm_no_alloc(const void* a, marlin_dtype_t a_dtype, int64_t a_row_stride,
                                     void* c, const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                     const void* b_bias, int64_t b_bias_numel,
                                     const void* b_scales, marlin_dtype_t b_scales_dtype,
                                     int64_t b_scales_numel, int64_t num_groups,
                                     int64_t a_scales_numel, const float* global_scale,
                                     int64_t global_scale_numel, const void* b_zeros,
                                     marlin_dtype_t b_zeros_dtype, int64_t b_zeros_numel,
                                     int64_t g_idx_numel, int64_t perm_numel, int64_t b_type_id,
                                     int64_t size_m, int64_t size_n, int64_t size_k,
                                     int is_zp_float, marlin_stream_t stream);

/*
 * MoE token alignment: sorts the flat route indices of topk_ids by expert and pads each
 * expert's run to a multiple of block_size.
 * Replaces torch.ops._moe_C.moe_align_block_size
 * (reference csrc/moe/moe_align_sum_kernels.cu:477-569).
 *   topk_ids        : [numel] int32 or int64 expert ids (flattened [tokens, top_k]).
 *   sorted_token_ids: [sorted_numel] int32 out; every slot not holding a route index holds
 *                     numel (the sentinel).  Within an expert, route indices are ascending.
 *   expert_ids      : [expert_ids_numel] int32 out; block b -> expert, -1 after the last
 *                     used block.
 *   num_tokens_post_pad: [1] int32 out.
 *   expert_map      : optional [num_experts] int32 global->local id map (-1 = not local).
 * Ids outside [0, num_experts) are skipped.
 */
marlin_status_t marlin_moe_align_block_size(const void* topk_ids, marlin_dtype_t topk_ids_dtype,
                                            int64_t numel, int64_t num_experts,
                                            int64_t block_size, int32_t* sorted_token_ids,
                                            int64_t sorted_numel, int32_t* expert_ids,
                                            int64_t expert_ids_numel,
                                            int32_t* num_tokens_post_pad,
                                            const int32_t* expert_map, int64_t expert_map_numel,
                                            marlin_stream_t stream);

/*
 * Grouped MoE GEMM over expert-sorted row blocks.
 * Replaces torch.ops._moe_C.moe_wna16_marlin_gemm
 * (reference csrc/moe/marlin_moe_wna16/ops.cu:102-529).
 * For every moe block b with expert e = expert_ids[b] >= 0 and b*moe_block_size <
 * num_tokens_past_padded[0], and every row r of the block with
 * id = sorted_token_ids[b*moe_block_size + r] < size_m*top_k:
 *   C[id, :] = ((A[id / top_k, :] . dequant(B[e])) * alpha_e + bias_e' ) * w
 * where alpha_e is the NVFP4 global scale of expert e (1 otherwise), bias_e' = bias_e *
 * (mul_topk_weights ? alpha_e : 1) when a bias is given, and w = topk_weights[id] when
 * mul_topk_weights, else 1.
 *   a: [size_m, size_k]; c: [size_m*top_k, size_n]; b_q_weight: [E, size_k/16, ...];
 *   b_scales / b_zeros: [E, num_groups, size_n]; b_bias: [E, size_n]; global_scale: [E].
 *   thread_k, thread_n, blocks_per_sm, is_k_full, use_atomic_add, use_fp32_reduce:
 *   accepted and ignored, as in the reference (ops.cu:125-133).
 */
marlin_status_t marlin_moe_wna16_marlin_gemm(
    const void* a, marlin_dtype_t a_dtype, void* c, const int32_t* b_q_weight,
    int64_t b_q_weight_numel, int64_t num_experts, const void* b_bias, int64_t b_bias_numel,
    const void* b_scales, marlin_dtype_t b_scales_dtype, int64_t b_scales_numel,
    int64_t num_groups, int64_t a_scales_numel, const float* global_scale,
    int64_t global_scale_numel, const void* b_zeros, marlin_dtype_t b_zeros_dtype,
    int64_t b_zeros_numel, int64_t g_idx_numel, int64_t perm_numel, void* workspace,
    int64_t workspace_bytes, const int32_t* sorted_token_ids, int64_t sorted_numel,
    const int32_t* expert_ids, int64_t expert_ids_numel,
    const int32_t* num_tokens_past_padded, const float* topk_weights,
    int64_t topk_weights_numel, int64_t moe_block_size, int64_t top_k, int mul_topk_weights,
    int64_t b_type_id, int64_t size_m, int64_t size_n, int64_t size_k, int is_k_full,
    int use_atomic_add, int use_fp32_reduce, int is_zp_float, int64_t thread_k,
    int64_t thread_n, int64_t blocks_per_sm, marlin_stream_t stream);

/*
 * MoE stage 1 with the SiLU-gated activation fused: the arguments of
 * marlin_moe_wna16_marlin_gemm (size_n = 2 * I, the gate columns first), but c receives
 * silu(h[:, :I]) * h[:, I:] as [size_m * top_k, size_n / 2] instead of h, rounded as
 * marlin_moe_wna16_marlin_gemm followed by marlin_silu_and_mul round it.  No counterpart op
 * in the reference: it fuses the reference's stage 1 and activation
 * (fused_marlin_moe.py:183-212, activation.py:45-52).  The multistage kernel's plans
 * (size_n % 256 == 0, no split K) and the few-routes decode kernel's plans (integer or fp8
 * weights with >= 128-deep groups or channelwise scales, at most 16 routes per expert on
 * average) are fused; for any other plan it returns MARLIN_STATUS_NOT_SUPPORTED before
 * launching anything, and the caller runs the two passes.
 */
marlin_status_t marlin_moe_wna16_marlin_gemm_silu(
    const void* a, marlin_dtype_t a_dtype, void* c, const int32_t* b_q_weight,
    int64_t b_q_weight_numel, int64_t num_experts, const void* b_bias, int64_t b_bias_numel,
    const void* b_scales, marlin_dtype_t b_scales_dtype, int64_t b_scales_numel,
    int64_t num_groups, int64_t a_scales_numel, const float* global_scale,
    int64_t global_scale_numel, const void* b_zeros, marlin_dtype_t b_zeros_dtype,
    int64_t b_zeros_numel, int64_t g_idx_numel, int64_t perm_numel, void* workspace,
    int64_t workspace_bytes, const int32_t* sorted_token_ids, int64_t sorted_numel,
    const int32_t* expert_ids, int64_t expert_ids_numel,
    const int32_t* num_tokens_past_padded, const float* topk_weights,
    int64_t topk_weights_numel, int64_t moe_block_size, int64_t top_k, int mul_topk_weights,
    int64_t b_type_id, int64_t size_m, int64_t size_n, int64_t size_k, int is_k_full,
    int use_atomic_add, int use_fp32_reduce, int is_zp_float, int64_t thread_k,
    int64_t thread_n, int64_t blocks_per_sm, marlin_stream_t stream);

/*
 * Dequantize repacked weights to [size_k, size_n] (row-major) in out_dtype (fp16 or bf16),
 * with the device dequant routines the GEMM uses.  Test and inspection aid, no counterpart
 * op in the reference: it restates the reference's dequant helpers
 * (tests/helpers.py:1094-1184, 1543-1641) so dequantization can be checked bit-exactly.
 * For NVFP4 the result is dtype(fp32(v * scale) * global) as in the reference helper.
 */
marlin_status_t marlin_dequantize(const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                  const void* b_scales, marlin_dtype_t b_scales_dtype,
                                  int64_t b_scales_numel, int64_t num_groups,
                                  const void* b_zeros, marlin_dtype_t b_zeros_dtype,
                                  int64_t b_zeros_numel, const float* global_scale,
                                  int64_t global_scale_numel, int64_t b_type_id,
                                  int64_t size_k, int64_t size_n, marlin_dtype_t out_dtype,
                                  void* out, marlin_stream_t stream);

/*
 * Top-k reduction of MoE route outputs: out[t, :] = sum_k input[t, k, :], input
 * [num_tokens, top_k, hidden] and out [num_tokens, hidden] contiguous, fp16, bf16 or fp32.
 * For 16-bit types and top_k 2..4 every addition rounds to the element type (the
 * reference's kernel); otherwise the sum is accumulated in fp32 and rounded once (the
 * reference's at::sum_out).  No limit on num_tokens.
 * Replaces torch.ops._moe_C.moe_sum (reference csrc/moe/moe_align_sum_kernels.cu:598-639).
 */
marlin_status_t marlin_moe_sum(const void* input, marlin_dtype_t dtype, int64_t num_tokens,
                               int64_t top_k, int64_t hidden, void* out,
                               marlin_stream_t stream);

/*
 * MoE SiLU-gated activation: out[r, j] = silu(input[r, j]) * input[r, d + j] for an input of
 * shape [rows, 2d] and an output of shape [rows, d], both contiguous; silu is rounded to the
 * element type before the product, as the reference's torch expression does.
 * Replaces the SiLU branch of apply_moe_activation
 * (reference vllm/model_executor/layers/fused_moe/activation.py:45-52).
 */
marlin_status_t marlin_silu_and_mul(const void* input, marlin_dtype_t dtype, int64_t rows,
                                    int64_t d, void* out, marlin_stream_t stream);

/*
 * MoE router, softmax scoring.  gating_output: [num_tokens, num_experts] fp16, bf16 or fp32,
 * contiguous.  Per row: scores = softmax(row) in fp32; the top_k experts by score + bias[e]
 * (bias optional, fp32 [num_experts]) in descending order, ties to the lower expert index;
 * topk_weights [num_tokens, top_k] fp32 = the unbiased scores, divided by their sum when
 * renormalize != 0 (a zero sum divides by 1); topk_indices [num_tokens, top_k] in int32,
 * uint32 or int64; token_expert_indices [num_tokens, top_k] int32 = j * num_tokens + t.
 * This build supports num_experts <= 4096 and top_k <= 256 (MARLIN_STATUS_NOT_SUPPORTED
 * beyond).
 * Replaces torch.ops._moe_C.topk_softmax (reference csrc/moe/topk_softmax_kernels.cu:773-809,
 * argument checks :732-739; schema csrc/moe/torch_bindings_marlin.cpp:5-9).
 */
marlin_status_t marlin_topk_softmax(float* topk_weights, void* topk_indices,
                                    marlin_dtype_t topk_indices_dtype,
                                    int32_t* token_expert_indices, int64_t top_k,
                                    const void* gating_output, marlin_dtype_t gating_dtype,
                                    int64_t num_tokens, int64_t num_experts, int renormalize,
                                    const float* bias, int64_t bias_numel,
                                    marlin_stream_t stream);

/*
 * MoE router, sigmoid scoring: as marlin_topk_softmax with scores = 1 / (1 + exp(-x)).
 * Replaces torch.ops._moe_C.topk_sigmoid (reference csrc/moe/topk_softmax_kernels.cu:811-847;
 * schema csrc/moe/torch_bindings_marlin.cpp:11-15).
 */
marlin_status_t marlin_topk_sigmoid(float* topk_weights, void* topk_indices,
                                    marlin_dtype_t topk_indices_dtype,
                                    int32_t* token_expert_indices, int64_t top_k,
                                    const void* gating_output, marlin_dtype_t gating_dtype,
                                    int64_t num_tokens, int64_t num_experts, int renormalize,
                                    const float* bias, int64_t bias_numel,
                                    marlin_stream_t stream);

/*
 * Grouped MoE router.  scores: [num_tokens, num_experts] fp16, bf16 or fp32, contiguous; the
 * experts form n_group equal groups.  Per row, with s = scores (scoring_func 0) or
 * sigmoid(scores) (scoring_func 1) in fp32 and choice = s + bias (bias [num_experts] fp16,
 * bf16 or fp32; non-finite inputs do not compete): a group's score is the sum of its two
 * largest choices; the topk_group best groups are kept (ties to the lower group); the topk
 * experts of the kept groups by choice follow (ties to the lower expert).
 * topk_values [num_tokens, topk] fp32 = s * routed_scaling_factor, divided by
 * (1e-20 + sum of the chosen s) when renormalize != 0; topk_indices [num_tokens, topk] int32.
 * A row whose last kept group scores -inf gets experts 0..topk-1 with weight 1/topk.
 * This build supports num_experts <= 1024 (MARLIN_STATUS_NOT_SUPPORTED beyond).
 * Replaces torch.ops._moe_C.grouped_topk (reference csrc/moe/grouped_topk_kernels.cu:987-1090;
 * schema csrc/moe/torch_bindings_marlin.cpp:48-54).
 */
marlin_status_t marlin_grouped_topk(const void* scores, marlin_dtype_t scores_dtype,
                                    int64_t num_tokens, int64_t num_experts, int64_t n_group,
                                    int64_t topk_group, int64_t topk, int renormalize,
                                    double routed_scaling_factor, const void* bias,
                                    marlin_dtype_t bias_dtype, int64_t bias_numel,
                                    int64_t scoring_func, float* topk_values,
                                    int32_t* topk_indices, marlin_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MARLIN_MI355X_H_ */
