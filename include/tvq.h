/*
 * tvq.h — C ABI of the MI355X (gfx950) quantized-linear library
 * (libtinyvllm_quant.so).
 *
 * This library is the device half of tiny-vLLM's quantized Linear hot path:
 * the INT8 weight-only GEMM (W8A16) and the W8A8 GEMM with per-token dynamic
 * activation quantization. Every entry point takes plain device pointers,
 * sizes and a hipStream_t passed as `void*`. The library never allocates,
 * never synchronises the stream and launches only on the stream it is given,
 * so every call is safe inside HIP-graph capture. All buffers (outputs
 * included) are owned by the caller.
 *
 * Layouts (all row-major, contiguous, leading dimension = number of columns):
 *   x        [M, K]  bf16 or fp16 activations
 *   xq       [M, K]  int8 quantized activations
 *   a_scales [M]     fp32 per-token activation scales
 *   qweight  [N, K]  int8 weights, the on-disk `*.qweight` layout unchanged
 *   scales   [N]     fp32 per-output-channel weight scales (`*.scales` /
 *                    `*.w_scales` on disk)
 *   bias     [N]     same dtype as the output, or NULL
 *   y        [M, N]  bf16 or fp16 output (int32 for tvq_w8a8_gemm_i32)
 *
 * GEMM workspace: the GEMM entry points take an optional device workspace
 * (workspace, workspace_bytes; NULL/0 disables its use). With one, decode-
 * size calls whose output tiles do not fill the GPU split K over several
 * workgroups and reduce the partial sums inside the same launch, in a fixed
 * order (results do not depend on scheduling). The workspace must be
 * 256-byte aligned and zero-filled once when it is allocated; every call
 * leaves it ready for the next. Calls that share a workspace must be ordered
 * (one stream). tvq_gemm_workspace_bytes() gives the size that enables every
 * split; a smaller one only limits them.
 *
 * Return codes: TVQ_OK (0) on success, a negative TVQ_E* code otherwise;
 * tvq_last_error() then describes the failure (thread-local string).
 */
#ifndef TVQ_H_
#define TVQ_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TVQ_ABI_VERSION 5

/* Activation / output element types. */
enum tvq_dtype {
  TVQ_DTYPE_F16 = 0,
  TVQ_DTYPE_BF16 = 1,
};

/* Operation ids for tvq_select_path. */
enum tvq_op {
  TVQ_OP_ACT_QUANT = 0,
  TVQ_OP_W8A16 = 1,
  TVQ_OP_W8A8 = 2,
};

enum tvq_status {
  TVQ_OK = 0,
  TVQ_E_INVALID = -1,     /* bad pointer, size or dtype */
  TVQ_E_UNSUPPORTED = -2, /* shape/alignment the library cannot run */
  TVQ_E_HIP = -3,         /* a HIP runtime call failed (launch error) */
};

/* Version of this ABI (TVQ_ABI_VERSION). No reference counterpart: the
 * reference's pybind11 modules are versioned by their JIT build hash. */
int tvq_abi_version(void);

/* Message for the last failing call on this thread ("" if none). Replaces the
 * TORCH_CHECK messages of int8_weight_only_gemm.cpp:19-36 and w8a8_gemm.cpp. */
const char* tvq_last_error(void);

/* Name of the kernel path the library would pick for this op and shape.
 * Replaces `select_path(x, qweight)` of the reference's extensions
 * (int8_weight_only_gemm.cpp:42, int8_weight_only_gemm.cu:545-547;
 * w8a8_gemm.cpp, w8a8_gemm.cu:405-411). `dtype` is the activation dtype for
 * W8A16 / ACT_QUANT and the output dtype for W8A8. The returned string is
 * static. Returns NULL for an invalid op. */
const char* tvq_select_path(int op, int64_t M, int64_t N, int64_t K, int dtype);

/* Per-token (per-row) dynamic symmetric int8 quantization of x [M, K]:
 *   s[m]    = max(amax_k |x[m,k]| / 127, eps)           (fp32, IEEE RN)
 *   xq[m,k] = clamp(rint_half_even(x[m,k] / s[m]), -127, 127)
 * Bit-exact restatement of quantize_int8_per_row_dynamic
 * (nanovllm/quantization/utils.py:28-32) as called by
 * W8A8QuantMethod.quantize_activation (nanovllm/quantization/w8a8.py:21-23).
 * The reference runs this as ~9 torch kernels; here it is one pass. */
int tvq_act_quant(const void* x, int dtype, int64_t M, int64_t K, float eps,
                  int8_t* xq, float* a_scales, void* stream);

/* W8A16: y = x · (qweight · diag(scales))^T + bias, fp32 accumulation, the
 * per-channel fp32 scale applied once per output. Replaces the extension
 * `forward(x, qweight, scales, bias)` (int8_weight_only_gemm.cpp:14-37,
 * int8_weight_only_gemm.cu:549-618) behind native_int8_weight_only_linear
 * (nanovllm/quantization/cuda.py:261-274). */
int tvq_w8a16_gemm(const void* x, int dtype, const int8_t* qweight,
                   const float* scales, const void* bias, void* y, int64_t M,
                   int64_t N, int64_t K, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* W8A8: acc[m,n] = sum_k xq[m,k]·qweight[n,k] (exact int32),
 *   y[m,n] = out((float(acc)·a_scales[m])·w_scales[n] + bias[n]).
 * Replaces the extension `forward(x_q, a_scales, qweight, w_scales, bias,
 * use_bfloat16)` (w8a8_gemm.cpp:16-54, w8a8_gemm.cu:426-507) behind
 * native_w8a8_linear (nanovllm/quantization/cuda.py:435-452). `out_dtype`
 * selects bf16 (use_bfloat16=True) or fp16 output. */
int tvq_w8a8_gemm(const int8_t* xq, const float* a_scales,
                  const int8_t* qweight, const float* w_scales,
                  const void* bias, void* y, int out_dtype, int64_t M,
                  int64_t N, int64_t K, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* W8A16 with the reference kernel's rounding: every weight is first
 * dequantized to wd[n,k] = T(T(qweight[n,k]) * T(scales[n])) in the
 * activation type T (bf16 or fp16), then y = out(sum_k x[m,k] * wd[n,k] +
 * bias[n]) with fp32 accumulation and no further scaling. Replaces the
 * dequantization of int8_weight_only_gemm_wmma_kernel
 * (int8_weight_only_gemm.cu:397-413, epilogue 507-516), which
 * int8_weight_only_linear_fallback (nanovllm/quantization/cuda.py:293-300)
 * also applies, for callers that need those roundings rather than the fp32
 * per-output scale of tvq_w8a16_gemm. Never splits K. */
int tvq_w8a16_gemm_rounded(const void* x, int dtype, const int8_t* qweight,
                           const float* scales, const void* bias, void* y,
                           int64_t M, int64_t N, int64_t K, void* stream);

/* Measurement only, no reference counterpart: runs the operand stream of the
 * DMA GEMM tiles that tvq_w8a16_gemm (op TVQ_OP_W8A16, x 16-bit) or
 * tvq_w8a8_gemm (TVQ_OP_W8A8, x int8) would launch for this shape -- the same
 * grid, tile walk, global->LDS transfers, waits and barriers, with the
 * fragment reads, MFMAs and output compiled out (unsplit). Its time is the
 * operand-delivery floor of that tiling. Writes no output. Needs K % 128 == 0
 * and 16-byte aligned operands (TVQ_E_UNSUPPORTED otherwise). */
int tvq_gemm_operand_floor(int op, const void* x, const int8_t* qweight,
                           int64_t M, int64_t N, int64_t K, void* stream);

/* The raw exact int32 accumulator acc[m,n] = sum_k xq[m,k]·qweight[n,k] of
 * the W8A8 path, written to y_i32 [M, N], using the same kernel selection as
 * tvq_w8a8_gemm. No reference counterpart as an entry point: it exposes the
 * accumulator the reference forms inside w8a8_gemm_wmma_kernel
 * (w8a8_gemm.cu:336-375) so it can be checked bit-exactly. */
int tvq_w8a8_gemm_i32(const int8_t* xq, const int8_t* qweight, int32_t* y_i32,
                      int64_t M, int64_t N, int64_t K, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* Fused W8A8 linear: tvq_act_quant(x) into the caller's xq / a_scales buffers
 * followed by tvq_w8a8_gemm, both on `stream`. Replaces the pair
 * W8A8QuantMethod.quantize_activation + apply_w8a8_linear inside
 * W8A8QuantMethod.apply (nanovllm/quantization/w8a8.py:25-40). */
int tvq_w8a8_linear(const void* x, int dtype, const int8_t* qweight,
                    const float* w_scales, const void* bias, void* y,
                    int64_t M, int64_t N, int64_t K, int8_t* xq_buf,
                    float* a_scales_buf, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* Limits of tvq_w8a8_linear_noalloc's scratch array (per device). */
#define TVQ_NOALLOC_MAX_XQ_BYTES (8ll << 20) /* M*K int8 activation codes */
#define TVQ_NOALLOC_MAX_ROWS 65536ll         /* M (per-token scales) */

/* tvq_w8a8_linear without caller scratch buffers: the activation codes, the
 * per-token scales and the split-K workspace live in a static device array
 * of the library (about 24.3 MiB per device, held until the process ends), so
 * the call allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP-graph capture, tight serving
 * loops, harnesses that forbid allocation). Same arguments and result as
 * tvq_w8a8_linear without xq_buf / a_scales_buf / workspace. Rejects
 * M > TVQ_NOALLOC_MAX_ROWS or M*K > TVQ_NOALLOC_MAX_XQ_BYTES with
 * TVQ_E_UNSUPPORTED. Calls on one device share the array: calls that overlap
 * on one GPU (other streams, unordered threads) race. */
int tvq_w8a8_linear_noalloc(const void* x, int dtype, const int8_t* qweight,
                            const float* w_scales, const void* bias, void* y,
                            int64_t M, int64_t N, int64_t K, void* stream);

/* Size in bytes of a GEMM workspace that enables every split-K launch (see
 * the top of this file). No reference counterpart: the reference's kernels
 * never split K. */
int64_t tvq_gemm_workspace_bytes(void);

/* Fused RMSNorm producer of a projection input. Replaces RMSNorm.rms_forward
 * / add_rms_forward (nanovllm/layers/layernorm.py:16-40), optionally followed
 * by quantize_int8_per_row_dynamic (nanovllm/quantization/utils.py:28-32) of
 * its output, as W8A8QuantMethod.quantize_activation (w8a8.py:21-23) would
 * apply it in the next qkv_proj / gate_up_proj. Per row of K elements:
 *   h = x (+ residual);  residual <- h  (in place, when residual != NULL)
 *   y = (h * rsqrt(mean(h^2) + eps)) * weight   (rounded as torch rounds)
 * and, when xq != NULL, xq / a_scales = per-token int8 codes and scale of y,
 * bit-identical to tvq_act_quant(y). y and xq may each be NULL (not both).
 * x, residual, weight and y have `dtype`; weight is [K]. No buffer may alias
 * another. */
int tvq_rmsnorm(const void* x, void* residual, const void* weight, float eps,
                void* y, int8_t* xq, float* a_scales, int dtype, int64_t M,
                int64_t K, void* stream);

/* W8A8 gate_up projection with the SiLU-and-multiply in its epilogue:
 * y[m, c] = out(silu(g) * u) with g = out(W8A8 result of gate channel c),
 * u = the same for up channel c, each rounded to the output type first, so
 * y is bit-identical to tvq_w8a8_gemm of gate_up followed by tvq_silu_mul.
 * Fuses MergedColumnParallelLinear(gate_up_proj) with SiluAndMul
 * (nanovllm/layers/activation.py:11-14); the gate_up output [M, 2I] never
 * reaches HBM. qweight_glu / w_scales_glu are gate_up's [2I, K] weights and
 * scales with their rows regrouped in 32-row blocks: block 2b holds gate
 * channels 32b .. 32b+31, block 2b+1 the up channels 32b .. 32b+31
 * (rows 64b + 32h + k <- gate_up row h*I + 32b + k). N2 = 2I must be a
 * multiple of 64, K a multiple
 * of 128 (at most 2^22); all pointers 16-byte aligned; y is [M, I] of
 * out_dtype. No workspace. */
int tvq_w8a8_gemm_glu(const int8_t* xq, const float* a_scales,
                      const int8_t* qweight_glu, const float* w_scales_glu,
                      void* y, int out_dtype, int64_t M, int64_t N2, int64_t K,
                      void* stream);

/* Fused SiLU-and-multiply producer of the down_proj input. Replaces
 * SiluAndMul.forward (nanovllm/layers/activation.py:11-14) on gate_up
 * [M, 2*I] (gate = columns [0, I), up = [I, 2I)): y = silu(gate) * up,
 * [M, I], optionally followed by the per-token int8 quantization of y as in
 * tvq_rmsnorm (xq / a_scales bit-identical to tvq_act_quant(y)). y and xq
 * may each be NULL (not both). */
int tvq_silu_mul(const void* gate_up, void* y, int8_t* xq, float* a_scales,
                 int dtype, int64_t M, int64_t I, void* stream);

/* Decode attention with the KV-cache append, one query token per sequence.
 * Replaces the decode branch of Attention.forward
 * (nanovllm/layers/attention.py:59-88: store_kvcache then
 * flash_attn_with_kvcache(..., cache_seqlens, causal=True)).
 *   q      [B, Hq, head_dim]   row stride q_stride (elements) between tokens
 *   k_new, v_new [B, Hkv, head_dim]  row strides k_stride / v_stride
 *   k_cache, v_cache [num_slots, Hkv, max_len, head_dim] (a slot per sequence)
 *   slots, lens [B] int32: sequence b owns slot slots[b] and has lens[b]
 *          tokens including the new one (1 <= lens[b] <= max_len); a
 *          sequence whose slot or length is out of range gets zeros and its
 *          cache is not touched
 *   out    [B, Hq, head_dim] contiguous
 * Writes k_new/v_new at position lens[b]-1 of the slot, then
 * out = softmax(scale * q K^T) V over positions 0..lens[b]-1 (fp32 math).
 * head_dim must be 128, Hq/Hkv in {1, 2, 4}, all pointers 16-byte aligned and
 * strides multiples of 8. Lengths and slots are read on the device: safe in
 * HIP-graph capture. */
int tvq_decode_attention(const void* q, int64_t q_stride, const void* k_new,
                         int64_t k_stride, const void* v_new, int64_t v_stride,
                         void* k_cache, void* v_cache, const int32_t* slots,
                         const int32_t* lens, int64_t B, int Hq, int Hkv,
                         int head_dim, int64_t num_slots, int64_t max_len,
                         float scale, void* out, int dtype, void* stream);

/* Per-head q/k RMSNorm and rotary embedding of one layer's attention input,
 * fused. Replaces q_norm / k_norm (RMSNorm.rms_forward,
 * nanovllm/layers/layernorm.py:16-26) followed by RotaryEmbedding.forward
 * (nanovllm/layers/rotary_embedding.py:6-14, 36-46; rotate-half).
 *   qkv        [T, row_stride] packed q|k|v projection output (q heads first,
 *              then Hkv key heads; values are not read)
 *   positions  [T] int64 (clamped to [0, max_pos))
 *   cos_t, sin_t [max_pos, head_dim/2] fp32
 *   q_weight, k_weight [head_dim] in `dtype`, or both NULL (rotation only)
 *   q_out [T, Hq, head_dim], k_out [T, Hkv, head_dim] contiguous
 *   k_cache, v_cache [num_slots, Hkv, max_len, head_dim] and slots [T] int64,
 *          or all NULL: when given, each token's rotated key and its value
 *          (read from qkv after the keys) are also stored at
 *          (slots[t], positions[t]) of the caches, replacing store_kvcache
 *          (attention.py:10-40) for prompt tokens; tokens whose slot or
 *          position is out of range are not stored.
 * head_dim must be 128; every pointer 16-byte aligned and row_stride a
 * multiple of 8 elements (TVQ_E_UNSUPPORTED otherwise). */
int tvq_qk_norm_rope(const void* qkv, int64_t row_stride,
                     const int64_t* positions, const float* cos_t,
                     const float* sin_t, const void* q_weight,
                     const void* k_weight, float eps, int64_t T, int Hq,
                     int Hkv, int head_dim, int64_t max_pos, void* q_out,
                     void* k_out, void* k_cache, void* v_cache,
                     const int64_t* slots, int64_t num_slots, int64_t max_len,
                     int dtype, void* stream);

/* Queries per row of the tvq_prefill_attention block table. */
#define TVQ_PREFILL_BLOCK_Q 64

/* Causal attention over the packed prompts of a prefill step (no cached
 * prefix). Replaces flash_attn_varlen_func(q, k, v, cu_seqlens..., causal=True)
 * in the prefill branch of Attention.forward (nanovllm/layers/attention.py:75-84).
 *   q [T, Hq, head_dim], k [T, Hkv, head_dim]   contiguous, packed tokens
 *   v [T, ...]  row stride v_stride elements, heads contiguous (head_dim each)
 *   blocks [nblocks, 3] int32: (token offset of the sequence, its length,
 *          first query of a TVQ_PREFILL_BLOCK_Q-query block), one row per
 *          query block
 *   out [T, Hq, head_dim] contiguous
 * out[t, h] = softmax(scale * q[t,h] . K_seq[0..pos]) V_seq[0..pos] over the
 * sequence's own keys up to its position (kv head h / (Hq/Hkv)). fp32 math;
 * the probabilities are rounded to `dtype` for the value product. head_dim
 * must be 128, Hq/Hkv an integer, pointers 16-byte aligned. */
int tvq_prefill_attention(const void* q, const void* k, const void* v,
                          int64_t v_stride, const int32_t* blocks,
                          int64_t nblocks, int Hq, int Hkv, int head_dim,
                          float scale, void* out, int dtype, void* stream);

/* The attention entry points with o_proj's per-token int8 quantization
 * fused into the same launch: the W8A8 QuantMethod's quantize_activation of
 * the attention output (quantize_int8_per_row_dynamic, reference
 * nanovllm/quantization/utils.py:28-32, applied to o_proj's input in
 * W8A8QuantMethod.apply, w8a8.py:21-40, called from linear.py:65-68), which
 * otherwise reads the output back in a separate tvq_act_quant launch.
 * Arguments as tvq_decode_attention / tvq_prefill_attention, plus
 *   xq [rows, Hq*head_dim] int8 and a_scales [rows] fp32: exactly what
 *          tvq_act_quant(out, eps) writes (rows = B, or the prompt tokens)
 *   counters int32 [counters_len], all zero on entry and left zero on
 *          return; counters_len >= B (decode) or nblocks (prefill); calls
 *          sharing a counters array must not overlap
 * `out` is still written (the quantizer's input). eps > 0; xq 4-byte
 * aligned. Each token row is quantized by the last of its workgroups to
 * finish; no workgroup waits for another. */
int tvq_decode_attention_quant(const void* q, int64_t q_stride,
                               const void* k_new, int64_t k_stride,
                               const void* v_new, int64_t v_stride,
                               void* k_cache, void* v_cache,
                               const int32_t* slots, const int32_t* lens,
                               int64_t B, int Hq, int Hkv, int head_dim,
                               int64_t num_slots, int64_t max_len, float scale,
                               void* out, int dtype, int8_t* xq,
                               float* a_scales, float eps, int32_t* counters,
                               int64_t counters_len, void* stream);

int tvq_prefill_attention_quant(const void* q, const void* k, const void* v,
                                int64_t v_stride, const int32_t* blocks,
                                int64_t nblocks, int Hq, int Hkv,
                                int head_dim, float scale, void* out,
                                int dtype, int8_t* xq, float* a_scales,
                                float eps, int32_t* counters,
                                int64_t counters_len, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TVQ_H_ */
