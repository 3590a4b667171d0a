/*
 * gr_decoder.h -- fused elementwise stages of the Qwen-style decoder that
 * drives the beam path end to end (libgr_beam.so).
 *
 * The reference serves its model through vLLM's model executor
 * (vllm==0.14, vllm_gr pyproject.toml:29, not vendored), whose custom ops
 * fused_add_rms_norm, rotary_embedding + reshape_and_cache_flash and
 * silu_and_mul these entry points replace.  Same conventions as gr_beam.h:
 * stream-ordered, no allocation, no host synchronisation, element strides,
 * float32 arithmetic with one rounding per stored element.
 */
#ifndef GR_DECODER_H_
#define GR_DECODER_H_

#include "gr_beam.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Residual add + RMSNorm over rows of `hidden` elements:
 *   residual == NULL: y = x
 *   residual != NULL: y = round(x + residual), written back to residual
 *   out = round(y * w / sqrt(mean(y^2) + eps))
 * out may alias x.  Rows at the given element strides.
 */
gr_status_t gr_rms_norm(void* out, int64_t out_stride, const void* x, int64_t x_stride,
                        void* residual, int64_t res_stride, const void* weight, int num_tokens,
                        int hidden, float eps, int dtype, hipStream_t stream);

/*
 * Per token t of qkv [num_tokens, (Hq + 2*Hkv) * head_dim] (q heads, then
 * k heads, then v heads): each q and k head is RMS-normalised over head_dim
 * with q_norm_weight / k_norm_weight (both NULL: no norm) and rotated by the
 * rotate-half rotary embedding at position positions[t] (int64): pair
 * (i, i + head_dim/2) turns by the angle whose cosine / sine are
 * cos_table / sin_table [table_len, head_dim/2] float32 at row positions[t].
 * Rotated queries go to q_out [num_tokens, Hq, head_dim]; rotated keys and the
 * values go to the paged cache at slot_mapping[t] (int64, block * block_size
 * + offset; < 0 skips the token's K/V; slot_mapping NULL writes no K/V).
 * A position outside [0, table_len) flags GR_DEV_BAD_LENGTH and skips the
 * token; a block id >= num_blocks flags GR_DEV_BAD_BLOCK and skips its K/V.
 */
gr_status_t gr_qk_norm_rope_cache(
    void* q_out, int64_t q_out_stride, const void* qkv, int64_t qkv_stride,
    const int64_t* positions, const float* cos_table, const float* sin_table, int64_t table_len,
    const void* q_norm_weight, const void* k_norm_weight,
    void* k_cache, void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int64_t* slot_mapping, int block_size, int num_tokens,
    int num_q_heads, int num_kv_heads, int head_dim, float eps, int dtype,
    int32_t* dev_status, hipStream_t stream);

/*
 * SwiGLU gate: out[t, i] = round(silu(x[t, i]) * x[t, ffn + i]) for
 * x [num_tokens, 2 * ffn] (gate | up), silu(g) = g / (1 + exp(-g)).
 * num_tokens <= 65535.
 */
gr_status_t gr_silu_mul(void* out, int64_t out_stride, const void* x, int64_t x_stride,
                        int num_tokens, int ffn, int dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* GR_DECODER_H_ */
