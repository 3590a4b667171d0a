/*
 * gr_beam.h -- C ABI of the MI355X (gfx950) beam-aware KV-cache hot path.
 *
 * One shared library (libgr_beam.so) exports these entry points.  Every call
 * is stream-ordered on the HIP stream it is given, allocates nothing, does
 * no host synchronisation, and returns a gr_status_t.  Pointers are device
 * pointers unless stated otherwise.  Element strides are in elements, not
 * bytes.  The paged KV cache keeps the reference's per-K/V layout
 * [num_blocks, block_size, num_kv_heads, head_dim] with head_dim contiguous
 * (vllm_gr/v1/attention/backends/beam_attn.py:784-785); other block layouts
 * (the HND stride order, :787-798) are expressed through the three strides.
 *
 * Table contents (block ids, lengths, parents) live on the device, so the
 * library cannot reject them before launch; kernels skip any access they
 * would make out of bounds and OR a GR_DEV_* bit into *dev_status (when not
 * NULL), which the caller may read back after the stream completes.
 */
#ifndef GR_BEAM_H_
#define GR_BEAM_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int gr_status_t;
enum {
  GR_OK = 0,
  GR_ERR_INVALID_ARG = 1, /* bad size, stride, pointer or combination */
  GR_ERR_UNSUPPORTED = 2, /* valid but not implemented (dtype, head size) */
  GR_ERR_LAUNCH = 3,      /* the HIP runtime refused the launch */
  GR_ERR_WORKSPACE = 4    /* workspace missing or too small */
};

/* bits OR-ed into *dev_status by kernels */
enum {
  GR_DEV_BAD_BLOCK = 1,   /* block id outside [0, num_blocks) */
  GR_DEV_BAD_LENGTH = 2,  /* length beyond the block-table row capacity */
  GR_DEV_BAD_PARENT = 4,  /* parent index outside [0, beam width) */
  GR_DEV_SUFFIX_FULL = 8, /* append past the row capacity (token dropped) */
  GR_DEV_BAD_NODE = 16    /* catalog node id or child range outside the trie */
};

enum { GR_DTYPE_F32 = 0, GR_DTYPE_F16 = 1, GR_DTYPE_BF16 = 2,
       /* KV-cache element type only: OCP fp8 e4m3 (float8_e4m3fn: 1 sign, 4
        * exponent bits with bias 7, 3 mantissa bits, no infinities, 0x7F/0xFF
        * NaN, largest finite 448) -- the reference's fp8 / fp8_e4m3 cache
        * (beam_attn.py:617-618, :734-737, :801-804) */
       GR_DTYPE_FP8_E4M3 = 3 };

/* Human-readable name of a status code (static storage). */
const char* gr_status_string(gr_status_t status);
/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int gr_version(void);
/* Decode kernel selection for tests and measurement (no reference
 * counterpart): 0 = automatic (the matrix-core kernel where supported, else
 * the generic one), 1 = always the generic kernel.  Process-wide. */
gr_status_t gr_set_decode_kernel(int which);

/*
 * BeamAttention decode step.
 *
 * Replaces BeamAttentionImpl.cascade_attention
 * (vllm_gr/v1/attention/backends/beam_attn.py:629-701): the flash-attention
 * prefix pass (:656-678), the Triton suffix gather (:679-684, :62-117), the
 * suffix pass (:686-695) and merge_attn_states (:697-699), as one launch.
 *
 * Request r owns prefix tokens [0, prefix_len[r]) of block-table row
 * prefix_bt[r * prefix_bt_stride ...] and beams [beam_start[r],
 * beam_start[r+1]).  Beam n owns suffix_len[n] suffix tokens; token j sits at
 * logical position (suffix_start ? suffix_start[n] : 0) + j of row
 * suffix_bt[n * suffix_bt_stride ...] (capacity suffix_bt_stride blocks).
 * Each beam has q_per_beam query tokens: rows n*q_per_beam + i of q/out.
 * Query i sees the whole prefix and suffix tokens j <= L - q_per_beam + i
 * (bottom-right causal, the suffix pass's causal=True at :693).
 * GQA: query head h reads KV head h / (num_q_heads / num_kv_heads) (:612).
 * score = scale * q.k, soft-capped as softcap*tanh(score/softcap) when
 * softcap > 0 (:607-609).  Rows with no visible key get output 0 and LSE
 * -inf.  lse_out (nullable) receives the natural-log LSE as
 * [num_beams*q_per_beam, num_q_heads] float32.
 * q and out are [num_beams*q_per_beam, num_q_heads, head_dim] with token
 * strides q_tok_stride / out_tok_stride; head_dim % 8 == 0, head_dim <= 256
 * (BeamAttentionBackend.supports_head_size, :807-808).
 */
gr_status_t gr_beam_attn_decode(
    void* out, int64_t out_tok_stride,
    const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start,
    const int32_t* suffix_bt, int suffix_bt_stride, const int32_t* suffix_len,
    const int32_t* suffix_start,
    int num_reqs, int max_beams_per_req, int num_beams, int q_per_beam,
    int num_q_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
    float scale, float softcap, float* lse_out, int32_t* dev_status, hipStream_t stream);

/*
 * gr_beam_attn_decode with a split prefix for small batches.
 *
 * Same arguments and results as gr_beam_attn_decode.  When the batch's row
 * tiles (requests x KV heads x beam rows / 128) would leave the GPU's 256
 * compute units idle, each tile's prefix is split over several workgroups
 * that write partial outputs and LSEs to `workspace`, and a second kernel on
 * the same stream merges them as merge_attn_states does
 * (beam_attn.py:697-699).  max_prefix_len (host hint, 0 = unknown) keeps at
 * least 256 prefix keys per split.  workspace: device memory of
 * gr_beam_attn_decode_workspace_size() bytes (0 = no split: workspace may be
 * NULL), 256-byte aligned, no initial contents.  Calls that share one
 * workspace must not overlap (one stream).
 */
size_t gr_beam_attn_decode_workspace_size(int num_reqs, int max_beams_per_req, int q_per_beam,
                                          int num_q_heads, int num_kv_heads, int head_dim,
                                          int max_prefix_len);
gr_status_t gr_beam_attn_decode_ws(
    void* out, int64_t out_tok_stride,
    const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start,
    const int32_t* suffix_bt, int suffix_bt_stride, const int32_t* suffix_len,
    const int32_t* suffix_start,
    int num_reqs, int max_beams_per_req, int num_beams, int q_per_beam,
    int num_q_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
    float scale, float softcap, float* lse_out, int32_t* dev_status,
    int max_prefix_len, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Varlen causal attention of the standard (non-beam) requests of a batch --
 * prefill chunks and single-token decodes -- over the paged KV cache.
 *
 * Replaces flash_attn_varlen_func(cu_seqlens_q, seqused_k, causal=True,
 * block_table) on the standard path of the reference's cascade attention
 * (vllm_gr/v1/attention/backends/beam_attn.py:643-654).
 *
 * Request r owns query rows query_start[r] .. query_start[r+1]-1 of q/out
 * (ql = their count <= max_query_len) and seq_len[r] keys in block-table row
 * block_table[r * bt_stride ...], its new tokens' K/V already written there.
 * Query i of request r sees keys 0 .. seq_len[r] - ql + i (bottom-right
 * causal).  GQA, scale, softcap, LSE and row layout as in
 * gr_beam_attn_decode; q/out [num_tokens, num_q_heads, head_dim].  Table
 * contents are checked on the device (GR_DEV_BAD_LENGTH for an inconsistent
 * request, which is then skipped; GR_DEV_BAD_BLOCK for a block id outside
 * the pool, whose keys read as zeros).
 */
gr_status_t gr_paged_attn_prefill(
    void* out, int64_t out_tok_stride,
    const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* block_table, int bt_stride, const int32_t* query_start,
    const int32_t* seq_len, int num_reqs, int num_tokens, int max_query_len,
    int num_q_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
    float scale, float softcap, float* lse_out, int32_t* dev_status, hipStream_t stream);

/*
 * Optional attention features: the sliding window, attention sinks and ALiBi
 * slopes BeamAttentionImpl takes (vllm_gr/v1/attention/backends/beam_attn.py:
 * 597-625) and hands to every flash_attn_varlen_func call of the cascade
 * (window_size, alibi_slopes, s_aux: :643-695), and the non-causal standard
 * path of the encoder attention types (causal flag, :648; ENCODER,
 * ENCODER_ONLY, ENCODER_DECODER accepted at :771-773).
 *
 * Positions are indices into a row's key sequence: a request's prefix
 * (decode: shared prefix then the beam's own suffix), a query sitting at its
 * own token's position.  A key at kpos is visible to a query at qpos when
 * qpos - window_left <= kpos (window_left >= 0) and kpos <= qpos +
 * window_right (window_right >= 0, non-causal prefill only); -1 = unbounded.
 * The reference's sliding_window w maps to window_left = w - 1 (decoder: right
 * 0) or left = right = w - 1 (ENCODER_ONLY).  alibi_slopes[h] adds
 * -slope * |qpos - kpos| to the (soft-capped) score; sinks[h] joins head h's
 * softmax as one more logit without a value (natural-log units).  causal = 0
 * (prefill only) lets every query see all of its sequence's keys.  Passing
 * NULL options is the same as the functions without _opt.
 */
typedef struct gr_attn_options {
  int window_left;            /* -1: no left bound */
  int window_right;           /* -1: no right bound (non-causal prefill only) */
  int causal;                 /* 1: causal (required for decode); 0: prefill over every key */
  const float* sinks;         /* [num_q_heads] or NULL */
  const float* alibi_slopes;  /* [num_q_heads] or NULL */
  /* GR_DTYPE_FP8_E4M3: the caches hold fp8 e4m3 elements, read as
   * fp8_value * k_scale[0] (K) and * v_scale[0] (V); any other value: the
   * caches hold elements of `dtype`, like q */
  int kv_dtype;
  const float* k_scale;       /* [1] device float, or NULL for 1.0 */
  const float* v_scale;       /* [1] device float, or NULL for 1.0 */
} gr_attn_options;

/* gr_beam_attn_decode_ws with options.  bf16/fp16 head-dim-128 decodes with a
 * left window, sinks, ALiBi and / or an fp8 cache run on the matrix-core
 * kernel (split like a plain decode when a workspace is given); a right
 * window, fp32 or another head size takes the generic kernel. */
gr_status_t gr_beam_attn_decode_opt(
    void* out, int64_t out_tok_stride,
    const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start,
    const int32_t* suffix_bt, int suffix_bt_stride, const int32_t* suffix_len,
    const int32_t* suffix_start,
    int num_reqs, int max_beams_per_req, int num_beams, int q_per_beam,
    int num_q_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
    float scale, float softcap, float* lse_out, int32_t* dev_status,
    int max_prefix_len, void* workspace, size_t workspace_bytes,
    const gr_attn_options* options, hipStream_t stream);

/* gr_paged_attn_prefill with options.  Causal bf16/fp16 head-dim-128 prefills
 * with sinks and / or an fp8 cache run on the matrix-core kernel (head dim 64
 * too, with an even KV head count: adjacent KV heads read as one 128-dim
 * head); windows, ALiBi, non-causal batches, fp32 and other head sizes take
 * the generic kernel. */
gr_status_t gr_paged_attn_prefill_opt(
    void* out, int64_t out_tok_stride,
    const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* block_table, int bt_stride, const int32_t* query_start,
    const int32_t* seq_len, int num_reqs, int num_tokens, int max_query_len,
    int num_q_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
    float scale, float softcap, float* lse_out, int32_t* dev_status,
    const gr_attn_options* options, hipStream_t stream);

/*
 * Scatter new K/V tokens into the paged cache by flat slot
 * (slot = block * block_size + offset; slot < 0 is skipped).
 *
 * Replaces reshape_and_cache_flash as called by BeamAttentionImpl.forward
 * (vllm_gr/v1/attention/backends/beam_attn.py:727-732).
 * key/value: [num_tokens, num_kv_heads, head_dim], token stride in elements.
 */
gr_status_t gr_reshape_and_cache(
    const void* key, int64_t key_tok_stride, const void* value, int64_t value_tok_stride,
    void* k_cache, void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int64_t* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
    int block_size, int dtype, int32_t* dev_status, hipStream_t stream);

/*
 * gr_reshape_and_cache into an fp8 e4m3 cache: each element is stored as
 * e4m3(clamp(x / scale, -448, 448)), rounded to nearest even (x of `dtype`,
 * scale = k_scale[0] / v_scale[0], NULL for 1.0) -- reshape_and_cache_flash
 * with the layer's _k_scale / _v_scale and an fp8 kv_cache_dtype
 * (beam_attn.py:727-732).  Strides count elements of their own tensors;
 * head_dim a multiple of 4.
 */
gr_status_t gr_reshape_and_cache_fp8(
    const void* key, int64_t key_tok_stride, const void* value, int64_t value_tok_stride,
    void* k_cache, void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int64_t* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
    int block_size, int dtype, const float* k_scale, const float* v_scale, int32_t* dev_status,
    hipStream_t stream);

/*
 * Beam KV fork, optionally fused with the append of one new token per beam.
 *
 * Replaces the reference's per-step suffix rebuild: _mega_request_step
 * (vllm_gr/entrypoints/openai/serving_engine.py:107-120: child suffix =
 * parent's tokens ++ chosen token), _handle_mega_request_step_update
 * (vllm_gr/v1/engine/core.py:108-112) and the whole-prefix-block cache cap
 * that forces the suffix to be recomputed
 * (vllm_gr/v1/engine/engine_core_patch.py:245-252).
 *
 * parent [num_reqs, beam_width]: parent beam (within the request) of each
 * child.  A parent's lowest-index child inherits its row in place; every
 * other child takes, in ascending order, the row of the next childless
 * parent of the same request (ascending), and receives a copy of the
 * parent's suffix_len valid tokens.  Tables are written out of place:
 * bt_out/len_out must not alias bt_in/len_in.  When k_new/v_new
 * ([num_reqs*beam_width, num_kv_heads, head_dim]) are given, each child's
 * token is appended at position len_out[c] and len_out[c] is incremented.
 * dtype may be GR_DTYPE_FP8_E4M3 (the copies move bytes; k_new/v_new then
 * hold e4m3 elements; the same holds for gr_beam_kv_append).
 */
gr_status_t gr_beam_kv_fork(
    const int32_t* parent, int num_reqs, int beam_width,
    const int32_t* bt_in, const int32_t* len_in, int32_t* bt_out, int32_t* len_out,
    int bt_stride,
    void* k_cache, void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const void* k_new, const void* v_new, int64_t new_tok_stride,
    int num_kv_heads, int head_dim, int block_size, int dtype,
    int32_t* dev_status, hipStream_t stream);

/*
 * gr_beam_kv_fork over every layer's cache in one launch (without the
 * appended token, which the next forward writes per layer).  Replaces the
 * same reference code as gr_beam_kv_fork (serving_engine.py:107-120,
 * core.py:108-112, engine_core_patch.py:245-252), which touches all layers at
 * once since the child's suffix is recomputed through the whole model.
 * k_caches/v_caches: host arrays of num_layers base pointers, every layer
 * with the same geometry (strides, num_blocks, heads, dims, block size,
 * dtype); the tables are worked out once per launch and each workgroup copies
 * its share of the copy-on-write tokens in every layer (up to 32 layers per
 * launch; more take further launches on the same stream).
 */
gr_status_t gr_beam_kv_fork_layers(
    const int32_t* parent, int num_reqs, int beam_width,
    const int32_t* bt_in, const int32_t* len_in, int32_t* bt_out, int32_t* len_out,
    int bt_stride, int num_layers,
    void* const* k_caches, void* const* v_caches, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    int num_kv_heads, int head_dim, int block_size, int dtype,
    int32_t* dev_status, hipStream_t stream);

/*
 * Append one K/V token per beam at position suffix_len[n] of its row and
 * increment suffix_len[n] (in place).  The reshape_and_cache_flash role
 * (beam_attn.py:727-732) in block-table form.
 */
gr_status_t gr_beam_kv_append(
    const void* k_new, const void* v_new, int64_t new_tok_stride,
    void* k_cache, void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* suffix_bt, int bt_stride, int32_t* suffix_len, int num_beams,
    int num_kv_heads, int head_dim, int block_size, int dtype,
    int32_t* dev_status, hipStream_t stream);

/*
 * Fused beam pruning: log_softmax + cumulative logprob + top-k over
 * beams x vocab, per request.
 *
 * Replaces the sampler's logprobs=W top-K (serving_engine.py:300-308) and the
 * host pruning body (vllm_gr/entrypoints/openai/serving_engine.py:457-592;
 * offline twin vllm_gr/entrypoints/llm.py:201-280).
 *
 * logits [num_reqs*beam_width, vocab] float32 (row stride logits_row_stride,
 * vocab % 4 == 0, 16-byte aligned rows), cum [num_reqs*beam_width] float32.
 * score(b, v) = (double)x + ((double)cum[b] - lse[b]), lse[b] = (double)m +
 * log(S) with m the row max and S the float32 sum of exp(x - m), each term
 * computed as exp2 of (x - m) * log2(e) by a degree-5 polynomial fit and
 * summed in a fixed order (256 threads x float4 groups, then a xor
 * butterfly per 64-lane wave, then (w0 + w1) + (w2 + w3)); the log is an
 * atanh-series float64 evaluation.  All steps are single IEEE operations, so
 * a CPU restatement reproduces every score bit for bit.
 * Stage 1: each beam's top-k by (logit desc, token
 * asc); a candidate equal to eos_token_id (>= 0) leaves the pool and its
 * score goes to eos_score[b] (nullable; -inf when absent) -- the EOS split
 * of :541-562.  Stage 2: top-k of the union by (score desc, flat index asc),
 * flat = b * vocab + v.  Outputs [num_reqs, k]: parent beam, token, score
 * (float32 of the float64 score); unfilled slots get -1, -1, -inf.
 * Requires 1 <= k <= 1024 and k <= vocab.  workspace: device memory of
 * gr_beam_prune_workspace_size() bytes, 256-byte aligned.
 */
size_t gr_beam_prune_workspace_size(int num_reqs, int beam_width, int vocab, int k);

/*
 * gr_beam_prune_topk constrained by a catalog of valid semantic-ID token
 * sequences (the reference's Catalog trie, vllm_gr/entrypoints/openai/
 * serving_models.py:18-49, applied at serving_engine.py:381-394, 504-506,
 * 526-528).
 *
 * The trie is given in CSR form: node n's children are
 * child_token[node_start[n] .. node_start[n+1]) (ascending) with node ids
 * child_node[...]; node 0 is the root.  beam_node[b] (int32 [R*W]) is the
 * node reached by beam b's generated tokens (-1: none, as Catalog.valid
 * returns the empty set).  Stage 1 is unchanged -- each beam's top-k by
 * (logit desc, token asc) -- and then, as the reference masks after the
 * sampler's per-beam top-K, every candidate that is not a child of the
 * beam's node leaves the pool (EOS reports its score only when it is a
 * child).  node_out [R, k] receives each selected beam's new node (-1 for an
 * unfilled slot).  Same workspace as gr_beam_prune_topk.  Node ids and child
 * ranges outside the trie flag GR_DEV_BAD_NODE in *dev_status (nullable) and
 * read as childless.
 */
gr_status_t gr_beam_prune_topk_catalog(
    const float* logits, int64_t logits_row_stride, const float* cum,
    int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
    const int32_t* beam_node, const int32_t* node_start, const int32_t* child_token,
    const int32_t* child_node, int num_nodes, int num_edges,
    int32_t* parent, int32_t* token, float* score, float* eos_score, int32_t* node_out,
    void* workspace, size_t workspace_bytes, int32_t* dev_status, hipStream_t stream);

gr_status_t gr_beam_prune_topk(
    const float* logits, int64_t logits_row_stride, const float* cum,
    int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
    int32_t* parent, int32_t* token, float* score, float* eos_score,
    void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * gr_beam_prune_topk without a workspace argument: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 *
 * Same arguments (minus workspace / workspace_bytes), kernels and results as
 * gr_beam_prune_topk.  The workspace is a static device array of
 * GR_PRUNE_SCRATCH_BYTES per GPU (held until the process ends; the device
 * address is looked up on the first call on each device, which must be the
 * current device, the stream's).  A call whose gr_beam_prune_workspace_size
 * exceeds GR_PRUNE_SCRATCH_BYTES returns GR_ERR_WORKSPACE and launches
 * nothing.  The call allocates nothing.  Every call on one GPU shares that
 * array: calls that may overlap on one GPU (different streams, or host
 * threads) race and must be serialised by the caller.
 */
#define GR_PRUNE_SCRATCH_BYTES ((size_t)16 << 20)
gr_status_t gr_beam_prune_topk_noalloc(
    const float* logits, int64_t logits_row_stride, const float* cum,
    int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
    int32_t* parent, int32_t* token, float* score, float* eos_score, hipStream_t stream);

/*
 * gr_beam_prune_topk / gr_beam_prune_topk_catalog with the beam scores
 * carried in float64 between steps.
 *
 * The reference keeps each beam's cumulative logprob as a Python float
 * (float64) from step to step and adds the new token's logprob to it in
 * float64 (vllm_gr/entrypoints/openai/serving_engine.py:511, :538-539;
 * offline twin vllm_gr/entrypoints/llm.py:231-245).  cum [R*W] float64 is
 * used as is (c_b = cum[b] - lse[b]); score [R, k] and eos_score [R*W]
 * receive the float64 scores themselves, not their float32 roundings, so a
 * multi-step search never rounds a beam's score.  One departure: a
 * candidate's score is cum + (x - lse) rounded once in float64, where the
 * reference adds the sampler's float32 logprob, cum + float64(float32(x -
 * lse)); the two differ by at most one float32 ulp of the logprob.  Selection, order, ties
 * and workspace as in gr_beam_prune_topk.  beam_node == NULL: no catalog
 * (the trie arguments and node_out are ignored); otherwise the catalog mode
 * of gr_beam_prune_topk_catalog.
 *
 * cand_token / cand_logprob [R*W, k] (both NULL or both given) receive each
 * beam's top-k by (logit desc, token asc) before EOS or the catalog take
 * anything out, with logprob = float32(x - lse) -- the per-step lists the
 * reference keeps for every beam and rebuilds along parent pointers
 * (vllm_gr/logprobs.py:34-53 extract_and_dedup_flat_logprobs, :56-85
 * reconstruct_beam_logprobs; vllm_gr/entrypoints/llm.py:203-220).
 */
gr_status_t gr_beam_prune_topk_f64(
    const float* logits, int64_t logits_row_stride, const double* cum,
    int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
    const int32_t* beam_node, const int32_t* node_start, const int32_t* child_token,
    const int32_t* child_node, int num_nodes, int num_edges,
    int32_t* parent, int32_t* token, double* score, double* eos_score, int32_t* node_out,
    int32_t* cand_token, float* cand_logprob,
    void* workspace, size_t workspace_bytes, int32_t* dev_status, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* GR_BEAM_H_ */
