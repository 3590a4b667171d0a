// Kernel argument block shared by the BeamAttention decode kernels.
#pragma once

#include "gr_common.h"

namespace gr {

struct DecodeArgs {
  void* out;
  int64_t out_tok_stride;
  const void* q;
  int64_t q_tok_stride;
  const void* k_cache;
  const void* v_cache;
  int64_t num_blocks;
  int64_t kv_block_stride, kv_tok_stride, kv_head_stride;
  const int32_t* prefix_bt;
  int prefix_bt_stride;
  const int32_t* prefix_len;
  const int32_t* beam_start;
  const int32_t* suffix_bt;
  int suffix_bt_stride;
  const int32_t* suffix_len;
  const int32_t* suffix_start;
  int num_reqs, max_beams, num_beams, T, Hq, Hkv, D, bs, dtype;
  int bs_shift;  // log2(bs) when bs is a power of two, else -1
  float scale, softcap;
  float* lse_out;
  int32_t* dev_status;
  // split prefix (MFMA decode only): nsplit workgroups share each row tile's
  // prefix; each writes its normalised partial O / LSE, a second kernel merges
  int nsplit;
  uint16_t* ws_o;  // [tiles * nsplit][128 rows][128] in the query dtype
  float* ws_lse;  // [tiles * nsplit][128 rows] float32 (natural log)
  // optional features (gr_attn_options); positions are indices into the
  // row's [prefix ; suffix] sequence, a query row sitting at its own token's
  int win_left, win_right;   // keys before / after the query's position it sees; -1 = unbounded
  int causal;                // prefill: 0 = every key of the sequence (decode is always causal)
  const float* sinks;        // [Hq] sink logits (natural log units) or null
  const float* alibi;        // [Hq] ALiBi slopes or null
  int kv8;                   // the caches hold fp8 e4m3 elements (dequantised by k_scale / v_scale)
  // head pairs (matrix-core kernel, head_dim 64): KV heads 2j and 2j + 1
  // read as one 128-dim head j; each query row fills and writes only its own
  // head's half of the 128 dims (mfma_pair_args).  (In kv8's padding: the
  // block's size and layout stay as they were.)
  int pair;
  const float* k_scale;      // [1] or null (1.0)
  const float* v_scale;      // [1] or null (1.0)
};


// MFMA path (gr_attn_mfma.hip): bf16/fp16, head_dim 128, 16-byte aligned rows.
// (decode: sinks, a left window and ALiBi run here too; prefill: sinks)
bool mfma_decode_supported(const DecodeArgs& a);
bool mfma_prefill_supported(const DecodeArgs& a);
// head_dim 64 on the matrix-core kernel: p = a with adjacent KV head pairs as
// 128-dim heads, when the cache allows it (an even KV head count, heads 64
// elements apart) and the kernel takes p.
bool mfma_pair_args(const DecodeArgs& a, DecodeArgs& p);
gr_status_t launch_mfma_decode(const DecodeArgs& a, hipStream_t stream);
// Varlen causal mode of the same kernel (see gr_paged_attn_prefill).
gr_status_t launch_mfma_prefill(const DecodeArgs& a, hipStream_t stream);
// Split-prefix decode (a.nsplit > 1, workspace set): the decode kernel, then
// the merge of its partials.
gr_status_t launch_mfma_decode_split(const DecodeArgs& a, hipStream_t stream);
// Row tiles of the MFMA decode grid and the prefix split it would use.
void mfma_decode_plan(int num_reqs, int max_beams, int q_per_beam, int Hq, int Hkv, int max_prefix_len,
                      int* tiles, int* nsplit);

// 0 = choose automatically (the MFMA kernel where supported), 1 = always the
// generic kernel (testing and measurement hook).
extern int g_decode_kernel_override;

}  // namespace gr
