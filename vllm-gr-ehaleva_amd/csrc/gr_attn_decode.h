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
};

// MFMA path (gr_attn_mfma.hip): bf16/fp16, head_dim 128, 16-byte aligned rows.
bool mfma_decode_supported(const DecodeArgs& a);
gr_status_t launch_mfma_decode(const DecodeArgs& a, hipStream_t stream);
// Varlen causal mode of the same kernel (see gr_paged_attn_prefill).
gr_status_t launch_mfma_prefill(const DecodeArgs& a, hipStream_t stream);

// 0 = choose automatically, 1 = always the generic kernel (testing hook).
extern int g_decode_kernel_override;

}  // namespace gr
