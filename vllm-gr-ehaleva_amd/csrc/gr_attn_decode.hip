// BeamAttention decode for gfx950.
//
// One launch computes, for every beam's query rows, softmax attention over
// [shared prefix ; own suffix] -- the work the reference spreads over a
// flash-attention prefix pass, a Triton suffix gather, a suffix pass and an
// LSE merge (vllm_gr/v1/attention/backends/beam_attn.py:629-701).
//
// Two kernels sit behind gr_beam_attn_decode:
//  * decode_generic: any dtype (fp32/fp16/bf16), head_dim % 8 == 0 <= 256.
//    One workgroup per (request, KV head, 32-row chunk of the request's beam
//    rows): the chunk's beams share each prefix tile; fp32 VALU math.
//  * the MFMA kernel in gr_attn_mfma.hip for bf16/fp16 at head_dim 128,
//    which stages each request's prefix tile once in LDS for all its beams.
#include "gr_common.h"
#include "gr_attn_decode.h"

namespace gr {

constexpr int GEN_ROWS = 32;     // query rows per workgroup
constexpr int GEN_TK = 32;       // keys per tile
constexpr int GEN_THREADS = 256;
constexpr int GEN_ACC = GEN_ROWS * 256 / GEN_THREADS;  // acc slots per thread at D=256
constexpr int GEN_KPAD = 4;      // floats past each staged K row: 16-byte rows, keys spread over banks

// PREFILL: the varlen mode (gr_paged_attn_prefill): blockIdx.x / chunks is
// the request, prefix_bt / prefix_len its block table and sequence length,
// beam_start its query start, T the largest query count; query i of a request
// with ql queries sees keys 0 .. seq - ql + i (causal) or all seq keys, and
// there is no suffix.
// Options (gr_attn_options): a key or query position is its index in the
// row's [prefix ; suffix] sequence (a query sits at its own token's); a
// window keeps keys with qpos - win_left <= kpos <= qpos + win_right; ALiBi
// adds -slope * |qpos - kpos| after the soft cap; a sink adds exp(sink) to
// the softmax denominator (beam_attn.py:597-625, flash_attn_varlen_func's
// window_size / alibi_slopes / s_aux).
// KV8: the caches hold fp8 e4m3 elements, dequantised on load by the
// per-tensor scales (value = e4m3 * scale).
// Decode: the chunk's rows belong to consecutive beams b_lo .. of request r
// (row rho of the request: beam rho / (T G), query (rho / G) % T, head
// rho % G).  Its keys are the prefix, then the chunk's beams' suffixes one
// after another (slot j of the concatenation: the beam whose cumulative
// lengths cover it); a suffix key is visible to the rows of its own beam only.
template <int DT, bool PREFILL = false, bool KV8 = false>
__global__ __launch_bounds__(GEN_THREADS) void decode_generic(DecodeArgs a) {
  using E = Elem<DT>;
  using S = typename E::storage;
  extern __shared__ float smem[];
  __shared__ int c_len[GEN_ROWS];       // decode: the chunk's beams' validated suffix lengths
  __shared__ int c_s0[GEN_ROWS];        // ... their first suffix positions
  __shared__ int c_cum[GEN_ROWS + 1];   // ... cumulative lengths (slot of each beam's first key)
  __shared__ int64_t k_off[GEN_TK];     // per tile key: element offset of its head-0 row (valid keys)
  __shared__ int k_beam[GEN_TK];        // ... chunk beam of a suffix key, -1 for a prefix key
  __shared__ int k_pos[GEN_TK];         // ... position in [prefix ; own suffix]
  const int D = a.D;
  float* q_s = smem;                              // [ROWS][D]
  const int KP = D + GEN_KPAD;
  float* k_s = q_s + GEN_ROWS * D;                // [TK][D+KPAD]
  float* v_s = k_s + GEN_TK * KP;                 // [TK][D]
  float* p_s = v_s + GEN_TK * D;                  // [ROWS][TK+1]
  float* m_s = p_s + GEN_ROWS * (GEN_TK + 1);     // [ROWS]
  float* l_s = m_s + GEN_ROWS;                    // [ROWS]
  float* a_s = l_s + GEN_ROWS;                    // [ROWS]
  int* kv_ok = reinterpret_cast<int*>(a_s + GEN_ROWS);  // [TK]

  const int G = a.Hq / a.Hkv;
  const int TG = a.T * G;  // decode: rows per beam
  const int chunks = PREFILL ? (TG + GEN_ROWS - 1) / GEN_ROWS : (a.max_beams * TG + GEN_ROWS - 1) / GEN_ROWS;
  const int r = blockIdx.x / chunks;
  const int chunk = blockIdx.x % chunks;
  const int hk = blockIdx.y;
  const int t = threadIdx.x;
  if (r >= a.num_reqs) return;
  const int row0 = chunk * GEN_ROWS;
  const int pre_cap = a.prefix_bt_stride * a.bs;
  int P, nrows, Pc, Lsum = 0, ctx = 0, nb0 = 0, b_lo = 0;
  int64_t tok0 = 0;  // prefill: token row of the request's first query
  if constexpr (PREFILL) {
    const int q0 = a.beam_start[r], ql = a.beam_start[r + 1] - q0, seq = a.prefix_len[r];
    if (q0 < 0 || ql < 0 || q0 + ql > a.num_beams || ql > a.T || seq < ql || seq > pre_cap) {
      if (t == 0 && chunk == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
      return;
    }
    if (row0 >= G * ql) return;
    nrows = min(GEN_ROWS, G * ql - row0);
    ctx = seq - ql;
    // keys up to the chunk's last query token (all of them when non-causal)
    P = Pc = a.causal ? ctx + (row0 + nrows - 1) / G + 1 : seq;
    tok0 = q0;
  } else {
    nb0 = a.beam_start[r];
    const int W = a.beam_start[r + 1] - nb0;
    // beam_start is device data: never trust it (a request past max_beams
    // would leave rows no workgroup computes)
    if (nb0 < 0 || W < 0 || nb0 + W > a.num_beams || W > a.max_beams) {
      if (t == 0 && chunk == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
      return;
    }
    if (row0 >= W * TG) return;
    nrows = min(GEN_ROWS, W * TG - row0);
    P = a.prefix_len[r];
    Pc = min(max(P, 0), pre_cap);
    if (t == 0 && chunk == 0 && Pc != P) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
    b_lo = row0 / TG;
    const int nbm = (row0 + nrows - 1) / TG - b_lo + 1;  // beams in the chunk (<= GEN_ROWS)
    if (t < nbm) {
      const int n = nb0 + b_lo + t;
      const int L = a.suffix_len[n], s0 = a.suffix_start ? a.suffix_start[n] : 0;
      const int suf_cap = a.suffix_bt_stride * a.bs;
      const int Lc = (L < 0 || s0 < 0 || s0 + L > suf_cap) ? 0 : L;
      if (Lc != L) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
      c_len[t] = Lc;
      c_s0[t] = s0;
    }
    __syncthreads();
    if (t == 0) {
      int c = 0;
      for (int j = 0; j < nbm; ++j) {
        c_cum[j] = c;
        c += c_len[j];
      }
      c_cum[nbm] = c;
    }
    __syncthreads();
    Lsum = c_cum[nbm];
  }
  // the chunk beam of a row, and its query index within the beam
  auto row_beam = [&](int row) { return (row0 + row) / TG - b_lo; };
  auto row_qi = [&](int row) { return PREFILL ? (row0 + row) / G : ((row0 + row) / G) % a.T; };
  // token row (of q / out) of a chunk row
  auto row_tok = [&](int row) -> int64_t {
    return PREFILL ? tok0 + row_qi(row) : (int64_t)(nb0 + b_lo + row_beam(row)) * a.T + row_qi(row);
  };

  const S* q = static_cast<const S*>(a.q);
  const S* kc = static_cast<const S*>(a.k_cache);
  const S* vc = static_cast<const S*>(a.v_cache);
  const uint8_t* kc8 = static_cast<const uint8_t*>(a.k_cache);
  const uint8_t* vc8 = static_cast<const uint8_t*>(a.v_cache);
  const float k_sc = KV8 && a.k_scale ? a.k_scale[0] : 1.f, v_sc = KV8 && a.v_scale ? a.v_scale[0] : 1.f;
  // every key row's eight-element chunks start on a vector boundary: bases
  // and strides in whole vectors (16 bytes; 8 for fp8)
  const int vbytes = KV8 ? 8 : 16, esz = KV8 ? 1 : (int)sizeof(S);
  const bool vec = (reinterpret_cast<uintptr_t>(a.k_cache) % vbytes) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.v_cache) % vbytes) == 0 && (a.kv_block_stride * esz) % vbytes == 0 &&
                   (a.kv_tok_stride * esz) % vbytes == 0 && (a.kv_head_stride * esz) % vbytes == 0;

  for (int e = t; e < GEN_ROWS * D; e += GEN_THREADS) {
    int row = e / D, d = e % D;
    float v = 0.f;
    if (row < nrows) {
      const int g = (row0 + row) % G;
      v = E::to_float(q[row_tok(row) * a.q_tok_stride + (int64_t)(hk * G + g) * D + d]);
    }
    q_s[e] = v;
  }
  if (t < GEN_ROWS) {
    m_s[t] = -INFINITY;
    l_s[t] = 0.f;
  }
  float acc[GEN_ACC];
#pragma unroll
  for (int i = 0; i < GEN_ACC; ++i) acc[i] = 0.f;

  // keys of the workgroup: the prefix (prefill: up to the chunk's last query),
  // then (decode) the chunk's beams' suffixes
  const int total = Pc + Lsum;
  // position of the query token of chunk row `row` in its [prefix ; suffix]
  auto qpos_of = [&](int row) {
    return PREFILL ? ctx + row_qi(row) : Pc + c_len[row_beam(row)] - a.T + row_qi(row);
  };
  // a left window: the prefix tiles before every row's window hold no visible key
  int k_start = 0;
  if (a.win_left >= 0) {
    int lo = INT_MAX;
    for (int row = 0; row < nrows; ++row) lo = min(lo, qpos_of(row) - a.win_left);
    k_start = min(max(0, lo), Pc) / GEN_TK * GEN_TK;
  }
  for (int k0 = k_start; k0 < total; k0 += GEN_TK) {
    __syncthreads();
    if (t < GEN_TK) {
      const int kk = k0 + t;
      int ok = 0, kb = -1, kp = kk;
      int64_t off = 0;
      if (kk < total) {
        int blk, o;
        if (kk < Pc) {
          blk = a.prefix_bt[(int64_t)r * a.prefix_bt_stride + kk / a.bs];
          o = kk % a.bs;
        } else {  // suffix slot j: beam kb holds slots c_cum[kb] .. c_cum[kb + 1] - 1
          const int j = kk - Pc;
          kb = 0;
          while (c_cum[kb + 1] <= j) ++kb;
          const int p = j - c_cum[kb], pos = c_s0[kb] + p;
          kp = Pc + p;
          blk = a.suffix_bt[(int64_t)(nb0 + b_lo + kb) * a.suffix_bt_stride + pos / a.bs];
          o = pos % a.bs;
        }
        ok = (blk >= 0 && blk < a.num_blocks);
        if (!ok) flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
        off = ok ? (int64_t)blk * a.kv_block_stride + (int64_t)o * a.kv_tok_stride : 0;
      }
      kv_ok[t] = ok;
      k_off[t] = off;
      k_beam[t] = kb;
      k_pos[t] = kp;
    }
    __syncthreads();
    // eight elements of one key row per step: one 16-byte load each for K
    // and V (two for fp32, 8 bytes for fp8) when the cache is aligned for it
    for (int e = t; e < GEN_TK * (D / 8); e += GEN_THREADS) {
      const int key = e / (D / 8), d = (e - key * (D / 8)) * 8;
      float kv[8], vv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) kv[j] = vv[j] = 0.f;
      if (kv_ok[key]) {
        const int64_t o = k_off[key] + (int64_t)hk * a.kv_head_stride + d;
        if constexpr (KV8) {
          if (vec) {
            const uint2 kb = *reinterpret_cast<const uint2*>(kc8 + o), vb = *reinterpret_cast<const uint2*>(vc8 + o);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              kv[j] = fp8e4m3_to_float(((j < 4 ? kb.x : kb.y) >> (8 * (j & 3))) & 0xFFu) * k_sc;
              vv[j] = fp8e4m3_to_float(((j < 4 ? vb.x : vb.y) >> (8 * (j & 3))) & 0xFFu) * v_sc;
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              kv[j] = fp8e4m3_to_float(kc8[o + j]) * k_sc;
              vv[j] = fp8e4m3_to_float(vc8[o + j]) * v_sc;
            }
          }
        } else {
          if (vec) {
            struct alignas(16) V16 { S e[16 / sizeof(S)]; };
            constexpr int PER = 16 / sizeof(S);  // elements per 16-byte load
#pragma unroll
            for (int h = 0; h < 8 / PER; ++h) {
              const V16 kq = *reinterpret_cast<const V16*>(kc + o + h * PER);
              const V16 vq = *reinterpret_cast<const V16*>(vc + o + h * PER);
#pragma unroll
              for (int j = 0; j < PER; ++j) {
                kv[h * PER + j] = E::to_float(kq.e[j]);
                vv[h * PER + j] = E::to_float(vq.e[j]);
              }
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              kv[j] = E::to_float(kc[o + j]);
              vv[j] = E::to_float(vc[o + j]);
            }
          }
        }
      }
      *reinterpret_cast<float4*>(k_s + key * KP + d) = float4{kv[0], kv[1], kv[2], kv[3]};
      *reinterpret_cast<float4*>(k_s + key * KP + d + 4) = float4{kv[4], kv[5], kv[6], kv[7]};
      *reinterpret_cast<float4*>(v_s + key * D + d) = float4{vv[0], vv[1], vv[2], vv[3]};
      *reinterpret_cast<float4*>(v_s + key * D + d + 4) = float4{vv[4], vv[5], vv[6], vv[7]};
    }
    __syncthreads();
    {
      // key t % TK against rows t / TK + 8 j: each K chunk read once for the
      // four rows, four dims per LDS read; every dot product sums over d in order
      const int key = t % GEN_TK;
      const int kk = k0 + key;
      const int kpos = k_pos[key], kbeam = k_beam[key];
      constexpr int RPT = GEN_ROWS / (GEN_THREADS / GEN_TK);  // rows per thread
      float sr[RPT];
#pragma unroll
      for (int j = 0; j < RPT; ++j) sr[j] = 0.f;
      for (int d = 0; d < D; d += 4) {
        const float4 k4 = *reinterpret_cast<const float4*>(k_s + key * KP + d);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
          const float4 q4 = *reinterpret_cast<const float4*>(q_s + (t / GEN_TK + j * (GEN_THREADS / GEN_TK)) * D + d);
          float s_ = sr[j];
          s_ += q4.x * k4.x;
          s_ += q4.y * k4.y;
          s_ += q4.z * k4.z;
          s_ += q4.w * k4.w;
          sr[j] = s_;
        }
      }
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int row = t / GEN_TK + j * (GEN_THREADS / GEN_TK);
        float s = sr[j] * a.scale;
        if (a.softcap > 0.f) s = a.softcap * tanhf(s / a.softcap);
        bool vis = row < nrows && kk < total && kv_ok[key];
        const int qpos = vis ? qpos_of(row) : 0;
        if (a.alibi) s -= a.alibi[hk * G + (row0 + row) % G] * (float)abs(qpos - kpos);
        if (PREFILL && a.causal) vis = vis && kpos <= qpos;
        // a suffix key: its own beam's rows only, up to the row's query (bottom-right causal)
        if (!PREFILL && vis && kbeam >= 0) vis = kbeam == row_beam(row) && kpos <= qpos;
        if (a.win_left >= 0) vis = vis && kpos >= qpos - a.win_left;
        if (a.win_right >= 0) vis = vis && kpos <= qpos + a.win_right;
        p_s[row * (GEN_TK + 1) + key] = vis ? s : -INFINITY;
      }
    }
    __syncthreads();
    if (t < GEN_ROWS) {
      float mt = -INFINITY;
      for (int key = 0; key < GEN_TK; ++key) mt = fmaxf(mt, p_s[t * (GEN_TK + 1) + key]);
      float m_old = m_s[t];
      float m_new = fmaxf(m_old, mt);
      float alpha = 1.f, lsum = 0.f;
      if (m_new != -INFINITY) {
        alpha = expf(m_old - m_new);
        for (int key = 0; key < GEN_TK; ++key) {
          float s = p_s[t * (GEN_TK + 1) + key];
          float p = (s == -INFINITY) ? 0.f : expf(s - m_new);
          p_s[t * (GEN_TK + 1) + key] = p;
          lsum += p;
        }
      } else {
        for (int key = 0; key < GEN_TK; ++key) p_s[t * (GEN_TK + 1) + key] = 0.f;
      }
      m_s[t] = m_new;
      l_s[t] = l_s[t] * alpha + lsum;
      a_s[t] = alpha;
    }
    __syncthreads();
    // slot i of a thread: four consecutive dims (one LDS read of V each key)
#pragma unroll
    for (int i = 0; i < GEN_ACC / 4; ++i) {
      const int e = (t + i * GEN_THREADS) * 4;
      if (e < GEN_ROWS * D) {
        const int row = e / D, d = e % D;
        const float al = a_s[row];
        float o0 = acc[4 * i] * al, o1 = acc[4 * i + 1] * al, o2 = acc[4 * i + 2] * al, o3 = acc[4 * i + 3] * al;
        for (int key = 0; key < GEN_TK; ++key) {
          const float p = p_s[row * (GEN_TK + 1) + key];
          const float4 v4 = *reinterpret_cast<const float4*>(v_s + key * D + d);
          o0 += p * v4.x;
          o1 += p * v4.y;
          o2 += p * v4.z;
          o3 += p * v4.w;
        }
        acc[4 * i] = o0;
        acc[4 * i + 1] = o1;
        acc[4 * i + 2] = o2;
        acc[4 * i + 3] = o3;
      }
    }
  }
  __syncthreads();
  if (a.sinks && t < GEN_ROWS) {
    // the sink joins the row's softmax: max over it too, exp(sink) in the
    // denominator; a_s carries the rescaling of the accumulated output
    const float sk = a.sinks[hk * G + (row0 + t) % G];
    const float m = m_s[t], mn = fmaxf(m, sk);
    const float al = m == -INFINITY ? 0.f : expf(m - mn);
    l_s[t] = l_s[t] * al + expf(sk - mn);
    m_s[t] = mn;
    a_s[t] = al;
  }
  __syncthreads();
  S* out = static_cast<S*>(a.out);
#pragma unroll
  for (int i = 0; i < GEN_ACC; ++i) {
    const int e = (t + (i / 4) * GEN_THREADS) * 4 + (i & 3);
    if (e < GEN_ROWS * D) {
      int row = e / D, d = e % D;
      if (row < nrows) {
        const int g = (row0 + row) % G;
        float l = l_s[row];
        float o = l > 0.f ? (a.sinks ? acc[i] * a_s[row] : acc[i]) / l : 0.f;
        out[row_tok(row) * a.out_tok_stride + (int64_t)(hk * G + g) * D + d] = E::from_float(o);
      }
    }
  }
  if (a.lse_out && t < nrows) {
    const int g = (row0 + t) % G;
    float l = l_s[t];
    a.lse_out[row_tok(t) * a.Hq + hk * G + g] = l > 0.f ? m_s[t] + logf(l) : -INFINITY;
  }
}

static size_t generic_smem_bytes(int D) {
  return sizeof(float) * ((size_t)GEN_ROWS * D + GEN_TK * (D + GEN_KPAD) + GEN_TK * D +
                          GEN_ROWS * (GEN_TK + 1) + 3 * GEN_ROWS) + sizeof(int) * GEN_TK;
}

int g_decode_kernel_override = 0;

template <bool PREFILL, bool KV8>
static gr_status_t launch_generic_kv(const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t stream) {
  static bool attr_done[3] = {};
  const void* fn = a.dtype == GR_DTYPE_F32 ? reinterpret_cast<const void*>(decode_generic<GR_DTYPE_F32, PREFILL, KV8>)
                   : a.dtype == GR_DTYPE_F16 ? reinterpret_cast<const void*>(decode_generic<GR_DTYPE_F16, PREFILL, KV8>)
                                             : reinterpret_cast<const void*>(decode_generic<GR_DTYPE_BF16, PREFILL, KV8>);
  if (!attr_done[a.dtype]) {  // head_dim 256 needs more than the default 64 KB
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)generic_smem_bytes(256));
    attr_done[a.dtype] = true;
  }
  switch (a.dtype) {
    case GR_DTYPE_F32:
      hipLaunchKernelGGL((decode_generic<GR_DTYPE_F32, PREFILL, KV8>), grid, dim3(GEN_THREADS), smem, stream, a);
      break;
    case GR_DTYPE_F16:
      hipLaunchKernelGGL((decode_generic<GR_DTYPE_F16, PREFILL, KV8>), grid, dim3(GEN_THREADS), smem, stream, a);
      break;
    default:
      hipLaunchKernelGGL((decode_generic<GR_DTYPE_BF16, PREFILL, KV8>), grid, dim3(GEN_THREADS), smem, stream, a);
      break;
  }
  return launch_status();
}

template <bool PREFILL>
static gr_status_t launch_generic(const DecodeArgs& a, hipStream_t stream) {
  const int G = a.Hq / a.Hkv;
  const int64_t chunks = ((int64_t)(PREFILL ? 1 : a.max_beams) * G * a.T + GEN_ROWS - 1) / GEN_ROWS;
  const int64_t gx = (int64_t)a.num_reqs * chunks;
  if (gx == 0) return GR_OK;
  if (gx > 0x7fffffff || a.Hkv > 65535) return GR_ERR_INVALID_ARG;
  dim3 grid((unsigned)gx, (unsigned)a.Hkv);
  const size_t smem = generic_smem_bytes(a.D);
  return a.kv8 ? launch_generic_kv<PREFILL, true>(a, grid, smem, stream)
               : launch_generic_kv<PREFILL, false>(a, grid, smem, stream);
}

}  // namespace gr

using namespace gr;

// Validates the decode arguments and fills the argument block; GR_OK means
// "launch" unless *empty is set (nothing to do).
static gr_status_t decode_args(
    DecodeArgs& a, bool& empty, void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start, const int32_t* suffix_bt, int suffix_bt_stride,
    const int32_t* suffix_len, const int32_t* suffix_start, int num_reqs, int max_beams_per_req,
    int num_beams, int q_per_beam, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status) {
  empty = false;
  if (num_beams < 0 || num_reqs < 0 || q_per_beam < 1 || num_q_heads < 1 || num_kv_heads < 1 ||
      num_q_heads % num_kv_heads != 0 || block_size < 1 || head_dim < 8 || head_dim % 8 != 0 ||
      num_blocks < 0 || prefix_bt_stride < 0 || suffix_bt_stride < 0 || max_beams_per_req < 0 ||
      !dtype_valid(dtype) || !(softcap >= 0.f))
    return GR_ERR_INVALID_ARG;
  if (head_dim > 256) return GR_ERR_UNSUPPORTED;
  if (num_beams == 0) {
    empty = true;
    return GR_OK;
  }
  if (num_reqs == 0 || !out || !q || !k_cache || !v_cache || !prefix_bt || !prefix_len ||
      !beam_start || !suffix_bt || !suffix_len)
    return GR_ERR_INVALID_ARG;
  if (q_tok_stride < (int64_t)num_q_heads * head_dim || out_tok_stride < (int64_t)num_q_heads * head_dim ||
      kv_block_stride < 1 || kv_tok_stride < 1 || kv_head_stride < 1)
    return GR_ERR_INVALID_ARG;
  a = DecodeArgs{};
  a.out = out; a.out_tok_stride = out_tok_stride;
  a.q = q; a.q_tok_stride = q_tok_stride;
  a.k_cache = k_cache; a.v_cache = v_cache; a.num_blocks = num_blocks;
  a.kv_block_stride = kv_block_stride; a.kv_tok_stride = kv_tok_stride; a.kv_head_stride = kv_head_stride;
  a.prefix_bt = prefix_bt; a.prefix_bt_stride = prefix_bt_stride; a.prefix_len = prefix_len;
  a.beam_start = beam_start;
  a.suffix_bt = suffix_bt; a.suffix_bt_stride = suffix_bt_stride; a.suffix_len = suffix_len;
  a.suffix_start = suffix_start;
  a.num_reqs = num_reqs; a.max_beams = max_beams_per_req; a.num_beams = num_beams; a.T = q_per_beam;
  a.Hq = num_q_heads; a.Hkv = num_kv_heads; a.D = head_dim; a.bs = block_size; a.dtype = dtype;
  a.scale = scale; a.softcap = softcap; a.lse_out = lse_out; a.dev_status = dev_status;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.nsplit = 1;
  a.win_left = a.win_right = -1;
  a.causal = 1;
  return GR_OK;
}

// Copies the optional features into the argument block.  Decode attention is
// causal over the beam's own tokens: a non-causal option is invalid there,
// and a right window is a no-op.
static gr_status_t apply_options(DecodeArgs& a, const gr_attn_options* opt, bool prefill) {
  if (!opt) return GR_OK;
  if (opt->window_left < -1 || opt->window_right < -1 || (opt->causal != 0 && opt->causal != 1))
    return GR_ERR_INVALID_ARG;
  if (!prefill && !opt->causal) return GR_ERR_INVALID_ARG;
  a.win_left = opt->window_left;
  a.win_right = prefill && !opt->causal ? opt->window_right : -1;
  a.causal = opt->causal;
  a.sinks = opt->sinks;
  a.alibi = opt->alibi_slopes;
  a.kv8 = opt->kv_dtype == GR_DTYPE_FP8_E4M3;
  a.k_scale = a.kv8 ? opt->k_scale : nullptr;
  a.v_scale = a.kv8 ? opt->v_scale : nullptr;
  return GR_OK;
}

#define GR_DECODE_ARG_NAMES                                                                         \
  out, out_tok_stride, q, q_tok_stride, k_cache, v_cache, num_blocks, kv_block_stride, kv_tok_stride, \
      kv_head_stride, prefix_bt, prefix_bt_stride, prefix_len, beam_start, suffix_bt, suffix_bt_stride, \
      suffix_len, suffix_start, num_reqs, max_beams_per_req, num_beams, q_per_beam, num_q_heads,       \
      num_kv_heads, head_dim, block_size, dtype, scale, softcap, lse_out, dev_status

extern "C" gr_status_t gr_beam_attn_decode(
    void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start, const int32_t* suffix_bt, int suffix_bt_stride,
    const int32_t* suffix_len, const int32_t* suffix_start, int num_reqs, int max_beams_per_req,
    int num_beams, int q_per_beam, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status,
    hipStream_t stream) {
  DecodeArgs a;
  bool empty;
  const gr_status_t st = decode_args(a, empty, GR_DECODE_ARG_NAMES);
  if (st != GR_OK || empty) return st;
  if (g_decode_kernel_override != 1) {
    if (mfma_decode_supported(a)) return launch_mfma_decode(a, stream);
    DecodeArgs p;
    if (mfma_pair_args(a, p)) return launch_mfma_decode(p, stream);
  }
  return launch_generic<false>(a, stream);
}

// Workspace layout of the split decode: partial LSEs, then partial outputs
// (256-byte aligned).
struct SplitLayout {
  size_t lse_off, o_off, total;
};
static SplitLayout split_layout(int tiles, int nsplit) {
  SplitLayout l;
  const size_t slots = (size_t)tiles * nsplit;
  l.lse_off = 0;
  l.o_off = (sizeof(float) * slots * 128 + 255) & ~(size_t)255;
  l.total = l.o_off + sizeof(uint16_t) * slots * 128 * 128;
  return l;
}

extern "C" size_t gr_beam_attn_decode_workspace_size(int num_reqs, int max_beams_per_req, int q_per_beam,
                                                     int num_q_heads, int num_kv_heads, int head_dim,
                                                     int max_prefix_len) {
  if (num_reqs <= 0 || max_beams_per_req <= 0 || q_per_beam <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0 || head_dim != 128)
    return 0;
  int tiles, nsplit;
  mfma_decode_plan(num_reqs, max_beams_per_req, q_per_beam, num_q_heads, num_kv_heads, max_prefix_len, &tiles,
                   &nsplit);
  return nsplit > 1 ? split_layout(tiles, nsplit).total : 0;
}

static gr_status_t decode_ws_impl(
    void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start, const int32_t* suffix_bt, int suffix_bt_stride,
    const int32_t* suffix_len, const int32_t* suffix_start, int num_reqs, int max_beams_per_req,
    int num_beams, int q_per_beam, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status,
    int max_prefix_len, void* workspace, size_t workspace_bytes, const gr_attn_options* opt,
    hipStream_t stream) {
  DecodeArgs a;
  bool empty;
  gr_status_t st = decode_args(a, empty, GR_DECODE_ARG_NAMES);
  if (st != GR_OK) return st;
  st = apply_options(a, opt, false);
  if (st != GR_OK || empty) return st;
  if (max_prefix_len < 0) return GR_ERR_INVALID_ARG;
  if (g_decode_kernel_override != 1 && !mfma_decode_supported(a)) {
    DecodeArgs p;  // head_dim 64 as head pairs, never split (the workspace is for head_dim 128)
    if (mfma_pair_args(a, p)) return launch_mfma_decode(p, stream);
  }
  if (g_decode_kernel_override == 1 || !mfma_decode_supported(a)) return launch_generic<false>(a, stream);
  int tiles, nsplit;
  mfma_decode_plan(num_reqs, max_beams_per_req, q_per_beam, num_q_heads, num_kv_heads, max_prefix_len, &tiles,
                   &nsplit);
  if (nsplit <= 1) return launch_mfma_decode(a, stream);
  const SplitLayout l = split_layout(tiles, nsplit);
  if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255) || workspace_bytes < l.total)
    return GR_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  a.nsplit = nsplit;
  a.ws_lse = reinterpret_cast<float*>(ws + l.lse_off);
  a.ws_o = reinterpret_cast<uint16_t*>(ws + l.o_off);
  return launch_mfma_decode_split(a, stream);
}

#define GR_DECODE_WS_NAMES GR_DECODE_ARG_NAMES, max_prefix_len, workspace, workspace_bytes

extern "C" gr_status_t gr_beam_attn_decode_ws(
    void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start, const int32_t* suffix_bt, int suffix_bt_stride,
    const int32_t* suffix_len, const int32_t* suffix_start, int num_reqs, int max_beams_per_req,
    int num_beams, int q_per_beam, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status,
    int max_prefix_len, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return decode_ws_impl(GR_DECODE_WS_NAMES, nullptr, stream);
}

extern "C" gr_status_t gr_beam_attn_decode_opt(
    void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* prefix_bt, int prefix_bt_stride, const int32_t* prefix_len,
    const int32_t* beam_start, const int32_t* suffix_bt, int suffix_bt_stride,
    const int32_t* suffix_len, const int32_t* suffix_start, int num_reqs, int max_beams_per_req,
    int num_beams, int q_per_beam, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status,
    int max_prefix_len, void* workspace, size_t workspace_bytes, const gr_attn_options* options,
    hipStream_t stream) {
  return decode_ws_impl(GR_DECODE_WS_NAMES, options, stream);
}

static gr_status_t prefill_impl(
    void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* block_table, int bt_stride, const int32_t* query_start, const int32_t* seq_len,
    int num_reqs, int num_tokens, int max_query_len, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status,
    const gr_attn_options* opt, hipStream_t stream) {
  if (num_reqs < 0 || num_tokens < 0 || max_query_len < 0 || num_q_heads < 1 || num_kv_heads < 1 ||
      num_q_heads % num_kv_heads != 0 || block_size < 1 || head_dim < 8 || head_dim % 8 != 0 ||
      num_blocks < 0 || bt_stride < 0 || !dtype_valid(dtype) || !(softcap >= 0.f))
    return GR_ERR_INVALID_ARG;
  if (head_dim > 256) return GR_ERR_UNSUPPORTED;
  if (num_reqs == 0 || num_tokens == 0 || max_query_len == 0) return GR_OK;
  if (!out || !q || !k_cache || !v_cache || !block_table || !query_start || !seq_len)
    return GR_ERR_INVALID_ARG;
  if (q_tok_stride < (int64_t)num_q_heads * head_dim || out_tok_stride < (int64_t)num_q_heads * head_dim ||
      kv_block_stride < 1 || kv_tok_stride < 1 || kv_head_stride < 1)
    return GR_ERR_INVALID_ARG;
  DecodeArgs a = {};
  a.out = out; a.out_tok_stride = out_tok_stride;
  a.q = q; a.q_tok_stride = q_tok_stride;
  a.k_cache = k_cache; a.v_cache = v_cache; a.num_blocks = num_blocks;
  a.kv_block_stride = kv_block_stride; a.kv_tok_stride = kv_tok_stride; a.kv_head_stride = kv_head_stride;
  a.prefix_bt = block_table; a.prefix_bt_stride = bt_stride; a.prefix_len = seq_len;
  a.beam_start = query_start;
  a.suffix_bt = nullptr; a.suffix_bt_stride = 0; a.suffix_len = nullptr; a.suffix_start = nullptr;
  a.num_reqs = num_reqs; a.max_beams = 1; a.num_beams = num_tokens; a.T = max_query_len;
  a.Hq = num_q_heads; a.Hkv = num_kv_heads; a.D = head_dim; a.bs = block_size; a.dtype = dtype;
  a.scale = scale; a.softcap = softcap; a.lse_out = lse_out; a.dev_status = dev_status;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.win_left = a.win_right = -1;
  a.causal = 1;
  const gr_status_t st = apply_options(a, opt, true);
  if (st != GR_OK) return st;
  if (g_decode_kernel_override != 1) {
    if (mfma_prefill_supported(a)) return launch_mfma_prefill(a, stream);
    DecodeArgs p;
    if (mfma_pair_args(a, p) && mfma_prefill_supported(p)) return launch_mfma_prefill(p, stream);
  }
  return launch_generic<true>(a, stream);
}

#define GR_PREFILL_ARG_NAMES                                                                             \
  out, out_tok_stride, q, q_tok_stride, k_cache, v_cache, num_blocks, kv_block_stride, kv_tok_stride,     \
      kv_head_stride, block_table, bt_stride, query_start, seq_len, num_reqs, num_tokens, max_query_len, \
      num_q_heads, num_kv_heads, head_dim, block_size, dtype, scale, softcap, lse_out, dev_status

extern "C" gr_status_t gr_paged_attn_prefill(
    void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* block_table, int bt_stride, const int32_t* query_start, const int32_t* seq_len,
    int num_reqs, int num_tokens, int max_query_len, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status,
    hipStream_t stream) {
  return prefill_impl(GR_PREFILL_ARG_NAMES, nullptr, stream);
}

extern "C" gr_status_t gr_paged_attn_prefill_opt(
    void* out, int64_t out_tok_stride, const void* q, int64_t q_tok_stride,
    const void* k_cache, const void* v_cache, int64_t num_blocks,
    int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
    const int32_t* block_table, int bt_stride, const int32_t* query_start, const int32_t* seq_len,
    int num_reqs, int num_tokens, int max_query_len, int num_q_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, float softcap, float* lse_out, int32_t* dev_status,
    const gr_attn_options* options, hipStream_t stream) {
  return prefill_impl(GR_PREFILL_ARG_NAMES, options, stream);
}



extern "C" int gr_set_decode_kernel(int which) {
  if (which < 0 || which > 1) return GR_ERR_INVALID_ARG;
  g_decode_kernel_override = which;
  return GR_OK;
}
