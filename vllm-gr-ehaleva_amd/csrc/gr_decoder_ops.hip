// Fused elementwise stages of the Qwen-style decoder that drives the beam
// path end to end: residual add + RMSNorm, per-head q/k RMSNorm + rotary
// embedding + K/V cache write, and the SiLU-gated product of the MLP.  They
// take the roles of vLLM's fused_add_rms_norm, rotary_embedding +
// reshape_and_cache_flash and silu_and_mul kernels (vllm==0.14, not vendored)
// in the model the reference serves.  All arithmetic is float32; each output
// element is rounded to the storage type once.
#include "gr_common.h"
#include "gr_decoder.h"

namespace gr {
namespace {

constexpr int EW_THREADS = 256;

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---- residual add + RMSNorm: one workgroup per token row -------------------
struct RmsArgs {
  void* out;
  int64_t out_stride;
  const void* x;
  int64_t x_stride;
  void* residual;  // nullable
  int64_t res_stride;
  const void* weight;
  int hidden;
  float eps;
};

// V elements per access: 16-byte vectors when every row start is aligned,
// single elements otherwise.
template <int DT, int V>
__global__ __launch_bounds__(EW_THREADS) void rms_norm_k(RmsArgs a) {
  using E = Elem<DT>;
  using S = typename E::storage;
  struct alignas(sizeof(S) * V) Vec { S e[V]; };
  const int64_t t = blockIdx.x;
  const S* x = static_cast<const S*>(a.x) + t * a.x_stride;
  S* res = a.residual ? static_cast<S*>(a.residual) + t * a.res_stride : nullptr;
  S* out = static_cast<S*>(a.out) + t * a.out_stride;
  const S* w = static_cast<const S*>(a.weight);
  const int H = a.hidden;
  float ss = 0.f;
  // pass 1: y = x (+ residual), rounded to the storage type; residual <- y
  for (int i = threadIdx.x * V; i < H; i += EW_THREADS * V) {
    Vec xv = *reinterpret_cast<const Vec*>(x + i);
    if (res) {
      Vec rv = *reinterpret_cast<const Vec*>(res + i);
#pragma unroll
      for (int j = 0; j < V; ++j) xv.e[j] = E::from_float(E::to_float(xv.e[j]) + E::to_float(rv.e[j]));
      *reinterpret_cast<Vec*>(res + i) = xv;
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float y = E::to_float(xv.e[j]);
      ss += y * y;
    }
  }
  __shared__ float part[EW_THREADS / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < EW_THREADS / 64; ++i) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / (float)H + a.eps);
  // pass 2: out = y * inv * w (this thread's own y, re-read)
  const S* ysrc = res ? res : x;
  for (int i = threadIdx.x * V; i < H; i += EW_THREADS * V) {
    const Vec yv = *reinterpret_cast<const Vec*>(ysrc + i);
    const Vec wv = *reinterpret_cast<const Vec*>(w + i);
    Vec ov;
#pragma unroll
    for (int j = 0; j < V; ++j) ov.e[j] = E::from_float(E::to_float(yv.e[j]) * inv * E::to_float(wv.e[j]));
    *reinterpret_cast<Vec*>(out + i) = ov;
  }
}

// ---- q/k RMSNorm + rotary + cache write: one workgroup per token -----------
struct RopeArgs {
  void* q_out;
  int64_t q_out_stride;
  const void* qkv;
  int64_t qkv_stride;
  const int64_t* positions;
  const float* cos_t;  // [table_len, D/2]
  const float* sin_t;
  int64_t table_len;
  const void* q_norm;  // [D], nullable
  const void* k_norm;
  void* k_cache;
  void* v_cache;
  int64_t num_blocks, kv_block_stride, kv_tok_stride, kv_head_stride;
  const int64_t* slot_mapping;  // nullable: no cache write
  int bs, Hq, Hkv, D;
  float eps;
  int32_t* dev_status;
};

// Register form of rms_norm_k for rows of at most 4 * EW_THREADS * V
// elements: each thread keeps its NV vectors of y (and of the weight) in
// registers from the first read, so the second pass re-reads nothing.  The
// same roundings as rms_norm_k, so the same results bit for bit.
template <int DT, int V, int NV>
__global__ __launch_bounds__(EW_THREADS) void rms_norm_reg_k(RmsArgs a) {
  using E = Elem<DT>;
  using S = typename E::storage;
  struct alignas(sizeof(S) * V) Vec { S e[V]; };
  const int64_t t = blockIdx.x;
  const S* x = static_cast<const S*>(a.x) + t * a.x_stride;
  S* res = a.residual ? static_cast<S*>(a.residual) + t * a.res_stride : nullptr;
  S* out = static_cast<S*>(a.out) + t * a.out_stride;
  const S* w = static_cast<const S*>(a.weight);
  const int H = a.hidden;
  Vec yv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = (threadIdx.x + k * EW_THREADS) * V;
    if (i < H) {
      yv[k] = *reinterpret_cast<const Vec*>(x + i);
      if (res) rv[k] = *reinterpret_cast<const Vec*>(res + i);
      wv[k] = *reinterpret_cast<const Vec*>(w + i);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = (threadIdx.x + k * EW_THREADS) * V;
    if (i < H) {
      if (res) {
#pragma unroll
        for (int j = 0; j < V; ++j) yv[k].e[j] = E::from_float(E::to_float(yv[k].e[j]) + E::to_float(rv[k].e[j]));
        *reinterpret_cast<Vec*>(res + i) = yv[k];
      }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float y = E::to_float(yv[k].e[j]);
        ss += y * y;
      }
    }
  }
  __shared__ float part[EW_THREADS / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < EW_THREADS / 64; ++i) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / (float)H + a.eps);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = (threadIdx.x + k * EW_THREADS) * V;
    if (i < H) {
      Vec ov;
#pragma unroll
      for (int j = 0; j < V; ++j) ov.e[j] = E::from_float(E::to_float(yv[k].e[j]) * inv * E::to_float(wv[k].e[j]));
      *reinterpret_cast<Vec*>(out + i) = ov;
    }
  }
}

// One wave per head: workgroup g covers heads 4*(g % hgroups) .. +3 of token
// g / hgroups, over the token's Hq query, Hkv key and Hkv value heads (in
// that order); lane l holds the rotary pairs (i, i + D/2), i = l, l + 64.
template <int DT>
__global__ __launch_bounds__(EW_THREADS) void qk_norm_rope_k(RopeArgs a, int hgroups) {
  using E = Elem<DT>;
  using S = typename E::storage;
  const int64_t t = blockIdx.x / hgroups;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = (blockIdx.x % hgroups) * (EW_THREADS / 64) + wave;
  const int nheads = a.Hq + 2 * a.Hkv;
  if (h >= nheads) return;
  const int D = a.D, half = D >> 1;
  const int64_t pos = a.positions[t];
  if (pos < 0 || pos >= a.table_len) {
    if (h == 0 && lane == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
    return;
  }
  int64_t kv_off = -1;  // element offset of this token's slot in the cache
  if (a.slot_mapping) {
    const int64_t slot = a.slot_mapping[t];
    if (slot >= 0) {
      const int64_t blk = slot / a.bs;
      if (blk < a.num_blocks) {
        kv_off = blk * a.kv_block_stride + (slot % a.bs) * a.kv_tok_stride;
      } else if (h == 0 && lane == 0) {
        flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
      }
    }
  }
  const S* src = static_cast<const S*>(a.qkv) + t * a.qkv_stride;
  const float* ct = a.cos_t + pos * half;
  const float* st = a.sin_t + pos * half;
  {
    const S* hp = src + (int64_t)h * D;
    if (h >= a.Hq + a.Hkv) {  // value head: copy into the cache
      if (kv_off >= 0) {
        S* dst = static_cast<S*>(a.v_cache) + kv_off + (int64_t)(h - a.Hq - a.Hkv) * a.kv_head_stride;
        for (int i = lane; i < D; i += 64) dst[i] = hp[i];
      }
      return;
    }
    const bool is_q = h < a.Hq;
    const S* nw = static_cast<const S*>(is_q ? a.q_norm : a.k_norm);
    float x1[2], x2[2];  // pairs i = lane, lane + 64 (D <= 256)
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = lane + 64 * k;
      x1[k] = i < half ? E::to_float(hp[i]) : 0.f;
      x2[k] = i < half ? E::to_float(hp[i + half]) : 0.f;
      ss += x1[k] * x1[k] + x2[k] * x2[k];
    }
    float inv = 1.f;
    if (nw) inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
    S* dst;
    if (is_q) {
      dst = static_cast<S*>(a.q_out) + t * a.q_out_stride + (int64_t)h * D;
    } else {
      if (kv_off < 0) return;
      dst = static_cast<S*>(a.k_cache) + kv_off + (int64_t)(h - a.Hq) * a.kv_head_stride;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = lane + 64 * k;
      if (i < half) {
        float y1 = x1[k] * inv, y2 = x2[k] * inv;
        if (nw) {
          y1 *= E::to_float(nw[i]);
          y2 *= E::to_float(nw[i + half]);
        }
        const float c = ct[i], s = st[i];
        dst[i] = E::from_float(y1 * c - y2 * s);
        dst[i + half] = E::from_float(y2 * c + y1 * s);
      }
    }
  }
}

// Vector form: every lane moves 16 bytes (EPL elements), a head spans
// L = D / EPL lanes (a power of two, 2 .. 64), a wave covers 64 / L heads and
// a workgroup 4 times that.  Lane j of a head holds elements
// [EPL*j, EPL*j + EPL); the rotary partner of its elements is lane j ^ L/2.
// A workgroup takes NT consecutive tokens and issues all their row, position
// and slot loads before it computes any (one 16-byte load in flight per lane
// leaves the chip's memory latency exposed on long prompts).
template <typename S>
struct alignas(16) Vec16 {
  S e[16 / sizeof(S)];
};

template <int DT, int NT>
__global__ __launch_bounds__(EW_THREADS) void qk_norm_rope_vec_k(RopeArgs a, int hgroups, int L, int num_tokens) {
  using E = Elem<DT>;
  using S = typename E::storage;
  using Vec = Vec16<S>;
  constexpr int EPL = 16 / sizeof(S);
  const int64_t t0 = (int64_t)(blockIdx.x / hgroups) * NT;
  const int lane = threadIdx.x & 63;
  const int hpw = 64 / L;  // heads per wave
  const int h = ((blockIdx.x % hgroups) * (EW_THREADS / 64) + (threadIdx.x >> 6)) * hpw + lane / L;
  const int j = lane % L;  // lane within the head
  const int nheads = a.Hq + 2 * a.Hkv;
  const int D = a.D, half = D >> 1;
  const bool valid = h < nheads;
  const int hc = valid ? h : 0;  // clamped: every lane joins the shuffles
  const bool is_v = hc >= a.Hq + a.Hkv, is_q = hc < a.Hq;
  Vec xv[NT];
  int64_t pos[NT], slot[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    const int64_t t = min(t0 + u, (int64_t)num_tokens - 1);  // clamped: loads stay in bounds
    xv[u] = *reinterpret_cast<const Vec*>(static_cast<const S*>(a.qkv) + t * a.qkv_stride + (int64_t)hc * D +
                                          j * EPL);
    pos[u] = a.positions[t];
    slot[u] = a.slot_mapping ? a.slot_mapping[t] : -1;
  }
  const S* nw = static_cast<const S*>(is_q ? a.q_norm : a.k_norm);
  const bool second = j >= (L >> 1);    // this lane holds the second half of its pairs
  const int i0 = (j % (L >> 1)) * EPL;  // pair index of element 0
  const int pj = j ^ (L >> 1);
  Vec wv{}, pw{};
  if (nw && valid && !is_v) {
    wv = *reinterpret_cast<const Vec*>(nw + j * EPL);
    pw = *reinterpret_cast<const Vec*>(nw + pj * EPL);
  }
  // one token; every branch before the shuffles is uniform over the workgroup
  auto one = [&](int64_t t, const Vec& x_v, int64_t p_t, int64_t s_t) {
    if (p_t < 0 || p_t >= a.table_len) {
      if (h == 0 && j == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
      return;
    }
    int64_t kv_off = -1;
    if (s_t >= 0) {
      const int64_t blk = s_t / a.bs;
      if (blk < a.num_blocks) {
        kv_off = blk * a.kv_block_stride + (s_t % a.bs) * a.kv_tok_stride;
      } else if (h == 0 && j == 0) {
        flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
      }
    }
    float x[EPL], p[EPL];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      x[e] = E::to_float(x_v.e[e]);
      ss += x[e] * x[e];
    }
    // partner elements (lane j ^ L/2) and the head's sum of squares
#pragma unroll
    for (int e = 0; e < EPL; ++e) p[e] = __shfl_xor(x[e], L >> 1, 64);
    for (int off = 1; off < L; off <<= 1) ss += __shfl_xor(ss, off, 64);
    if (!valid) return;
    if (is_v) {
      if (kv_off >= 0)
        *reinterpret_cast<Vec*>(static_cast<S*>(a.v_cache) + kv_off +
                                (int64_t)(hc - a.Hq - a.Hkv) * a.kv_head_stride + j * EPL) = x_v;
      return;
    }
    S* dst;
    if (is_q) {
      dst = static_cast<S*>(a.q_out) + t * a.q_out_stride + (int64_t)hc * D;
    } else {
      if (kv_off < 0) return;
      dst = static_cast<S*>(a.k_cache) + kv_off + (int64_t)(hc - a.Hq) * a.kv_head_stride;
    }
    const float inv = nw ? 1.0f / sqrtf(ss / (float)D + a.eps) : 1.f;
    const float* ct = a.cos_t + p_t * half + i0;
    const float* st = a.sin_t + p_t * half + i0;
    Vec ov;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float y = x[e] * inv, q = p[e] * inv;
      if (nw) {
        y *= E::to_float(wv.e[e]);
        q *= E::to_float(pw.e[e]);
      }
      const float c = ct[e], sn = st[e];
      ov.e[e] = E::from_float(second ? y * c + q * sn : y * c - q * sn);
    }
    *reinterpret_cast<Vec*>(dst + j * EPL) = ov;
  };
#pragma unroll
  for (int u = 0; u < NT; ++u)
    if (t0 + u < num_tokens) one(t0 + u, xv[u], pos[u], slot[u]);
}

// ---- SiLU-gated product: out[t, i] = silu(x[t, i]) * x[t, F + i] -----------
template <int DT, int V>
__global__ __launch_bounds__(EW_THREADS) void silu_mul_k(void* out, int64_t out_stride, const void* x,
                                                         int64_t x_stride, int F) {
  using E = Elem<DT>;
  using S = typename E::storage;
  struct alignas(sizeof(S) * V) Vec { S e[V]; };
  const int64_t t = blockIdx.y;
  const int i = (blockIdx.x * EW_THREADS + threadIdx.x) * V;
  if (i >= F) return;
  const S* xr = static_cast<const S*>(x) + t * x_stride;
  const Vec g = *reinterpret_cast<const Vec*>(xr + i);
  const Vec u = *reinterpret_cast<const Vec*>(xr + F + i);
  Vec o;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float gv = E::to_float(g.e[j]);
    const float sg = gv / (1.0f + __expf(-gv));
    o.e[j] = E::from_float(sg * E::to_float(u.e[j]));
  }
  *reinterpret_cast<Vec*>(static_cast<S*>(out) + t * out_stride + i) = o;
}

// rms_norm launch: the register form when a row fits 4 vectors per thread
template <int DT, int V>
void launch_rms(dim3 grid, hipStream_t stream, const RmsArgs& a, bool vec) {
  const int nv = vec ? (a.hidden + EW_THREADS * V - 1) / (EW_THREADS * V) : 0;
  if (nv == 1) hipLaunchKernelGGL((rms_norm_reg_k<DT, V, 1>), grid, dim3(EW_THREADS), 0, stream, a);
  else if (nv == 2) hipLaunchKernelGGL((rms_norm_reg_k<DT, V, 2>), grid, dim3(EW_THREADS), 0, stream, a);
  else if (nv == 3 || nv == 4) hipLaunchKernelGGL((rms_norm_reg_k<DT, V, 4>), grid, dim3(EW_THREADS), 0, stream, a);
  else if (vec) hipLaunchKernelGGL((rms_norm_k<DT, V>), grid, dim3(EW_THREADS), 0, stream, a);
  else hipLaunchKernelGGL((rms_norm_k<DT, 1>), grid, dim3(EW_THREADS), 0, stream, a);
}

template <int DT>
void launch_rope_vec(dim3 grid, hipStream_t stream, const RopeArgs& a, int hg, int L, int num_tokens, int nt) {
  if (nt == 4)
    hipLaunchKernelGGL((qk_norm_rope_vec_k<DT, 4>), grid, dim3(EW_THREADS), 0, stream, a, hg, L, num_tokens);
  else
    hipLaunchKernelGGL((qk_norm_rope_vec_k<DT, 1>), grid, dim3(EW_THREADS), 0, stream, a, hg, L, num_tokens);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace gr

using namespace gr;

extern "C" gr_status_t gr_rms_norm(void* out, int64_t out_stride, const void* x, int64_t x_stride,
                                   void* residual, int64_t res_stride, const void* weight, int num_tokens,
                                   int hidden, float eps, int dtype, hipStream_t stream) {
  if (num_tokens < 0 || hidden < 1 || !dtype_valid(dtype) || !(eps >= 0.f)) return GR_ERR_INVALID_ARG;
  if (num_tokens == 0) return GR_OK;
  if (!out || !x || !weight || out_stride < hidden || x_stride < hidden || (residual && res_stride < hidden))
    return GR_ERR_INVALID_ARG;
  RmsArgs a{out, out_stride, x, x_stride, residual, res_stride, weight, hidden, eps};
  const int es = dtype_size(dtype), V = 16 / es;
  const bool vec = hidden % V == 0 && aligned16(out) && aligned16(x) && aligned16(weight) &&
                   (!residual || aligned16(residual)) && (out_stride * es) % 16 == 0 &&
                   (x_stride * es) % 16 == 0 && (!residual || (res_stride * es) % 16 == 0);
  dim3 grid((unsigned)num_tokens);
  switch (dtype) {
    case GR_DTYPE_F32: launch_rms<GR_DTYPE_F32, 4>(grid, stream, a, vec); break;
    case GR_DTYPE_F16: launch_rms<GR_DTYPE_F16, 8>(grid, stream, a, vec); break;
    default: launch_rms<GR_DTYPE_BF16, 8>(grid, stream, a, vec); break;
  }
  return launch_status();
}

extern "C" gr_status_t gr_qk_norm_rope_cache(
    void* q_out, int64_t q_out_stride, const void* qkv, int64_t qkv_stride, const int64_t* positions,
    const float* cos_table, const float* sin_table, int64_t table_len, const void* q_norm_weight,
    const void* k_norm_weight, void* k_cache, void* v_cache, int64_t num_blocks, int64_t kv_block_stride,
    int64_t kv_tok_stride, int64_t kv_head_stride, const int64_t* slot_mapping, int block_size, int num_tokens,
    int num_q_heads, int num_kv_heads, int head_dim, float eps, int dtype, int32_t* dev_status,
    hipStream_t stream) {
  if (num_tokens < 0 || num_q_heads < 1 || num_kv_heads < 0 || head_dim < 2 || head_dim % 2 != 0 ||
      head_dim > 256 || !dtype_valid(dtype) || !(eps >= 0.f) || table_len < 0 || block_size < 1 ||
      num_blocks < 0)
    return GR_ERR_INVALID_ARG;
  if (num_tokens == 0) return GR_OK;
  if (!q_out || !qkv || !positions || !cos_table || !sin_table) return GR_ERR_INVALID_ARG;
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr)) return GR_ERR_INVALID_ARG;
  if (slot_mapping && (!k_cache || !v_cache || kv_block_stride < 1 || kv_tok_stride < 1 || kv_head_stride < 1))
    return GR_ERR_INVALID_ARG;
  if (q_out_stride < (int64_t)num_q_heads * head_dim ||
      qkv_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim)
    return GR_ERR_INVALID_ARG;
  RopeArgs a{q_out, q_out_stride, qkv, qkv_stride, positions, cos_table, sin_table, table_len,
             q_norm_weight, k_norm_weight, k_cache, v_cache, num_blocks, kv_block_stride, kv_tok_stride,
             kv_head_stride, slot_mapping, block_size, num_q_heads, num_kv_heads, head_dim, eps, dev_status};
  const int nheads = num_q_heads + 2 * num_kv_heads;
  // vector form: 16-byte rows, a power-of-two lane count per head
  const int es = dtype_size(dtype), L = head_dim * es / 16;
  const bool vec = (head_dim * es) % 16 == 0 && L >= 2 && L <= 64 && (L & (L - 1)) == 0 && aligned16(q_out) &&
                   aligned16(qkv) && (q_out_stride * es) % 16 == 0 && (qkv_stride * es) % 16 == 0 &&
                   (!q_norm_weight || (aligned16(q_norm_weight) && aligned16(k_norm_weight))) &&
                   (!slot_mapping || (aligned16(k_cache) && aligned16(v_cache) && (kv_block_stride * es) % 16 == 0 &&
                                      (kv_tok_stride * es) % 16 == 0 && (kv_head_stride * es) % 16 == 0));
  if (vec) {
    const int per_wg = (EW_THREADS / 64) * (64 / L);
    const int hg = (nheads + per_wg - 1) / per_wg;
    // four tokens per workgroup once there are enough tokens to fill the chip
    const int nt = num_tokens >= 1024 ? 4 : 1;
    const int64_t nwg = (int64_t)((num_tokens + nt - 1) / nt) * hg;
    if (nwg > 0x7fffffff) return GR_ERR_INVALID_ARG;
    dim3 grid((unsigned)nwg);
    switch (dtype) {
      case GR_DTYPE_F32: launch_rope_vec<GR_DTYPE_F32>(grid, stream, a, hg, L, num_tokens, nt); break;
      case GR_DTYPE_F16: launch_rope_vec<GR_DTYPE_F16>(grid, stream, a, hg, L, num_tokens, nt); break;
      default: launch_rope_vec<GR_DTYPE_BF16>(grid, stream, a, hg, L, num_tokens, nt); break;
    }
    return launch_status();
  }
  const int hgroups = (nheads + EW_THREADS / 64 - 1) / (EW_THREADS / 64);
  const int64_t nwg = (int64_t)num_tokens * hgroups;
  if (nwg > 0x7fffffff) return GR_ERR_INVALID_ARG;
  dim3 grid((unsigned)nwg);
  switch (dtype) {
    case GR_DTYPE_F32: hipLaunchKernelGGL(qk_norm_rope_k<GR_DTYPE_F32>, grid, dim3(EW_THREADS), 0, stream, a, hgroups); break;
    case GR_DTYPE_F16: hipLaunchKernelGGL(qk_norm_rope_k<GR_DTYPE_F16>, grid, dim3(EW_THREADS), 0, stream, a, hgroups); break;
    default: hipLaunchKernelGGL(qk_norm_rope_k<GR_DTYPE_BF16>, grid, dim3(EW_THREADS), 0, stream, a, hgroups); break;
  }
  return launch_status();
}

extern "C" gr_status_t gr_silu_mul(void* out, int64_t out_stride, const void* x, int64_t x_stride,
                                   int num_tokens, int ffn, int dtype, hipStream_t stream) {
  if (num_tokens < 0 || ffn < 1 || !dtype_valid(dtype)) return GR_ERR_INVALID_ARG;
  if (num_tokens == 0) return GR_OK;
  if (!out || !x || out_stride < ffn || x_stride < 2 * (int64_t)ffn || num_tokens > 65535)
    return GR_ERR_INVALID_ARG;
  const int es = dtype_size(dtype), V16 = 16 / es;
  const bool vec = ffn % V16 == 0 && aligned16(out) && aligned16(x) && (out_stride * es) % 16 == 0 &&
                   (x_stride * es) % 16 == 0;
  const int V = vec ? V16 : 1;
  dim3 grid((unsigned)((ffn / V + EW_THREADS - 1) / EW_THREADS), (unsigned)num_tokens);
  switch (dtype) {
    case GR_DTYPE_F32:
      if (vec) hipLaunchKernelGGL((silu_mul_k<GR_DTYPE_F32, 4>), grid, dim3(EW_THREADS), 0, stream, out, out_stride, x, x_stride, ffn);
      else hipLaunchKernelGGL((silu_mul_k<GR_DTYPE_F32, 1>), grid, dim3(EW_THREADS), 0, stream, out, out_stride, x, x_stride, ffn);
      break;
    case GR_DTYPE_F16:
      if (vec) hipLaunchKernelGGL((silu_mul_k<GR_DTYPE_F16, 8>), grid, dim3(EW_THREADS), 0, stream, out, out_stride, x, x_stride, ffn);
      else hipLaunchKernelGGL((silu_mul_k<GR_DTYPE_F16, 1>), grid, dim3(EW_THREADS), 0, stream, out, out_stride, x, x_stride, ffn);
      break;
    default:
      if (vec) hipLaunchKernelGGL((silu_mul_k<GR_DTYPE_BF16, 8>), grid, dim3(EW_THREADS), 0, stream, out, out_stride, x, x_stride, ffn);
      else hipLaunchKernelGGL((silu_mul_k<GR_DTYPE_BF16, 1>), grid, dim3(EW_THREADS), 0, stream, out, out_stride, x, x_stride, ffn);
      break;
  }
  return launch_status();
}
