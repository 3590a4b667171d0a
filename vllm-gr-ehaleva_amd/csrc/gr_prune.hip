// Fused beam pruning for gfx950: log_softmax + cumulative logprob + top-k
// over beams x vocab (the sampler's logprobs=W top-K plus the host pruning of
// vllm_gr/entrypoints/openai/serving_engine.py:457-592, as two launches).
//
// Kernel 1 (prune_rows): one workgroup of 256 threads per beam row.  Reads
// the row once (float4, rows up to 8192 held in registers), computes the row
// max, the fixed-order fp32 exp-sum, the float64 LSE, and the row's top-k by
// (logit desc, token asc): a three-pass radix select (11/11/10-bit digits,
// LDS histograms) over the order-preserving integer image of the logits finds
// the k-th largest key T exactly; keys above T are taken, then keys equal to
// T in ascending token order; the k selected are ranked by counting.
// Kernel 2 (prune_merge): one workgroup of 1024 threads per request.  A
// six-pass radix select over the order-preserving 64-bit image of the float64
// scores finds the k-th largest score exactly; candidates above it are taken,
// then exact ties in ascending flat index (rows in beam order, equal scores
// of one row in token order); the k selected are ranked by counting.
//
// This file is compiled with -ffp-contract=off: every float operation below
// is a single IEEE operation so the CPU restatement reproduces the scores
// bit for bit.
#include "gr_common.h"

#include <mutex>
#include <type_traits>

namespace gr {
namespace {

constexpr int PR_THREADS = 256;
constexpr int PR_VEC = 4;
constexpr int PR_CHUNK = PR_THREADS * PR_VEC;  // elements per chunk
constexpr int PR_REG_CHUNKS = 8;               // rows of up to 8192 stay in registers
constexpr int PR_MAXK = 1024;
constexpr int PR_MAXW = 1024;
constexpr int PR_BINS = 2048;                  // radix-select histogram bins (11-bit digits)
constexpr int PR_SURV = 512;                   // row survivors ranked directly (at most)
constexpr int MG_THREADS = 1024;               // merge workgroup

typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));

// ---- bit-exact numerics ------------------------------------------------------
// exp2 of t <= 0: t is first raised to -126 (-inf and NaN included), so
// k = rint(t) >= -126 and the result is a normal float (2^-126 at the floor,
// invisible in a row sum >= 1); then a degree-5 polynomial (Horner with fma; the
// Remez minimax of the relative error of 2^f on [-1/2, 1/2] with p(0) = 1,
// rounded to float32, c3 and c5 then nudged: within 2.02 ulp) on the fractional
// part f = t - k, scaled by 2^k.
__device__ inline float exp2_neg(float t) {
  t = fmaxf(t, -126.0f);
  const float k = __builtin_rintf(t);
  const float f = t - k;
  float p = 0x1.5bbea6p-10f;
  p = __builtin_fmaf(p, f, 0x1.3cea88p-7f);
  p = __builtin_fmaf(p, f, 0x1.c6b746p-5f);
  p = __builtin_fmaf(p, f, 0x1.ebf9bcp-3f);
  p = __builtin_fmaf(p, f, 0x1.62e42ap-1f);
  p = __builtin_fmaf(p, f, 0x1.000000p+0f);
  return __builtin_amdgcn_ldexpf(p, (int)k);
}

// natural log of s >= 1 in float64: s = mant * 2^e, mant in [sqrt(1/2), sqrt(2)),
// log(mant) = 2 atanh(z), z = (mant-1)/(mant+1), series to z^23.
__device__ inline double log_f64(double s) {
  double mant = __builtin_amdgcn_frexp_mant(s);
  int e = __builtin_amdgcn_frexp_exp(s);
  if (mant < 0x1.6a09e667f3bcdp-1) {
    mant = mant * 2.0;
    e -= 1;
  }
  const double z = (mant - 1.0) / (mant + 1.0);
  const double w = z * z;
  double q = 1.0 / 23.0;
  q = __builtin_fma(q, w, 1.0 / 21.0);
  q = __builtin_fma(q, w, 1.0 / 19.0);
  q = __builtin_fma(q, w, 1.0 / 17.0);
  q = __builtin_fma(q, w, 1.0 / 15.0);
  q = __builtin_fma(q, w, 1.0 / 13.0);
  q = __builtin_fma(q, w, 1.0 / 11.0);
  q = __builtin_fma(q, w, 1.0 / 9.0);
  q = __builtin_fma(q, w, 1.0 / 7.0);
  q = __builtin_fma(q, w, 1.0 / 5.0);
  q = __builtin_fma(q, w, 1.0 / 3.0);
  q = __builtin_fma(q, w, 1.0);
  const double de = (double)e;
  return de * 0x1.62e42p-1 + (de * 0x1.fdf473de6af28p-22 + (z + z) * q);
}

// order-preserving integer images (larger value -> larger key)
__device__ inline uint32_t fkey(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float fval(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// row order (logit desc, token asc) as one unsigned key: larger key first
__device__ inline uint64_t row_key(uint32_t fk, int token) {
  return ((uint64_t)fk << 32) | (uint32_t)~(uint32_t)token;
}
__device__ inline uint64_t dkey(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  return (u >> 63) ? ~u : (u | (1ull << 63));
}
__device__ inline double dval(uint64_t k) {
  return __builtin_bit_cast(double, (k >> 63) ? (k & ~(1ull << 63)) : ~k);
}

struct PruneArgs {
  const float* logits;
  int64_t row_stride;
  const float* cum;
  const double* cum64;  // float64 cumulative scores (gr_beam_prune_topk_f64); overrides cum
  int R, W, V, k1, k, eos;
  float* cand_x;    // [R*W, k1] row top-k logits, sorted; EOS removed, tail padded
  int32_t* cand_v;  // [R*W, k1] tokens (-1 = empty)
  double* row_c;    // [R*W]     cum - lse
  int32_t* parent;
  int32_t* token;
  float* score;
  float* eos_score;
  double* score64;      // float64 outputs (gr_beam_prune_topk_f64); override score / eos_score
  double* eos_score64;
  int32_t* cand_token;   // nullable [R*W, k1]: each row's top-k1 tokens before EOS / catalog removal
  float* cand_logprob;   // nullable [R*W, k1]: their logprobs x - lse
  uint64_t* part_key;  // [R, ng, k] stage-1 selections: score key (0 = empty) ...
  int64_t* part_flat;  // ... and flat index b * V + v
  int ng, gr;          // row groups per request, rows per group
  // catalog (nullable): the trie in CSR form -- node n's children are
  // child_token / child_node[node_start[n] .. node_start[n+1]), tokens
  // ascending; beam_node[b] is beam b's node (-1: no valid continuation)
  const int32_t* beam_node;
  const int32_t* node_start;
  const int32_t* child_token;
  const int32_t* child_node;
  int num_nodes, num_edges;
  int32_t* dev_status;
};

// Output slot o of the selection: the float64 score, or its float32 rounding.
__device__ inline void put_score(const PruneArgs& a, int64_t o, double v) {
  if (a.score64) a.score64[o] = v;
  else a.score[o] = (float)v;
}

// Position of token t among the children [c0, c1) of a trie node, or -1.
__device__ inline int catalog_find(const int32_t* child_token, int c0, int c1, int t) {
  int lo = c0, hi = c1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (child_token[mid] < t) lo = mid + 1; else hi = mid;
  }
  return lo < c1 && child_token[lo] == t ? lo : -1;
}

// Children range of beam b's trie node; empty for -1 and, flagged, for an
// id or range outside the trie.
__device__ inline void catalog_range(const PruneArgs& a, int b, int& c0, int& c1) {
  const int node = a.beam_node[b];
  c0 = c1 = 0;
  if (node < 0) return;
  if (node >= a.num_nodes) {
    flag_status(a.dev_status, GR_DEV_BAD_NODE);
    return;
  }
  const int s0 = a.node_start[node], s1 = a.node_start[node + 1];
  if (s0 < 0 || s1 < s0 || s1 > a.num_edges) {
    flag_status(a.dev_status, GR_DEV_BAD_NODE);
    return;
  }
  c0 = s0;
  c1 = s1;
}

// v of lane (lane ^ M), M < 32: ds_swizzle's bit-mask mode (and 0x1F, xor M)
// reads across the 32-lane half without the address arithmetic of a
// general shuffle
template <int M>
__device__ inline float lane_xor(float v) {
  static_assert(M > 0 && M < 32, "within a 32-lane half");
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (M << 10) | 0x1F));
}

__device__ inline float wave_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  v = fmaxf(v, lane_xor<16>(v));
  v = fmaxf(v, lane_xor<8>(v));
  v = fmaxf(v, lane_xor<4>(v));
  v = fmaxf(v, lane_xor<2>(v));
  return fmaxf(v, lane_xor<1>(v));
}

// xor butterfly sum over the wave, masks 32, 16, .., 1 in turn (every lane
// ends with the same float: each step adds the same two values)
__device__ inline float wave_sum_butterfly(float v) {
  v = v + __shfl_xor(v, 32, 64);
  v = v + lane_xor<16>(v);
  v = v + lane_xor<8>(v);
  v = v + lane_xor<4>(v);
  v = v + lane_xor<2>(v);
  return v + lane_xor<1>(v);
}

// block-wide exclusive scan of one int per thread (NT threads); returns the total
template <int NT = PR_THREADS>
__device__ int block_scan(int v, int& excl, int* tmp) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int incl = wave_incl_scan(v);
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    base += (w < wave) ? tmp[w] : 0;
    total += tmp[w];
  }
  excl = base + incl - v;
  __syncthreads();
  return total;
}

// Radix select: the need-th largest (1-based) of the unsigned keys that
// for_each(f) hands to f (each thread its own keys; at least `need` keys in
// total, all within [kmin, kmax]).  The bits above the highest bit in which
// kmin and kmax differ are common to every key; below it, digits of 11 bits
// from the top: a pass histograms the keys that match the digits fixed so far
// and walks the bins from the top.  Stops early once the bin holding the
// need-th key holds exactly the keys still needed.
// Result: keys with (key & mask) > prefix are above the boundary (need_in -
// need of them); the `need` remaining come from the eq keys with (key & mask)
// == prefix -- all of them when eq == need, else (mask all ones) a choice
// among equal keys left to the caller.
template <typename K>
struct RadixSel {
  K prefix, mask;
  int need, eq;
};

__device__ inline int clz_key(uint32_t x) { return __builtin_clz(x); }
__device__ inline int clz_key(uint64_t x) { return __builtin_clzll(x); }

template <int NT, typename K, typename ForEach>
__device__ RadixSel<K> radix_select(ForEach for_each, int need, K kmin, K kmax, int* hist, int* itmp, int* sel) {
  constexpr int KB = 8 * sizeof(K);
  constexpr int BPT = PR_BINS / NT;  // bins owned per thread in the top-down walk
  const int tid = threadIdx.x;
  const K dx = kmin ^ kmax;
  const int nbits = dx == 0 ? 1 : KB - clz_key(dx);
  RadixSel<K> rs;
  rs.mask = nbits >= KB ? K(0) : ~((K(1) << nbits) - 1);
  rs.prefix = kmax & rs.mask;
  rs.need = need;
  rs.eq = 0;
#pragma unroll 1
  for (int hi_bit = nbits; hi_bit > 0; hi_bit -= 11) {
    const int shift = hi_bit > 11 ? hi_bit - 11 : 0;
    const K dmask = (K(1) << (hi_bit - shift)) - 1;
    for (int i = tid; i < PR_BINS; i += NT) hist[i] = 0;
    __syncthreads();
    const K pm = rs.mask, pp = rs.prefix;
    for_each([&](K u) {
      if ((u & pm) == pp) atomicAdd(&hist[(int)((u >> shift) & dmask)], 1);
    });
    __syncthreads();
    int loc = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) loc += hist[BPT * tid + i];
    int excl;
    const int tot = block_scan<NT>(loc, excl, itmp);
    const int above = tot - excl - loc;  // keys in bins owned by higher threads
    if (above < rs.need && rs.need <= above + loc) {
      int acc = above;
      for (int i = BPT - 1; i >= 0; --i) {
        const int h = hist[BPT * tid + i];
        if (acc + h >= rs.need) {
          sel[0] = BPT * tid + i;
          sel[1] = acc;
          sel[2] = h;
          break;
        }
        acc += h;
      }
    }
    __syncthreads();
    rs.prefix |= (K)sel[0] << shift;
    rs.mask |= dmask << shift;
    rs.need -= sel[1];
    rs.eq = sel[2];
    __syncthreads();
    if (rs.eq == rs.need) break;
  }
  return rs;
}

// Row top-k1 by (logit desc, token asc) through a radix select of the k1-th
// largest key T over the keys >= t0, re-reading the row from memory: the path
// for rows with many keys near the top (ties, flat rows), kept out of line so
// the register-resident path does not carry its state.  Leaves the k1
// selected, ranked, in ox / ov.
__device__ __noinline__ void row_topk_radix(const float* xg, int V, int k1, uint32_t t0, uint32_t kmax, uint64_t* sk,
                                            float* ox, int* ov, int* hist, int* itmp, int* sel) {
  const int tid = threadIdx.x;
  const int nch = (V + PR_CHUNK - 1) / PR_CHUNK;
  auto valid = [&](int c) { return c * PR_CHUNK + PR_VEC * tid < V; };
  auto getk = [&](int c, int j) -> uint32_t { return fkey(xg[c * PR_CHUNK + PR_VEC * tid + j] + 0.0f); };
  const RadixSel<uint32_t> rs = radix_select<PR_THREADS, uint32_t>(
      [&](auto&& f) {
        for (int c = 0; c < nch; ++c) {
          if (valid(c)) {
#pragma unroll
            for (int j = 0; j < PR_VEC; ++j) {
              const uint32_t u = getk(c, j);
              if (u >= t0) f(u);
            }
          }
        }
      },
      k1, t0, kmax, hist, itmp, sel);
  const uint32_t T = rs.prefix, Tm = rs.mask;
  const int need = rs.need, eq_cnt = rs.eq;
  // keys above the boundary: k1 - need of them, all taken; keys at it: all
  // when eq_cnt == need, else the first `need` by token
  int gt = 0, eq = 0;
  for (int c = 0; c < nch; ++c) {
    if (valid(c)) {
#pragma unroll
      for (int j = 0; j < PR_VEC; ++j) {
        const uint32_t u = getk(c, j);
        gt += (u & Tm) > T;
        eq += (u & Tm) == T && u >= t0;
      }
    }
  }
  int off;
  const int ngt = block_scan(gt, off, itmp);
  for (int c = 0; c < nch; ++c) {
    if (valid(c)) {
#pragma unroll
      for (int j = 0; j < PR_VEC; ++j) {
        const uint32_t u = getk(c, j);
        if ((u & Tm) > T) sk[off++] = row_key(u, c * PR_CHUNK + PR_VEC * tid + j);
      }
    }
  }
  if (eq_cnt == need) {  // every key at the boundary is taken: order is irrelevant here
    int eoff;
    block_scan(eq, eoff, itmp);
    for (int c = 0; c < nch; ++c) {
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          const uint32_t u = getk(c, j);
          if ((u & Tm) == T && u >= t0) sk[ngt + eoff++] = row_key(u, c * PR_CHUNK + PR_VEC * tid + j);
        }
      }
    }
  } else {  // ties at T (all bits fixed): ascending token order (chunk, then thread, then lane)
    int taken = 0;
    for (int c = 0; c < nch; ++c) {
      int tc = 0;
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) tc += getk(c, j) == T;
      }
      int toff;
      const int ctot = block_scan(tc, toff, itmp);
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          if (getk(c, j) == T) {
            const int pos = taken + toff;
            if (pos < need) sk[ngt + pos] = row_key(T, c * PR_CHUNK + PR_VEC * tid + j);
            ++toff;
          }
        }
      }
      taken += ctot;
      if (taken >= need) break;
    }
  }
  __syncthreads();
  // rank the k1 selected: (logit desc, token asc)
  for (int i = tid; i < k1; i += PR_THREADS) {
    const uint64_t ki = sk[i];
    int rank = 0;
#pragma unroll 8
    for (int q = 0; q < k1; ++q) rank += sk[q] > ki;
    ox[rank] = fval((uint32_t)(ki >> 32));
    ov[rank] = (int)~(uint32_t)ki;
  }
}

// MAXC > 0: row held in registers (<= MAXC chunks); 0: re-read from memory.
// CATALOG: the beam's top-k candidates outside its trie node's children are
// dropped (the reference masks them to -inf after the sampler's per-beam
// top-K, serving_engine.py:504-506, 526-528).
// FULL: the row is exactly MAXC chunks (V = MAXC * PR_CHUNK), so every chunk
// and element is live: no padding, no per-chunk bounds tests (the same
// arithmetic, in the same order, as the general form).
template <int MAXC, bool CATALOG = false, bool FULL = false>
__global__ __launch_bounds__(PR_THREADS) void prune_rows(PruneArgs a) {
  static_assert(!FULL || MAXC > 0, "a full row is held in registers");
  __shared__ uint64_t sk[PR_MAXK];  // candidates as row_key
  // radix histogram (fallback path) or the survivors' partial ranks; then
  // the row's top-k1 logits and tokens (ox, ov), written once the histogram
  // or the partial ranks are dead (the LDS saved lets a seventh workgroup
  // share a CU)
  constexpr int HP_INTS = PR_BINS > PR_SURV * (PR_THREADS / 64) ? PR_BINS : PR_SURV * (PR_THREADS / 64);
  static_assert(HP_INTS >= 2 * PR_MAXK, "ox and ov fit the histogram's space");
  __shared__ int hist_part[HP_INTS];
  int* hist = hist_part;
  int* part = hist_part;
  float* ox = reinterpret_cast<float*>(hist_part);
  int* ov = hist_part + PR_MAXK;
  __shared__ float wred[PR_THREADS / 64];
  __shared__ int itmp[PR_THREADS / 64];
  __shared__ int sel[3];
  __shared__ uint32_t wkey[PR_THREADS / 64];
  __shared__ int eos_pos;
  __shared__ double lse_sh;  // the row's LSE, for the logprob lists

  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* xg = a.logits + (int64_t)row * a.row_stride;
  const int V = a.V, k1 = a.k1;
  const int nch = (V + PR_CHUNK - 1) / PR_CHUNK;

  float xr[MAXC > 0 ? MAXC : 1][PR_VEC];
  if constexpr (MAXC > 0) {
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int idx = c * PR_CHUNK + PR_VEC * tid;
      f32x4_t v;
      if constexpr (FULL) {
        v = *reinterpret_cast<const f32x4_t*>(xg + idx);
      } else {
        v = f32x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (c < nch && idx < V) v = *reinterpret_cast<const f32x4_t*>(xg + idx);
      }
#pragma unroll
      for (int j = 0; j < PR_VEC; ++j) xr[c][j] = v[j];  // (-0 stays: only survivor keys are made canonical)
    }
  }
  auto valid = [&](int c) { return c * PR_CHUNK + PR_VEC * tid < V; };
  // row max, exp-sum and survivor scan: with the row in registers the
  // padding past V is -inf -- neutral for the max, +0 for the sum, and a
  // survivor only when t0 admits every key, which sends the row to the
  // radix path (more than PR_SURV survivors) where valid() is checked
  auto live = [&](int c) { return MAXC > 0 || valid(c); };
  auto get = [&](int c, int j) -> float {
    if constexpr (MAXC > 0) return xr[c][j];
    else return xg[c * PR_CHUNK + PR_VEC * tid + j] + 0.0f;
  };
#define PR_FOR_CHUNKS(c) \
  _Pragma("unroll") for (int c = 0; c < (MAXC > 0 ? MAXC : nch); ++c) if (FULL || c < nch)

  // ---- row max; also the thread's second-largest chunk maximum (an element
  // other than the thread maximum: it tightens the selection bound below) ----
  float tm = -INFINITY, t2 = -INFINITY;
  PR_FOR_CHUNKS(c) {
    if (live(c)) {
      const float cm = fmaxf(fmaxf(get(c, 0), get(c, 1)), fmaxf(get(c, 2), get(c, 3)));
      t2 = fmaxf(t2, cm >= tm ? tm : cm);  // NaN chunk maxima (all four NaN) are skipped
      tm = fmaxf(tm, cm);
    }
  }
  const float wm = wave_max(tm);
  if (lane == 0) wred[wave] = wm;
  __syncthreads();
  float m = wred[0];
#pragma unroll
  for (int w = 1; w < PR_THREADS / 64; ++w) m = fmaxf(m, wred[w]);
  __syncthreads();

  // ---- fixed-order exp-sum: thread partial in element order, xor butterfly, waves pairwise ----
  double c_row = -INFINITY;
  double lse_row = INFINITY;  // a row of -inf logits has logprobs -inf
  if (m != -INFINITY) {
    float acc = 0.0f;
    const float ml = m * 0x1.715476p+0f;
    PR_FOR_CHUNKS(c) {
      if (live(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          const float t = __builtin_fmaf(get(c, j), 0x1.715476p+0f, -ml);
          acc = acc + exp2_neg(t);
        }
      }
    }
    acc = wave_sum_butterfly(acc);
    if (lane == 0) wred[wave] = acc;
    __syncthreads();
    // one wave works out the LSE (float64): only thread 0 and the logprob
    // lists, which read it from LDS, need it
    if (__builtin_amdgcn_readfirstlane(wave) == 0) {
      const float S = (wred[0] + wred[1]) + (wred[2] + wred[3]);
      const double lse = (double)m + log_f64((double)S);
      c_row = (a.cum64 ? a.cum64[row] : (double)a.cum[row]) - lse;
      lse_row = lse;
    }
  }

  // ---- stage 1: row top-k1 by (logit desc, token asc) ----
  // Lower bound t0 of the k1-th largest key: per wave, the ceil(k1/4)-th
  // largest of the threads' maxima and second-largest chunk maxima (two
  // distinct elements per thread) rounded down to its top 16 bits (bisection
  // over that range with wave ballots), least over the waves.  Every wave then
  // holds that many distinct elements with a key >= t0: at least k1 keys in
  // all.  Only keys >= t0 can be selected; with few of them they are ranked
  // directly.
  uint32_t t0 = 0;
  if (k1 <= PR_THREADS) {
    const int kw = (k1 + 3) >> 2;
    const uint32_t a0 = fkey(tm) >> 16;  // the top 16 bits of the key suffice for a bound
    const uint32_t a1 = fkey(t2) >> 16;
    // invariant: at least kw of the lanes' a0, a1 are >= lo; the answer is <= hi (bounds
    // are wave-uniform, kept in scalar registers)
    uint32_t lo = 0, hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(fkey(m) >> 16));
    auto count_ge = [&](uint32_t v) {
      return __builtin_popcountll(__builtin_amdgcn_ballot_w64(a0 >= v)) +
             __builtin_popcountll(__builtin_amdgcn_ballot_w64(a1 >= v));
    };
    // first one trial 256 units of the 16-bit key below the maximum (two
    // binades of the 7 mantissa bits it keeps): where it holds, the bisection
    // needs 8 steps instead of 16
    if (hi > 256 && count_ge(hi - 256) >= kw) lo = hi - 256;
    while (lo < hi) {
      const uint32_t mid = lo + ((hi - lo + 1) >> 1);
      if (count_ge(mid) >= kw) lo = mid;
      else hi = mid - 1;
    }
    if (lane == 0) wkey[wave] = lo << 16;
    __syncthreads();
    t0 = wkey[0];
#pragma unroll
    for (int w = 1; w < PR_THREADS / 64; ++w) t0 = min(t0, wkey[w]);
    // a bound at or below -inf (a wave of padding, rounded down into the NaN
    // patterns 0 .. fkey(-inf)) admits every key
    if (t0 <= fkey(-INFINITY)) t0 = 0;
  }
  // the same bound on the logits (t0 = 0 admits every key)
  const float t0f = t0 == 0 ? -INFINITY : fval(t0);
  // survivors -> LDS in thread order (a block scan hands out each thread's slots)
  int ns = 0;
  PR_FOR_CHUNKS(c) {
    if (live(c)) {
#pragma unroll
      for (int j = 0; j < PR_VEC; ++j) ns += get(c, j) >= t0f;
    }
  }
  int pos;
  // (the total is the same in every thread: held in a scalar register)
  const int n_surv = __builtin_amdgcn_readfirstlane(block_scan(ns, pos, itmp));
  // more than PR_SURV survivors: the radix path below selects from the row
  // itself, so nothing is written (and no write needs a bound check)
  if (n_surv <= PR_SURV && ns > 0) {
    PR_FOR_CHUNKS(c) {
      if (live(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          const float y = get(c, j);
          if (y >= t0f) {  // (logit bits, token); made a row key once, below
            sk[pos] = ((uint64_t)__builtin_bit_cast(uint32_t, y) << 32) | (uint32_t)(c * PR_CHUNK + PR_VEC * tid + j);
            ++pos;
          }
        }
      }
    }
  }
  __syncthreads();
  const int S = n_surv;
  if (S <= PR_SURV && k1 <= PR_THREADS) {
    // the survivors as row keys (all distinct: the token is part of the key)
    auto to_key = [](uint64_t raw) {  // (+ 0.0f: -0 orders as +0)
      return row_key(fkey(__builtin_bit_cast(float, (uint32_t)(raw >> 32)) + 0.0f), (int)(uint32_t)raw);
    };
#pragma unroll
    for (int h = 0; h < PR_SURV / PR_THREADS; ++h) {
      const int i = tid + h * PR_THREADS;
      if (i < S) sk[i] = to_key(sk[i]);
    }
    __syncthreads();
    // rank of survivor i = number of survivors with a greater key; the k1 of
    // rank < k1 are the row's top-k1, in order.  Wave w counts over the
    // survivors [w*Q, (w+1)*Q) for every target; lane l holds the targets l,
    // l + 64, ...; the four partial counts are summed in LDS.
    // (wave-uniform bounds in scalar registers: the count loop is a scalar loop)
    const int Q = (S + 3) >> 2, q0 = __builtin_amdgcn_readfirstlane(wave) * Q, q1 = min(S, q0 + Q);
    auto partial = [&](auto tg_c) {
      constexpr int TG = decltype(tg_c)::value;
      uint64_t kt[TG];
      int rk[TG];
#pragma unroll
      for (int mi = 0; mi < TG; ++mi) {
        const int i = lane + 64 * mi;
        kt[mi] = i < S ? sk[i] : ~0ull;
        rk[mi] = 0;
      }
#pragma unroll 4
      for (int q = q0; q < q1; ++q) {
        const uint64_t kq = sk[q];
#pragma unroll
        for (int mi = 0; mi < TG; ++mi) rk[mi] += kq > kt[mi];
      }
#pragma unroll
      for (int mi = 0; mi < TG; ++mi) {
        const int i = lane + 64 * mi;
        if (i < S) part[wave * PR_SURV + i] = rk[mi];
      }
    };
    if (S <= 128) partial(std::integral_constant<int, 2>{});
    else if (S <= 192) partial(std::integral_constant<int, 3>{});
    else if (S <= 256) partial(std::integral_constant<int, 4>{});
    else partial(std::integral_constant<int, 8>{});
    __syncthreads();
    int rk_h[PR_SURV / PR_THREADS];
#pragma unroll
    for (int h = 0; h < PR_SURV / PR_THREADS; ++h) {
      const int i = tid + h * PR_THREADS;
      int rank = k1;
      if (i < S) {
        rank = 0;
#pragma unroll
        for (int w = 0; w < PR_THREADS / 64; ++w) rank += part[w * PR_SURV + i];
      }
      rk_h[h] = rank;
    }
    __syncthreads();  // ox and ov take the partial ranks' space
#pragma unroll
    for (int h = 0; h < PR_SURV / PR_THREADS; ++h) {
      const int i = tid + h * PR_THREADS;
      if (rk_h[h] < k1) {
        const uint64_t ki = sk[i];
        ox[rk_h[h]] = fval((uint32_t)(ki >> 32));
        ov[rk_h[h]] = (int)~(uint32_t)ki;
      }
    }
  } else {
    row_topk_radix(xg, V, k1, t0, fkey(m), sk, ox, ov, hist, itmp, sel);
  }
#undef PR_FOR_CHUNKS
  if (tid == 0) {
    eos_pos = -1;
    lse_sh = lse_row;
  }
  __syncthreads();
  if (a.cand_token) {
    // the row's whole top-k1 list with its logprobs (the sampler's per-beam
    // logprobs, before EOS or the catalog take anything out)
    const double lse = lse_sh;
    for (int i = tid; i < k1; i += PR_THREADS) {
      a.cand_token[(int64_t)row * k1 + i] = ov[i];
      a.cand_logprob[(int64_t)row * k1 + i] = (float)((double)ox[i] - lse);
    }
  }
  float* cx = a.cand_x + (int64_t)row * k1;
  int32_t* cv = a.cand_v + (int64_t)row * k1;
  if constexpr (CATALOG) {
    // keep the candidates among the node's children, in order; EOS (when a
    // child) leaves the pool with its score
    int c0, c1;
    catalog_range(a, row, c0, c1);
    constexpr int PER = PR_MAXK / PR_THREADS;
    bool kf[PER];
    int keep = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = tid * PER + j;
      bool k = false;
      if (i < k1 && catalog_find(a.child_token, c0, c1, ov[i]) >= 0) {
        if (ov[i] == a.eos) eos_pos = i;
        else k = true;
      }
      kf[j] = k;
      keep += k;
    }
    int dst;
    const int total = block_scan(keep, dst, itmp);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = tid * PER + j;
      if (kf[j]) {
        cx[dst] = ox[i];
        cv[dst] = ov[i];
        ++dst;
      }
    }
    for (int i = total + tid; i < k1; i += PR_THREADS) {
      cx[i] = -INFINITY;
      cv[i] = -1;
    }
  } else {
    if (a.eos >= 0)
      for (int i = tid; i < k1; i += PR_THREADS)
        if (ov[i] == a.eos) eos_pos = i;
    __syncthreads();
    const int e = eos_pos;
    for (int i = tid; i < k1; i += PR_THREADS) {
      const int src = (e >= 0 && i >= e) ? i + 1 : i;
      cx[i] = src < k1 ? ox[src] : -INFINITY;
      cv[i] = src < k1 ? ov[src] : -1;
    }
  }
  const int e = eos_pos;
  if (tid == 0) {
    a.row_c[row] = c_row;
    const double es = e >= 0 && c_row != -INFINITY ? (double)ox[e] + c_row : -INFINITY;
    if (a.eos_score64) a.eos_score64[row] = es;
    else if (a.eos_score) a.eos_score[row] = (float)es;
  }
}

// ---- kernel 2: per-request top-k over the rows' candidate lists -----------
typedef int32_t i32x4_t __attribute__((__vector_size__(4 * sizeof(int32_t))));
constexpr int MG_REG = 16;  // candidates per thread held in registers (W * k1 <= 16384)

template <int MPT>  // > 0: thread t holds candidates [MPT t, MPT t + MPT) in registers; 0: re-read per pass
__global__ __launch_bounds__(MG_THREADS) void prune_merge(PruneArgs a) {
  kernarg_lines<kernarg_line_count<PruneArgs>()>();
  __shared__ double cs[PR_MAXW];
  // the radix histogram during the selection, then the selected keys / flats
  __shared__ __attribute__((aligned(16))) uint8_t work[PR_MAXK * 16];
  __shared__ int itmp[MG_THREADS / 64];
  __shared__ uint64_t kred[MG_THREADS / 64][2];
  __shared__ int sel[3];
  int* hist = reinterpret_cast<int*>(work);
  uint64_t* fkeys = reinterpret_cast<uint64_t*>(work);
  int64_t* ffl = reinterpret_cast<int64_t*>(work + PR_MAXK * 8);

  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int W = a.W, k1 = a.k1, k = a.k;
  const int n = W * k1;
  const int64_t rbase = (int64_t)r * W;
  const float* gx = a.cand_x + rbase * k1;
  const int32_t* gv = a.cand_v + rbase * k1;
  for (int b = tid; b < W; b += MG_THREADS) cs[b] = a.row_c[rbase + b];
  __syncthreads();

  // candidate i = b * k1 + j (row b, list position j): score cum - lse + logit
  // as its order-preserving key; padding entries (token -1) are no candidates
  // and get key 0, which no score has
  auto score_key = [&](float x, int b) -> uint64_t {
    const double c = cs[b];
    return dkey(c == -INFINITY ? -INFINITY : ((double)x + c) + 0.0);  // -0 -> +0
  };
  constexpr int NR = MPT > 0 ? MPT : 1;
  uint64_t ck[NR];
  int cv[NR];
  const int i0 = NR * tid;
  if constexpr (MPT > 0) {
    float xv[MPT];
    if (i0 + MPT <= n) {  // the request's lists start 16-byte aligned (n % 4 == 0 on this path)
#pragma unroll
      for (int q = 0; q < MPT; q += 4) {
        const f32x4_t x4 = *reinterpret_cast<const f32x4_t*>(gx + i0 + q);
        const i32x4_t v4 = *reinterpret_cast<const i32x4_t*>(gv + i0 + q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xv[q + e] = x4[e];
          cv[q + e] = v4[e];
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < MPT; ++q) {
        const bool in = i0 + q < n;
        xv[q] = in ? gx[in ? i0 + q : 0] : 0.0f;
        cv[q] = in ? gv[in ? i0 + q : 0] : -1;
      }
    }
    int b = min(i0 / k1, W - 1), j = i0 - b * k1;
#pragma unroll
    for (int q = 0; q < MPT; ++q) {
      ck[q] = cv[q] >= 0 ? score_key(xv[q], b) : 0;
      if (++j == k1) {
        j = 0;
        b = min(b + 1, W - 1);
      }
    }
  }
  // f(q, key) for this thread's candidates (MPT = 0: keys recomputed from memory)
  auto for_cand = [&](auto&& f) {
    if constexpr (MPT > 0) {
#pragma unroll
      for (int q = 0; q < MPT; ++q)
        if (ck[q] != 0) f(q, ck[q]);
    } else {
      for (int i = tid; i < n; i += MG_THREADS) {
        const int v = gv[i];
        if (v >= 0) f(i, score_key(gx[i], i / k1));
      }
    }
  };
  // (row, token) of candidate q (MPT > 0: index i0 + q; else flat index i)
  auto cand_bv = [&](int q, int& b, int& v) {
    const int i = MPT > 0 ? i0 + q : q;
    b = i / k1;
    v = MPT > 0 ? cv[MPT > 0 ? q : 0] : gv[i];
  };
  int mv = 0;
  uint64_t kmin = ~0ull, kmax = 0;
  for_cand([&](int, uint64_t u) {
    ++mv;
    kmin = u < kmin ? u : kmin;
    kmax = u > kmax ? u : kmax;
  });
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) {
    const uint64_t a0 = __shfl_xor(kmin, msk, 64), a1 = __shfl_xor(kmax, msk, 64);
    kmin = a0 < kmin ? a0 : kmin;
    kmax = a1 > kmax ? a1 : kmax;
  }
  if ((tid & 63) == 0) {
    kred[tid >> 6][0] = kmin;
    kred[tid >> 6][1] = kmax;
  }
  int excl;
  const int M = block_scan<MG_THREADS>(mv, excl, itmp);  // its barriers order the kred writes
  for (int w = 0; w < MG_THREADS / 64; ++w) {
    kmin = kred[w][0] < kmin ? kred[w][0] : kmin;
    kmax = kred[w][1] > kmax ? kred[w][1] : kmax;
  }
  const int nsel = M < k ? M : k;

  // boundary score (k-th largest), then among exact ties at it the lowest flat
  // index b * V + v (key ~(b << 32 | v): the largest key is the lowest index)
  RadixSel<uint64_t> r1{0, 0, 0, 0}, r2{0, 0, 0, 0};
  bool ties = false;
  if (M > k) {
    r1 = radix_select<MG_THREADS, uint64_t>(
        [&](auto&& f) { for_cand([&](int, uint64_t u) { f(u); }); }, k, kmin, kmax, hist, itmp, sel);
    if (r1.eq != r1.need) {
      ties = true;
      const uint64_t tmin = ~(((uint64_t)(W - 1) << 32) | (uint32_t)(a.V - 1));
      r2 = radix_select<MG_THREADS, uint64_t>(
          [&](auto&& f) {
            for_cand([&](int q, uint64_t u) {
              if (u == r1.prefix) {
                int b, v;
                cand_bv(q, b, v);
                f(~(((uint64_t)b << 32) | (uint32_t)v));
              }
            });
          },
          r1.need, tmin, ~0ull, hist, itmp, sel);
    }
  }
  auto selected = [&](int q, uint64_t key) -> bool {
    if (M <= k) return true;
    const uint64_t u = key & r1.mask;
    if (u != r1.prefix) return u > r1.prefix;
    if (!ties) return true;
    int b, v;
    cand_bv(q, b, v);
    return (~(((uint64_t)b << 32) | (uint32_t)v) & r2.mask) >= r2.prefix;
  };
  int cnt = 0;
  for_cand([&](int q, uint64_t u) { cnt += selected(q, u); });
  int off;
  block_scan<MG_THREADS>(cnt, off, itmp);  // nsel in total; the histogram is dead from here
  for_cand([&](int q, uint64_t u) {
    if (selected(q, u)) {
      int b, v;
      cand_bv(q, b, v);
      fkeys[off] = u;
      ffl[off] = (int64_t)b * a.V + v;
      ++off;
    }
  });
  __syncthreads();
  // final order of the selected set: (score desc, flat asc)
  for (int i = tid; i < nsel; i += MG_THREADS) {
    const uint64_t ki = fkeys[i];
    const int64_t fi = ffl[i];
    int rank = 0;
#pragma unroll 8
    for (int u = 0; u < nsel; ++u) {
      const uint64_t kq = fkeys[u];
      const int64_t fq = ffl[u];
      rank += (kq > ki) | ((kq == ki) & (fq < fi));
    }
    const int64_t o = (int64_t)r * k + rank;
    const int b = (int)(fi / a.V);
    a.parent[o] = b;
    a.token[o] = (int32_t)(fi - (int64_t)b * a.V);
    put_score(a, o, dval(ki));
  }
  for (int i = nsel + tid; i < k; i += MG_THREADS) {
    const int64_t o = (int64_t)r * k + i;
    a.parent[o] = -1;
    a.token[o] = -1;
    put_score(a, o, -INFINITY);
  }
}

// ---- two-stage merge -------------------------------------------------------
// Stage 1 (prune_merge_part): one workgroup per (request, group of gr rows,
// gr * k1 <= MG_GROUP_CAND candidates, MG_PART_PER_THREAD per thread): the
// group's top-k by (score desc, flat asc), sorted, into the part buffer as
// (score key, flat index) pairs.  Stage 2, one workgroup per request, merges
// the groups' sorted lists (prune_merge_lists: each entry's rank is its
// position plus, per other list, a binary search) or, for very many groups,
// selects again (prune_merge_final).  A candidate of
// the request's top-k is within its group's top-k under the same order, so
// both stages together select what a single pass over all candidates does;
// the work of stage 1 is spread over every request's groups.  The rows' lists
// arrive sorted, so stage 1 bounds the group's k-th score from below by the
// k-th score of the MG_TOP_ROWS rows with the highest k-th entries (their
// lists merged by a small tournament) and merges the few other entries at or
// above it into that list by search; groups whose lists are out of flat
// order, or with more rows or such entries than the tables hold, select by
// radix select and counting.
constexpr int MG_PART_PER_THREAD = 4;
constexpr int MG_GROUP_CAND = MG_PART_PER_THREAD * MG_THREADS;

// Top-k by (key desc, flat asc) of the candidates the NT threads hold
// (thread's ck[q] = 0: no candidate).  Sets take[q] for the selected ones and
// returns their number, min(valid, k); *off is this thread's first output
// slot (exclusive scan over the threads in thread order).
template <int NT, int MPT>
__device__ int merge_select(const uint64_t (&ck)[MPT], const int64_t (&cf)[MPT], int k, int64_t flat_end,
                            bool (&take)[MPT], int& off, int* hist, int* itmp, int* sel, uint64_t (*kred)[2]) {
  const int tid = threadIdx.x;
  int mv = 0;
  uint64_t kmin = ~0ull, kmax = 0;
#pragma unroll
  for (int q = 0; q < MPT; ++q) {
    if (ck[q] != 0) {
      ++mv;
      kmin = ck[q] < kmin ? ck[q] : kmin;
      kmax = ck[q] > kmax ? ck[q] : kmax;
    }
  }
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) {
    const uint64_t a0 = __shfl_xor(kmin, msk, 64), a1 = __shfl_xor(kmax, msk, 64);
    kmin = a0 < kmin ? a0 : kmin;
    kmax = a1 > kmax ? a1 : kmax;
  }
  if ((tid & 63) == 0) {
    kred[tid >> 6][0] = kmin;
    kred[tid >> 6][1] = kmax;
  }
  int excl;
  const int M = block_scan<NT>(mv, excl, itmp);  // its barriers order the kred writes
  for (int w = 0; w < NT / 64; ++w) {
    kmin = kred[w][0] < kmin ? kred[w][0] : kmin;
    kmax = kred[w][1] > kmax ? kred[w][1] : kmax;
  }
  // boundary key (k-th largest), then among exact ties at it the lowest flat
  // indices (tie key ~flat: the largest is the lowest index)
  RadixSel<uint64_t> r1{0, 0, 0, 0}, r2{0, 0, 0, 0};
  bool ties = false;
  if (M > k) {
    r1 = radix_select<NT, uint64_t>(
        [&](auto&& f) {
#pragma unroll
          for (int q = 0; q < MPT; ++q)
            if (ck[q] != 0) f(ck[q]);
        },
        k, kmin, kmax, hist, itmp, sel);
    if (r1.eq != r1.need) {
      ties = true;
      r2 = radix_select<NT, uint64_t>(
          [&](auto&& f) {
#pragma unroll
            for (int q = 0; q < MPT; ++q)
              if (ck[q] != 0 && ck[q] == r1.prefix) f(~(uint64_t)cf[q]);
          },
          r1.need, ~(uint64_t)(flat_end - 1), ~0ull, hist, itmp, sel);
    }
  }
  int cnt = 0;
#pragma unroll
  for (int q = 0; q < MPT; ++q) {
    bool t = ck[q] != 0;
    if (t && M > k) {
      const uint64_t u = ck[q] & r1.mask;
      if (u != r1.prefix) t = u > r1.prefix;
      else if (ties) t = (~(uint64_t)cf[q] & r2.mask) >= r2.prefix;
    }
    take[q] = t;
    cnt += t;
  }
  block_scan<NT>(cnt, off, itmp);
  return M < k ? M : k;
}

// floor(i / d) for 0 <= i < 2^20 and d >= 1: the float estimate is off by at
// most one either way, which the two corrections remove.
__device__ inline int div_small(int i, int d, float rcp) {
  int q = (int)((float)i * rcp);
  q += (q + 1) * d <= i;
  q -= q * d > i;
  return q;
}

// Entries of a list sorted by (key desc, position asc) that come before
// (ke, ie): list entry j has key lk[j] and position li[j] (li null: position
// j).  Branch-free lower bound; positions are read only at equal keys.
__device__ inline int count_before(const uint64_t* lk, const unsigned short* li, int n, uint64_t ke, int ie) {
  int b = 0;
  while (n > 1) {
    const int h = n >> 1;
    const uint64_t kj = lk[b + h - 1];
    bool bf = kj > ke;
    if (kj == ke) bf = (li ? (int)li[b + h - 1] : b + h - 1) < ie;
    b = bf ? b + h : b;
    n -= h;
  }
  if (n == 1) {
    const uint64_t kj = lk[b];
    bool bf = kj > ke;
    if (kj == ke) bf = (li ? (int)li[b] : b) < ie;
    b += bf;
  }
  return b;
}

constexpr int MG_TOP_ROWS = 8;    // rows whose merged top-k bounds the group's k-th score
constexpr int MG_MAX_ROWS = 128;  // rows a group may hold on the bounded path
constexpr int MG_MAX_EXTRA = 64;  // other rows' entries at or above the bound, merged one by one

__global__ __launch_bounds__(MG_THREADS) void prune_merge_part(PruneArgs a) {
  __shared__ uint64_t mk[2][MG_GROUP_CAND];        // [0]: the group's keys by position; then merge lists
  __shared__ unsigned short mi[2][MG_GROUP_CAND];  // position in the group of each merge-list entry
  __shared__ int mtok[MG_GROUP_CAND];              // token of the group's candidate i
  __shared__ uint64_t rowk[MG_MAX_ROWS];           // key of each row's k-th entry
  __shared__ int top_row[MG_TOP_ROWS];
  __shared__ unsigned char is_top[MG_MAX_ROWS];
  __shared__ uint64_t xk[MG_MAX_EXTRA];
  __shared__ int xi[MG_MAX_EXTRA];
  __shared__ int hist[PR_BINS];
  __shared__ uint64_t fkeys[PR_MAXK];
  __shared__ int64_t ffl[PR_MAXK];
  __shared__ int itmp[MG_THREADS / 64];
  __shared__ uint64_t kred[MG_THREADS / 64][2];
  __shared__ int sel[3];
  __shared__ int unsorted, n_extra;
  constexpr int MPT = MG_PART_PER_THREAD;
  const int r = blockIdx.x / a.ng, g = blockIdx.x - r * a.ng;
  const int tid = threadIdx.x;
  const int k1 = a.k1, k = a.k;
  const float rk1 = 1.0f / (float)k1;
  const int b0 = g * a.gr, b1 = min(a.W, b0 + a.gr), nl = b1 - b0;
  const int n = nl * k1;  // <= MG_GROUP_CAND
  const int64_t row0 = (int64_t)r * a.W + b0;
  const float* gx = a.cand_x + row0 * k1;
  const int32_t* gv = a.cand_v + row0 * k1;
  // the bounded path: the k-th entry of a row exists and the rows fit the tables
  const bool bounded = k <= k1 && nl <= MG_MAX_ROWS;
  if (tid == 0) {
    unsorted = 0;
    n_extra = 0;
  }
  // thread t: candidates i = t + q NT of the group (row i / k1); every load
  // is issued at a clamped index before any is used
  int vq[MPT], bq[MPT];
  float xq[MPT];
  double cq[MPT];
#pragma unroll
  for (int q = 0; q < MPT; ++q) {
    const int i = min(tid + q * MG_THREADS, n - 1);
    bq[q] = div_small(i, k1, rk1);
    vq[q] = gv[i];
    xq[q] = gx[i];
    cq[q] = a.row_c[row0 + bq[q]];
  }
  // pin every load ahead of the first use (else the compiler sinks the
  // logit and row loads under the validity test: a second round trip)
#pragma unroll
  for (int q = 0; q < MPT; ++q) __asm__ volatile("" ::"v"(xq[q]), "v"(cq[q]));
  uint64_t ck[MPT];
  int64_t cf[MPT];
#pragma unroll
  for (int q = 0; q < MPT; ++q) {
    const int i = tid + q * MG_THREADS;
    const bool ok = i < n && vq[q] >= 0;
    const double c = cq[q];
    ck[q] = ok ? dkey(c == -INFINITY ? -INFINITY : ((double)xq[q] + c) + 0.0) : 0;  // -0 -> +0
    cf[q] = ok ? (int64_t)(b0 + bq[q]) * a.V + vq[q] : 0;
    if (i < n) {
      mk[0][i] = ck[q];
      mtok[i] = vq[q];
      if (bounded && i - bq[q] * k1 == k - 1) rowk[bq[q]] = ck[q];
    }
  }
  __syncthreads();
  // The rows' lists are ranked by (logit desc, token asc), so with c + x
  // monotone in x each is sorted by (score desc, flat asc) -- unless the
  // float64 sum rounds two logits of a row to one score, or the row's score
  // is -inf (all ties): then the order by flat is not the list order.  Check
  // every adjacent pair of a row; empty entries (key 0) are at the tail.
  // Meanwhile each row is ranked by its k-th key (ties: lower row first; one
  // wave per row, a ballot per 64 rows) and the MG_TOP_ROWS best are marked.
  const int T = min(MG_TOP_ROWS, nl);
  {
    bool bad = false;
#pragma unroll
    for (int q = 0; q < MPT; ++q) {
      const int i = tid + q * MG_THREADS;
      if (i + 1 < n && i + 1 != (bq[q] + 1) * k1) {
        const uint64_t kb = mk[0][i + 1];
        if (kb != 0 && (ck[q] < kb || (ck[q] == kb && vq[q] >= mtok[i + 1]))) bad = true;
      }
    }
    if (bad) unsorted = 1;
    if (bounded) {
      const int wave = tid >> 6, lane = tid & 63;
      for (int j = wave; j < nl; j += MG_THREADS / 64) {
        const uint64_t bj = rowk[j];
        int rank = 0;
        for (int h = 0; h < nl; h += 64) {
          const int jj = h + lane;
          const uint64_t bo = jj < nl ? rowk[jj] : 0;
          rank += __popcll(__ballot(jj < nl && (bo > bj || (bo == bj && jj < j))));
        }
        if (lane == 0) {
          is_top[j] = rank < T;
          if (rank < T) top_row[rank] = j;
        }
      }
    }
  }
  __syncthreads();
  const int64_t o = ((int64_t)r * a.ng + g) * k;
  if (bounded && unsorted == 0) {
    // (1) the top-k of the MG_TOP_ROWS rows' union by a tournament of sorted
    // lists: each level merges lists 2j and 2j+1, keeping the first k of each
    // merge; entry e of list l goes to (its position in l) + (the entries of
    // l's partner ordered before it, by binary search).  Ties of score go by
    // group position, which is flat order in sorted rows.  The lists of a
    // level have length L but the last (len_last).  Level 0 reads the top
    // rows where they lie (positions implicit); with one top row it copies
    // that row's first k.
    int nt = T, L = k1, len_last = k1, cur = 1;
    {
      const int L2 = min(2 * k1, k);
      for (int e = tid; e < T * k1; e += MG_THREADS) {
        const int t = div_small(e, k1, rk1), p = e - t * k1, src = top_row[t] * k1 + p;
        const uint64_t ke = mk[0][src];
        int cnt = 0;
        if ((t ^ 1) < T) {
          const int pb = top_row[t ^ 1] * k1;
          cnt = count_before(mk[0] + pb, nullptr, k1, ke, src - pb);
        }
        if (p + cnt < L2) {
          mk[1][(t >> 1) * L2 + p + cnt] = ke;
          mi[1][(t >> 1) * L2 + p + cnt] = (unsigned short)src;
        }
      }
      len_last = (nt & 1) ? min(k1, k) : L2;
      L = L2;
      nt = (nt + 1) >> 1;
      __syncthreads();
    }
    while (nt > 1) {
      const int E = (nt - 1) * L + len_last, L2 = min(2 * L, k);
      const float rL = 1.0f / (float)L;
      const uint64_t* sk = mk[cur];
      const unsigned short* si = mi[cur];
      uint64_t* dk = mk[cur ^ 1];
      unsigned short* di = mi[cur ^ 1];
      for (int e = tid; e < E; e += MG_THREADS) {
        const int l = div_small(e, L, rL), p = e - l * L, pl = l ^ 1;
        const uint64_t ke = sk[e];
        const int ie = si[e];
        int cnt = 0;
        if (pl < nt) {
          const int pb = pl * L;
          cnt = count_before(sk + pb, si + pb, pl == nt - 1 ? len_last : L, ke, ie);
        }
        if (p + cnt < L2) {
          dk[(l >> 1) * L2 + p + cnt] = ke;
          di[(l >> 1) * L2 + p + cnt] = (unsigned short)ie;
        }
      }
      len_last = (nt & 1) ? min(len_last, k) : min(L + len_last, k);
      L = L2;
      nt = (nt + 1) >> 1;
      cur ^= 1;
      __syncthreads();
    }
    const int fl = min(len_last, k);  // entries of the merged list F
    const uint64_t* fk = mk[cur];
    const unsigned short* fi = mi[cur];
    // (2) bound: F's k-th key is at most the group's k-th; the group's top-k
    // is F plus the other rows' entries at or above it (the extras)
    const uint64_t B = fl == k ? fk[k - 1] : 0;
    {
      int c = 0;
#pragma unroll
      for (int q = 0; q < MPT; ++q) c += ck[q] != 0 && ck[q] >= B && !is_top[bq[q]];
      if (c > 0) {
        int off = atomicAdd(&n_extra, c);
#pragma unroll
        for (int q = 0; q < MPT; ++q) {
          if (ck[q] != 0 && ck[q] >= B && !is_top[bq[q]]) {
            if (off < MG_MAX_EXTRA) {
              xk[off] = ck[q];
              xi[off] = tid + q * MG_THREADS;
            }
            ++off;
          }
        }
      }
    }
    __syncthreads();
    const int nx = n_extra;
    if (nx <= MG_MAX_EXTRA) {
      // (3) ranks in F + extras: an F entry's position plus the extras before
      // it; an extra's count of F entries before it (binary search) plus the
      // extras before it
      auto out = [&](int rank, uint64_t key, int pos) {
        if (rank < k) {
          a.part_key[o + rank] = key;
          if (key != 0) a.part_flat[o + rank] = (int64_t)(b0 + div_small(pos, k1, rk1)) * a.V + mtok[pos];
        }
      };
      if (tid < fl) {
        const uint64_t ke = fk[tid];
        const int ie = fi[tid];
        int rank = tid;
        for (int j = 0; j < nx; ++j) rank += xk[j] > ke || (xk[j] == ke && xi[j] < ie);
        out(rank, ke, ie);
      }
      if (tid >= MG_THREADS - 64 && tid - (MG_THREADS - 64) < nx) {
        const int x = tid - (MG_THREADS - 64);
        const uint64_t ke = xk[x];
        const int ie = xi[x];
        int rank = count_before(fk, fi, fl, ke, ie);
        for (int j = 0; j < nx; ++j) rank += xk[j] > ke || (xk[j] == ke && xi[j] < ie);
        out(rank, ke, ie);
      }
      for (int i = fl + nx + tid; i < k; i += MG_THREADS) a.part_key[o + i] = 0;
      return;
    }
  }
  // rows out of flat order, too many rows or extras: radix select of the
  // group's top-k, then ranking by counting
  bool take[MPT];
  int off;
  const int nsel = merge_select<MG_THREADS, MPT>(ck, cf, k, (int64_t)a.W * a.V, take, off, hist, itmp, sel, kred);
#pragma unroll
  for (int q = 0; q < MPT; ++q) {
    if (take[q]) {
      fkeys[off] = ck[q];
      ffl[off] = cf[q];
      ++off;
    }
  }
  __syncthreads();
  // the group's list, sorted by (score desc, flat asc); empty tail entries
  // have key 0, below every score.  Rank of entry i = entries ordered before
  // it: wave w counts over the entries [w*Q, (w+1)*Q) for every target, lane
  // l holding targets l, l + 64, ...; the partial counts meet in LDS.
  const int wave = tid >> 6, lane = tid & 63;
  for (int i = tid; i < nsel; i += MG_THREADS) hist[i] = 0;  // the histogram is dead: rank counters
  __syncthreads();
  {
    constexpr int NW = MG_THREADS / 64;
    const int Q = (nsel + NW - 1) / NW, q0 = wave * Q, q1 = min(nsel, q0 + Q);
    for (int t0 = 0; t0 < nsel; t0 += 64 * 4) {
      uint64_t kt[4];
      int64_t ft[4];
      int rk[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int i = t0 + lane + 64 * m;
        kt[m] = i < nsel ? fkeys[i] : 0;
        ft[m] = i < nsel ? ffl[i] : 0;
        rk[m] = 0;
      }
      for (int q = q0; q < q1; ++q) {
        const uint64_t kq = fkeys[q];
        const int64_t fq = ffl[q];
#pragma unroll
        for (int m = 0; m < 4; ++m) rk[m] += (kq > kt[m]) | ((kq == kt[m]) & (fq < ft[m]));
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int i = t0 + lane + 64 * m;
        if (i < nsel && rk[m]) atomicAdd(&hist[i], rk[m]);
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < nsel; i += MG_THREADS) {
    const int rank = hist[i];
    a.part_key[o + rank] = fkeys[i];
    a.part_flat[o + rank] = ffl[i];
  }
  for (int i = nsel + tid; i < a.k; i += MG_THREADS) a.part_key[o + i] = 0;
}

template <int NT, int MPT>  // threads, candidates per thread: ng * k <= MPT * NT
__global__ __launch_bounds__(NT) void prune_merge_final(PruneArgs a) {
  kernarg_lines<kernarg_line_count<PruneArgs>()>();
  __shared__ int hist[PR_BINS];
  __shared__ uint64_t fkeys[PR_MAXK];
  __shared__ int64_t ffl[PR_MAXK];
  __shared__ int itmp[NT / 64];
  __shared__ uint64_t kred[NT / 64][2];
  __shared__ int sel[3];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int k = a.k;
  const int n = a.ng * k;
  const uint64_t* pk = a.part_key + (int64_t)r * n;
  const int64_t* pf = a.part_flat + (int64_t)r * n;
  uint64_t ck[MPT];
  int64_t cf[MPT];
#pragma unroll
  for (int q = 0; q < MPT; ++q) {
    const int i = tid + q * NT;
    ck[q] = i < n ? pk[i] : 0;
    cf[q] = ck[q] != 0 ? pf[i] : 0;
  }
  bool take[MPT];
  int off;
  const int nsel = merge_select<NT, MPT>(ck, cf, k, (int64_t)a.W * a.V, take, off, hist, itmp, sel, kred);
#pragma unroll
  for (int q = 0; q < MPT; ++q) {
    if (take[q]) {
      fkeys[off] = ck[q];
      ffl[off] = cf[q];
      ++off;
    }
  }
  __syncthreads();
  // final order of the selected set: (score desc, flat asc)
  for (int i = tid; i < nsel; i += NT) {
    const uint64_t ki = fkeys[i];
    const int64_t fi = ffl[i];
    int rank = 0;
#pragma unroll 8
    for (int u = 0; u < nsel; ++u) {
      const uint64_t kq = fkeys[u];
      const int64_t fq = ffl[u];
      rank += (kq > ki) | ((kq == ki) & (fq < fi));
    }
    const int64_t o = (int64_t)r * k + rank;
    const int b = (int)(fi / a.V);
    a.parent[o] = b;
    a.token[o] = (int32_t)(fi - (int64_t)b * a.V);
    put_score(a, o, dval(ki));
  }
  for (int i = nsel + tid; i < k; i += NT) {
    const int64_t o = (int64_t)r * k + i;
    a.parent[o] = -1;
    a.token[o] = -1;
    put_score(a, o, -INFINITY);
  }
}

// Stage 2 over sorted lists: entry i of list g has rank i + (entries of the
// other lists ordered before it); those below k are written out at their
// rank.  Unfilled output slots (fewer than k candidates) get -1, -1, -inf.
constexpr int MG_LIST_MAX = 4096;  // ng * k staged in LDS
constexpr int MG_LIST_THREADS = 512;
constexpr int MG_LIST_MAXG = 16;   // lists searched side by side
__global__ __launch_bounds__(MG_LIST_THREADS) void prune_merge_lists(PruneArgs a) {
  kernarg_lines<kernarg_line_count<PruneArgs>()>();
  __shared__ uint64_t lk[MG_LIST_MAX];
  __shared__ int64_t lf[MG_LIST_MAX];
  __shared__ int cnt_s;
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int k = a.k, ng = a.ng;
  const int n = ng * k;
  const uint64_t* pk = a.part_key + (int64_t)r * n;
  const int64_t* pf = a.part_flat + (int64_t)r * n;
  if (tid == 0) cnt_s = 0;
  constexpr int PER = MG_LIST_MAX / MG_LIST_THREADS;
  uint64_t ek[PER];
  int64_t ef[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {  // all loads in flight together
    const int e = tid + u * MG_LIST_THREADS;
    ek[u] = e < n ? pk[e] : 0;
    ef[u] = e < n ? pf[e] : 0;
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = tid + u * MG_LIST_THREADS;
    if (e < n) {
      lk[e] = ek[u];
      lf[e] = ef[u];
    }
  }
  __syncthreads();
  int filled = 0;
#pragma unroll 1
  for (int u = 0; u < PER; ++u) {
    const int e = tid + u * MG_LIST_THREADS;
    if (__builtin_amdgcn_readfirstlane(e - tid) >= n) break;  // wave-uniform: no entries left
    const uint64_t ke = ek[u];
    const int64_t fe = ef[u];
    const int g = e / k;
    int rank = e - g * k;
    // per other list, the first position ordered after (ke, fe); the
    // searches run side by side, MG_LIST_MAXG lists at a time
    for (int h0 = 0; h0 < ng; h0 += MG_LIST_MAXG) {
      int lo[MG_LIST_MAXG], hi[MG_LIST_MAXG];
#pragma unroll
      for (int j = 0; j < MG_LIST_MAXG; ++j) {
        lo[j] = 0;
        hi[j] = h0 + j < ng && h0 + j != g ? k : 0;
      }
      for (int span = k; span > 0; span >>= 1) {
#pragma unroll
        for (int j = 0; j < MG_LIST_MAXG; ++j) {
          if (h0 + j < ng) {  // wave-uniform
            // branch-free step: both words are read whether or not the
            // search is still open (an open search reads inside its list)
            const bool open = lo[j] < hi[j];
            const int mid = (lo[j] + hi[j]) >> 1;
            const int idx = (h0 + j) * k + (open ? mid : 0);
            const uint64_t km = lk[idx];
            const int64_t fm = lf[idx];
            const bool before = (km > ke) | ((km == ke) & (fm < fe));
            lo[j] = (open & before) ? mid + 1 : lo[j];
            hi[j] = (open & !before) ? mid : hi[j];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < MG_LIST_MAXG; ++j) rank += lo[j];
    }
    if (e < n && ke != 0 && rank < k) {
      const int64_t o = (int64_t)r * k + rank;
      const int b = (int)(fe / a.V);
      a.parent[o] = b;
      a.token[o] = (int32_t)(fe - (int64_t)b * a.V);
      put_score(a, o, dval(ke));
      ++filled;
    }
  }
  if (filled) atomicAdd(&cnt_s, filled);
  __syncthreads();
  for (int i = cnt_s + tid; i < k; i += MG_LIST_THREADS) {
    const int64_t o = (int64_t)r * k + i;
    a.parent[o] = -1;
    a.token[o] = -1;
    put_score(a, o, -INFINITY);
  }
}

// merge layout: rows per stage-1 group and groups per request
void merge_groups(int W, int k1, int k, int& gr, int& ng) {
  gr = MG_GROUP_CAND / k1;
  if (gr < 1) gr = 1;
  if (gr > W) gr = W;
  ng = (W + gr - 1) / gr;
  (void)k;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace
}  // namespace gr

using namespace gr;

extern "C" size_t gr_beam_prune_workspace_size(int num_reqs, int beam_width, int vocab, int k) {
  if (num_reqs < 0 || beam_width < 1 || vocab < 1 || k < 1) return 0;
  const int k1 = k < vocab ? k : vocab;
  const size_t rows = (size_t)num_reqs * beam_width;
  int gr, ng;
  merge_groups(beam_width, k1, k, gr, ng);
  const size_t parts = (size_t)num_reqs * ng * k;
  return align256(rows * k1 * sizeof(float)) + align256(rows * k1 * sizeof(int32_t)) +
         align256(rows * sizeof(double)) + align256(parts * sizeof(uint64_t)) + align256(parts * sizeof(int64_t));
}

// The new beam's trie node: the child of its parent's node reached by its
// token (a selected candidate is always such a child).
__global__ void catalog_advance(PruneArgs a, int32_t* node_out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.R * a.k) return;
  const int r = i / a.k, p = a.parent[i], t = a.token[i];
  int node = -1;
  if (p >= 0 && p < a.W && t >= 0) {
    int c0, c1;
    catalog_range(a, r * a.W + p, c0, c1);
    const int e = catalog_find(a.child_token, c0, c1, t);
    node = e >= 0 ? a.child_node[e] : -1;
  }
  node_out[i] = node;
}

// a.cum / a.cum64, a.score / a.score64, a.eos_score / a.eos_score64 and the
// catalog fields are set by the caller.
static gr_status_t prune_launch(PruneArgs& a, const float* logits, int64_t logits_row_stride,
                                int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
                                int32_t* parent, int32_t* token, void* workspace, size_t workspace_bytes,
                                hipStream_t stream) {
  if (num_reqs < 0 || beam_width < 1 || vocab < 4 || vocab % 4 != 0 || k < 1 || k > PR_MAXK || k > vocab ||
      beam_width > PR_MAXW || logits_row_stride < vocab || logits_row_stride % 4 != 0)
    return GR_ERR_INVALID_ARG;
  if (num_reqs == 0) return GR_OK;
  if (!logits || !(a.cum || a.cum64) || !parent || !token || !(a.score || a.score64)) return GR_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(logits) & 15) != 0) return GR_ERR_INVALID_ARG;
  const size_t need = gr_beam_prune_workspace_size(num_reqs, beam_width, vocab, k);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return GR_ERR_WORKSPACE;
  const int k1 = k;
  const size_t rows = (size_t)num_reqs * beam_width;
  a.logits = logits;
  a.row_stride = logits_row_stride;
  a.R = num_reqs;
  a.W = beam_width;
  a.V = vocab;
  a.k1 = k1;
  a.k = k;
  a.eos = eos_token_id;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  a.cand_x = reinterpret_cast<float*>(ws);
  a.cand_v = reinterpret_cast<int32_t*>(ws + align256(rows * k1 * sizeof(float)));
  a.row_c = reinterpret_cast<double*>(ws + align256(rows * k1 * sizeof(float)) +
                                      align256(rows * k1 * sizeof(int32_t)));
  a.parent = parent;
  a.token = token;
  merge_groups(beam_width, k1, k, a.gr, a.ng);
  const size_t parts = (size_t)num_reqs * a.ng * k;
  uint8_t* part_base = ws + align256(rows * k1 * sizeof(float)) + align256(rows * k1 * sizeof(int32_t)) +
                       align256(rows * sizeof(double));
  a.part_key = reinterpret_cast<uint64_t*>(part_base);
  a.part_flat = reinterpret_cast<int64_t*>(part_base + align256(parts * sizeof(uint64_t)));
  const bool cat = a.beam_node != nullptr;
  if (vocab == PR_CHUNK * PR_REG_CHUNKS) {
    if (cat) hipLaunchKernelGGL((prune_rows<PR_REG_CHUNKS, true, true>), dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
    else hipLaunchKernelGGL((prune_rows<PR_REG_CHUNKS, false, true>), dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
  } else if (vocab <= PR_CHUNK * PR_REG_CHUNKS) {
    if (cat) hipLaunchKernelGGL((prune_rows<PR_REG_CHUNKS, true>), dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
    else hipLaunchKernelGGL((prune_rows<PR_REG_CHUNKS, false>), dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
  } else {
    if (cat) hipLaunchKernelGGL((prune_rows<0, true>), dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
    else hipLaunchKernelGGL((prune_rows<0, false>), dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
  }
  gr_status_t st = launch_status();
  if (st != GR_OK) return st;
  const size_t per_req = (size_t)a.ng * k;  // stage-2 candidates per request
  if (per_req > (size_t)MG_REG * MG_THREADS) {
    // very wide requests: one pass over all candidates, re-read from memory
    hipLaunchKernelGGL(prune_merge<0>, dim3((unsigned)num_reqs), dim3(MG_THREADS), 0, stream, a);
    return launch_status();
  }
  hipLaunchKernelGGL(prune_merge_part, dim3((unsigned)(num_reqs * a.ng)), dim3(MG_THREADS), 0, stream, a);
  st = launch_status();
  if (st != GR_OK) return st;
  if (per_req <= MG_LIST_MAX)
    hipLaunchKernelGGL(prune_merge_lists, dim3((unsigned)num_reqs), dim3(MG_LIST_THREADS), 0, stream, a);
  else if (per_req <= 4 * MG_THREADS)
    hipLaunchKernelGGL((prune_merge_final<MG_THREADS, 4>), dim3((unsigned)num_reqs), dim3(MG_THREADS), 0, stream, a);
  else
    hipLaunchKernelGGL((prune_merge_final<MG_THREADS, MG_REG>), dim3((unsigned)num_reqs), dim3(MG_THREADS), 0, stream, a);
  return launch_status();
}

// The catalog fields of the arguments; false on an inconsistent trie.
static bool set_catalog(PruneArgs& a, const int32_t* beam_node, const int32_t* node_start,
                        const int32_t* child_token, const int32_t* child_node, int num_nodes, int num_edges,
                        const int32_t* node_out) {
  if (num_nodes < 1 || num_edges < 0 || !beam_node || !node_start || !node_out ||
      (num_edges > 0 && (!child_token || !child_node)))
    return false;
  a.beam_node = beam_node;
  a.node_start = node_start;
  a.child_token = child_token;
  a.child_node = child_node;
  a.num_nodes = num_nodes;
  a.num_edges = num_edges;
  return true;
}

static gr_status_t catalog_advance_launch(PruneArgs& a, int32_t* node_out, hipStream_t stream) {
  const int n = a.R * a.k;
  if (n == 0) return GR_OK;
  hipLaunchKernelGGL(catalog_advance, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, node_out);
  return launch_status();
}

extern "C" gr_status_t gr_beam_prune_topk(const float* logits, int64_t logits_row_stride, const float* cum,
                                          int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
                                          int32_t* parent, int32_t* token, float* score, float* eos_score,
                                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
  PruneArgs a = {};
  a.cum = cum;
  a.score = score;
  a.eos_score = eos_score;
  return prune_launch(a, logits, logits_row_stride, num_reqs, beam_width, vocab, k, eos_token_id, parent, token,
                      workspace, workspace_bytes, stream);
}

extern "C" gr_status_t gr_beam_prune_topk_catalog(
    const float* logits, int64_t logits_row_stride, const float* cum,
    int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
    const int32_t* beam_node, const int32_t* node_start, const int32_t* child_token,
    const int32_t* child_node, int num_nodes, int num_edges,
    int32_t* parent, int32_t* token, float* score, float* eos_score, int32_t* node_out,
    void* workspace, size_t workspace_bytes, int32_t* dev_status, hipStream_t stream) {
  PruneArgs a = {};
  if (!set_catalog(a, beam_node, node_start, child_token, child_node, num_nodes, num_edges, node_out))
    return GR_ERR_INVALID_ARG;
  a.cum = cum;
  a.score = score;
  a.eos_score = eos_score;
  a.dev_status = dev_status;
  gr_status_t st = prune_launch(a, logits, logits_row_stride, num_reqs, beam_width, vocab, k, eos_token_id,
                                parent, token, workspace, workspace_bytes, stream);
  if (st != GR_OK || num_reqs == 0) return st;
  return catalog_advance_launch(a, node_out, stream);
}

extern "C" gr_status_t gr_beam_prune_topk_f64(
    const float* logits, int64_t logits_row_stride, const double* cum,
    int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
    const int32_t* beam_node, const int32_t* node_start, const int32_t* child_token,
    const int32_t* child_node, int num_nodes, int num_edges,
    int32_t* parent, int32_t* token, double* score, double* eos_score, int32_t* node_out,
    int32_t* cand_token, float* cand_logprob,
    void* workspace, size_t workspace_bytes, int32_t* dev_status, hipStream_t stream) {
  PruneArgs a = {};
  if (!cand_token != !cand_logprob) return GR_ERR_INVALID_ARG;
  a.cand_token = cand_token;
  a.cand_logprob = cand_logprob;
  if (beam_node &&
      !set_catalog(a, beam_node, node_start, child_token, child_node, num_nodes, num_edges, node_out))
    return GR_ERR_INVALID_ARG;
  a.cum64 = cum;
  a.score64 = score;
  a.eos_score64 = eos_score;
  a.dev_status = dev_status;
  gr_status_t st = prune_launch(a, logits, logits_row_stride, num_reqs, beam_width, vocab, k, eos_token_id,
                                parent, token, workspace, workspace_bytes, stream);
  if (st != GR_OK || num_reqs == 0 || !beam_node) return st;
  return catalog_advance_launch(a, node_out, stream);
}

// ---- the entry point that allocates nothing -----------------------------
// Scratch of gr_beam_prune_topk_noalloc: the workspace of gr_beam_prune_topk
// in a static device array.  Each device holds its own copy until the
// process ends.  In host code `scratch` names a host-side stand-in, never the
// device memory: the device address comes from hipGetSymbolAddress, taken
// once per device with that device current, and only that address is passed
// to kernels.
static __device__ __attribute__((aligned(256))) uint8_t scratch[GR_PRUNE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// The current device's address of `scratch` (looked up on its first use).
gr_status_t scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return GR_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return GR_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return GR_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GR_OK;
}
}  // namespace

extern "C" gr_status_t gr_beam_prune_topk_noalloc(const float* logits, int64_t logits_row_stride,
                                                  const float* cum, int num_reqs, int beam_width, int vocab,
                                                  int k, int eos_token_id, int32_t* parent, int32_t* token,
                                                  float* score, float* eos_score, hipStream_t stream) {
  if (num_reqs < 0 || beam_width < 1 || vocab < 1 || k < 1) return GR_ERR_INVALID_ARG;
  if (gr_beam_prune_workspace_size(num_reqs, beam_width, vocab, k) > GR_PRUNE_SCRATCH_BYTES)
    return GR_ERR_WORKSPACE;
  void* ws = nullptr;
  const gr_status_t st = scratch_address(&ws);
  if (st != GR_OK) return st;
  return gr_beam_prune_topk(logits, logits_row_stride, cum, num_reqs, beam_width, vocab, k, eos_token_id, parent,
                            token, score, eos_score, ws, GR_PRUNE_SCRATCH_BYTES, stream);
}
