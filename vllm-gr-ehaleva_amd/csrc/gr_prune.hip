// Fused beam pruning for gfx950: log_softmax + cumulative logprob + top-k
// over beams x vocab (the sampler's logprobs=W top-K plus the host pruning of
// vllm_gr/entrypoints/openai/serving_engine.py:457-592, as two launches).
//
// Kernel 1 (prune_rows): one workgroup of 256 threads per beam row.  Reads
// the row once (float4, rows up to 8192 held in registers), computes the row
// max, the fixed-order fp32 exp-sum, the float64 LSE, and the row's top-k by
// (logit desc, token asc):
//   * the k-th largest of the 256 per-thread maxima bounds the k-th largest
//     element from below, so only elements >= that bound survive (about
//     k * 1.4 for random data); survivors are ranked exactly by counting;
//   * rows with too many survivors (heavy ties) fall back to an exact
//     bisection over the order-preserving integer image of the logits and
//     take tied elements in ascending token order.
// Kernel 2 (prune_merge): one workgroup per request.  The per-row lists are
// sorted, so "how many candidates score >= t" is one binary search per row.
// A bisection over the order-preserving integer image of float64 scores
// narrows [lo, hi) until few candidates remain between, which are ranked
// exactly; exact ties are resolved by lowest flat index (rows in ascending
// beam order, tokens ascending inside a row).
//
// This file is compiled with -ffp-contract=off: every float operation below
// is a single IEEE operation so the CPU restatement reproduces the scores
// bit for bit.
#include "gr_common.h"

namespace gr {
namespace {

constexpr int PR_THREADS = 256;
constexpr int PR_VEC = 4;
constexpr int PR_CHUNK = PR_THREADS * PR_VEC;  // elements per chunk
constexpr int PR_REG_CHUNKS = 8;               // rows of up to 8192 stay in registers
constexpr int PR_CAP = 1024;                   // survivor capacity of the fast path
constexpr int PR_MAXK = 1024;
constexpr int PR_MAXW = 1024;
constexpr int PR_CAP2 = 512;                   // merge: candidates ranked exactly at the end

typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));

// ---- bit-exact numerics ------------------------------------------------------
// exp2 of t <= 0: Taylor series of e^(f ln2) (degree 7, Horner with fma) on the
// fractional part f = t - rint(t), scaled by 2^rint(t).
__device__ inline float exp2_neg(float t) {
  if (!(t >= -125.0f)) return 0.0f;
  const float k = __builtin_rintf(t);
  const float f = t - k;
  float p = 0x1.ffcbfcp-17f;
  p = __builtin_fmaf(p, f, 0x1.430912p-13f);
  p = __builtin_fmaf(p, f, 0x1.5d87fep-10f);
  p = __builtin_fmaf(p, f, 0x1.3b2ab6p-7f);
  p = __builtin_fmaf(p, f, 0x1.c6b08ep-5f);
  p = __builtin_fmaf(p, f, 0x1.ebfbe0p-3f);
  p = __builtin_fmaf(p, f, 0x1.62e430p-1f);
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
__device__ inline uint64_t dkey(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  return (u >> 63) ? ~u : (u | (1ull << 63));
}
__device__ inline double dval(uint64_t k) {
  const uint64_t u = (k >> 63) ? (k & ~(1ull << 63)) : ~k;
  return __builtin_bit_cast(double, u);
}

struct PruneArgs {
  const float* logits;
  int64_t row_stride;
  const float* cum;
  int R, W, V, k1, k, eos;
  float* cand_x;    // [R*W, k1] row top-k logits, sorted; EOS removed, tail padded
  int32_t* cand_v;  // [R*W, k1] tokens (-1 = empty)
  double* row_c;    // [R*W]     cum - lse
  int32_t* parent;
  int32_t* token;
  float* score;
  float* eos_score;
};

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ inline int wave_sum_i(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// block-wide exclusive scan of one int per thread; returns the total
__device__ int block_scan(int v, int& excl, int* tmp) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < PR_THREADS / 64; ++w) {
    base += (w < wave) ? tmp[w] : 0;
    total += tmp[w];
  }
  excl = base + incl - v;
  __syncthreads();
  return total;
}

__device__ int block_sum(int v, int* tmp) {
  int e;
  return block_scan(v, e, tmp);
}

template <int MAXC>  // MAXC > 0: row held in registers (<= MAXC chunks); 0: re-read from memory
__global__ __launch_bounds__(PR_THREADS) void prune_rows(PruneArgs a) {
  __shared__ float sx[PR_CAP];
  __shared__ int sv[PR_CAP];
  __shared__ float ox[PR_MAXK];
  __shared__ int ov[PR_MAXK];
  __shared__ float tmx[PR_THREADS];
  __shared__ int has[PR_THREADS];
  __shared__ float wred[PR_THREADS / 64];
  __shared__ int itmp[PR_THREADS / 64];
  __shared__ float t0_s;
  __shared__ int eos_pos;

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
      f32x4_t v = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      if (c < nch && idx < V) v = *reinterpret_cast<const f32x4_t*>(xg + idx);
#pragma unroll
      for (int j = 0; j < PR_VEC; ++j) xr[c][j] = v[j] + 0.0f;  // -0 -> +0
    }
  }
  auto valid = [&](int c) { return c * PR_CHUNK + PR_VEC * tid < V; };
  auto get = [&](int c, int j) -> float {
    if constexpr (MAXC > 0) return xr[c][j];
    else return xg[c * PR_CHUNK + PR_VEC * tid + j] + 0.0f;
  };
#define PR_FOR_CHUNKS(c) \
  _Pragma("unroll") for (int c = 0; c < (MAXC > 0 ? MAXC : nch); ++c) if (c < nch)

  // ---- row max ----
  float tm = -INFINITY;
  PR_FOR_CHUNKS(c) {
    if (valid(c)) {
#pragma unroll
      for (int j = 0; j < PR_VEC; ++j) tm = fmaxf(tm, get(c, j));
    }
  }
  const float wm = wave_max(tm);
  if (lane == 0) wred[wave] = wm;
  tmx[tid] = tm;
  has[tid] = valid(0) ? 1 : 0;
  __syncthreads();
  float m = wred[0];
#pragma unroll
  for (int w = 1; w < PR_THREADS / 64; ++w) m = fmaxf(m, wred[w]);
  __syncthreads();

  // ---- fixed-order exp-sum: thread partial in element order, xor butterfly, waves pairwise ----
  double c_row = -INFINITY;
  if (m != -INFINITY) {
    float acc = 0.0f;
    PR_FOR_CHUNKS(c) {
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          const float d = get(c, j) - m;
          const float t = d * 0x1.715476p+0f;
          acc = acc + exp2_neg(t);
        }
      }
    }
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) acc = acc + __shfl_xor(acc, msk, 64);
    if (lane == 0) wred[wave] = acc;
    __syncthreads();
    const float S = (wred[0] + wred[1]) + (wred[2] + wred[3]);
    const double lse = (double)m + log_f64((double)S);
    c_row = (double)a.cum[row] - lse;
  }

  // ---- stage 1: row top-k1 by (logit desc, token asc) ----
  int nthr = 0;  // threads owning elements
  for (int u = 0; u < PR_THREADS; ++u) nthr += has[u];
  bool fast = k1 <= nthr;
  if (fast) {
    if (has[tid]) {
      int rank = 0;
      for (int u = 0; u < PR_THREADS; ++u) {
        const float y = tmx[u];
        rank += has[u] && (y > tm || (y == tm && u < tid));
      }
      if (rank == k1 - 1) t0_s = tm;
    }
    __syncthreads();
    const float t0 = t0_s;
    int cnt = 0;
    PR_FOR_CHUNKS(c) {
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) cnt += get(c, j) >= t0;
      }
    }
    int off;
    const int total = block_scan(cnt, off, itmp);
    fast = total <= PR_CAP;
    if (fast) {
      PR_FOR_CHUNKS(c) {
        if (valid(c)) {
#pragma unroll
          for (int j = 0; j < PR_VEC; ++j) {
            const float y = get(c, j);
            if (y >= t0) {
              sx[off] = y;
              sv[off] = c * PR_CHUNK + PR_VEC * tid + j;
              ++off;
            }
          }
        }
      }
      __syncthreads();
      for (int i = tid; i < total; i += PR_THREADS) {
        const float xi = sx[i];
        const int vi = sv[i];
        int rank = 0;
        for (int q = 0; q < total; ++q) {
          const float y = sx[q];
          rank += (y > xi) || (y == xi && sv[q] < vi);
        }
        if (rank < k1) {
          ox[rank] = xi;
          ov[rank] = vi;
        }
      }
    }
  }
  if (!fast) {
    // exact fallback: largest key T with count(key >= T) >= k1
    uint64_t lo = 0, hi = 1ull << 32;
    while (hi - lo > 1) {
      const uint64_t mid = lo + (hi - lo) / 2;
      int cnt = 0;
      PR_FOR_CHUNKS(c) {
        if (valid(c)) {
#pragma unroll
          for (int j = 0; j < PR_VEC; ++j) cnt += (uint64_t)fkey(get(c, j)) >= mid;
        }
      }
      const int tot = block_sum(cnt, itmp);
      if (tot >= k1) lo = mid; else hi = mid;
    }
    const uint32_t T = (uint32_t)lo;
    int gt = 0;
    PR_FOR_CHUNKS(c) {
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) gt += fkey(get(c, j)) > T;
      }
    }
    int off;
    const int ngt = block_scan(gt, off, itmp);
    PR_FOR_CHUNKS(c) {
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          const float y = get(c, j);
          if (fkey(y) > T) {
            sx[off] = y;
            sv[off] = c * PR_CHUNK + PR_VEC * tid + j;
            ++off;
          }
        }
      }
    }
    // ties at T in ascending token order until k1 are taken
    int taken = ngt;
    PR_FOR_CHUNKS(c) {
      int tc = 0;
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) tc += fkey(get(c, j)) == T;
      }
      int toff;
      const int ctot = block_scan(tc, toff, itmp);
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          if (fkey(get(c, j)) == T) {
            const int pos = taken + toff;
            if (pos < k1) {
              sx[pos] = get(c, j);
              sv[pos] = c * PR_CHUNK + PR_VEC * tid + j;
            }
            ++toff;
          }
        }
      }
      taken += ctot;
      if (taken >= k1) break;
    }
    __syncthreads();
    for (int i = tid; i < k1; i += PR_THREADS) {
      const float xi = sx[i];
      const int vi = sv[i];
      int rank = 0;
      for (int q = 0; q < k1; ++q) {
        const float y = sx[q];
        rank += (y > xi) || (y == xi && sv[q] < vi);
      }
      ox[rank] = xi;
      ov[rank] = vi;
    }
  }
#undef PR_FOR_CHUNKS
  if (tid == 0) eos_pos = -1;
  __syncthreads();
  if (a.eos >= 0)
    for (int i = tid; i < k1; i += PR_THREADS)
      if (ov[i] == a.eos) eos_pos = i;
  __syncthreads();
  const int e = eos_pos;
  float* cx = a.cand_x + (int64_t)row * k1;
  int32_t* cv = a.cand_v + (int64_t)row * k1;
  for (int i = tid; i < k1; i += PR_THREADS) {
    const int src = (e >= 0 && i >= e) ? i + 1 : i;
    cx[i] = src < k1 ? ox[src] : -INFINITY;
    cv[i] = src < k1 ? ov[src] : -1;
  }
  if (tid == 0) {
    a.row_c[row] = c_row;
    if (a.eos_score) {
      float es = -INFINITY;
      if (e >= 0 && c_row != -INFINITY) es = (float)((double)ox[e] + c_row);
      a.eos_score[row] = es;
    }
  }
}

// ---- kernel 2: per-request merge of the sorted row lists --------------------
struct MergeCtx {
  const float* xs;  // [W, k1] (LDS copy or workspace)
  const int32_t* vs;
  const double* cs;  // [W]
  int k1;
  int64_t V;
};

__device__ inline double cand_score(const MergeCtx& m, int b, int j) {
  const int v = m.vs[b * m.k1 + j];
  if (v < 0) return -INFINITY;
  const double c = m.cs[b];
  return c == -INFINITY ? -INFINITY : (double)m.xs[b * m.k1 + j] + c;
}
__device__ inline int64_t cand_flat(const MergeCtx& m, int b, int j) {
  const int v = m.vs[b * m.k1 + j];
  return v < 0 ? INT64_MAX : (int64_t)b * m.V + v;
}
// number of candidates of row b (first nvalid entries) with score >= t
__device__ inline int count_ge(const MergeCtx& m, int b, int nvalid, double t) {
  int lo = 0, hi = nvalid;  // first index with score < t
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (cand_score(m, b, mid) >= t) lo = mid + 1; else hi = mid;
  }
  return lo;
}

template <bool LDS_LISTS>
__global__ __launch_bounds__(PR_THREADS) void prune_merge(PruneArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  __shared__ double cs[PR_MAXW];
  __shared__ int nval[PR_MAXW], ge_lo[PR_MAXW], ge_hi[PR_MAXW];
  __shared__ int between[PR_CAP2];
  __shared__ int fin[PR_MAXK];
  __shared__ int itmp[PR_THREADS / 64];
  __shared__ double dred[PR_THREADS / 64][2];

  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int W = a.W, k1 = a.k1, k = a.k;
  // each thread owns a contiguous row range, so thread order is beam order
  const int rpt = (W + PR_THREADS - 1) / PR_THREADS;
  const int rb0 = min(W, tid * rpt), rb1 = min(W, rb0 + rpt);
  const int64_t rbase = (int64_t)r * W;
  MergeCtx m;
  m.k1 = k1;
  m.V = a.V;
  m.cs = cs;
  if constexpr (LDS_LISTS) {
    float* xs = reinterpret_cast<float*>(dyn);
    int32_t* vs = reinterpret_cast<int32_t*>(dyn + sizeof(float) * (size_t)W * k1);
    for (int i = tid; i < W * k1; i += PR_THREADS) {
      xs[i] = a.cand_x[rbase * k1 + i];
      vs[i] = a.cand_v[rbase * k1 + i];
    }
    m.xs = xs;
    m.vs = vs;
  } else {
    m.xs = a.cand_x + rbase * k1;
    m.vs = a.cand_v + rbase * k1;
  }
  for (int b = tid; b < W; b += PR_THREADS) cs[b] = a.row_c[rbase + b];  // any order
  __syncthreads();
  // per-row valid counts, global score range
  double smin = INFINITY, smax = -INFINITY;
  int nv_loc = 0;
  for (int b = rb0; b < rb1; ++b) {
    int nv = 0;
    {
      int lo = 0, hi = k1;  // valid entries form a prefix
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (m.vs[b * k1 + mid] >= 0) lo = mid + 1; else hi = mid;
      }
      nv = lo;
    }
    nval[b] = nv;
    nv_loc += nv;
    if (nv > 0) {
      smax = fmax(smax, cand_score(m, b, 0));
      smin = fmin(smin, cand_score(m, b, nv - 1));
    }
  }
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) {
    smin = fmin(smin, __shfl_xor(smin, msk, 64));
    smax = fmax(smax, __shfl_xor(smax, msk, 64));
  }
  if (lane == 0) {
    dred[wave][0] = smin;
    dred[wave][1] = smax;
  }
  const int M = block_sum(nv_loc, itmp);  // includes a barrier after dred writes
  for (int w = 0; w < PR_THREADS / 64; ++w) {
    smin = fmin(smin, dred[w][0]);
    smax = fmax(smax, dred[w][1]);
  }

  int n_above = 0;  // candidates certainly selected (score >= value(hi))
  int q = 0;        // how many to take from the "between" range
  bool ties = false;
  if (M <= k) {
    for (int b = rb0; b < rb1; ++b) {
      ge_hi[b] = nval[b];
      ge_lo[b] = nval[b];
    }
    n_above = M;
  } else {
    uint64_t lo = dkey(smin), hi = dkey(smax) + 1;
    int cnt_lo = M, cnt_hi = 0;
    while (hi - lo > 1 && cnt_lo - cnt_hi > PR_CAP2) {
      const uint64_t mid = lo + (hi - lo) / 2;
      const double t = dval(mid);
      int c = 0;
      for (int b = rb0; b < rb1; ++b) c += count_ge(m, b, nval[b], t);
      const int tot = block_sum(c, itmp);
      if (tot >= k) {
        lo = mid;
        cnt_lo = tot;
      } else {
        hi = mid;
        cnt_hi = tot;
      }
    }
    const double tlo = dval(lo), thi = dval(hi);
    for (int b = rb0; b < rb1; ++b) {
      ge_lo[b] = count_ge(m, b, nval[b], tlo);
      ge_hi[b] = count_ge(m, b, nval[b], thi);
    }
    n_above = cnt_hi;
    q = k - cnt_hi;
    ties = cnt_lo - cnt_hi > PR_CAP2;  // hi == lo + 1: all "between" share one score
  }
  __syncthreads();
  // gather: above-hi candidates and the between set (as b * k1 + j)
  {
    int na = 0, nb = 0;
    for (int b = rb0; b < rb1; ++b) {
      na += ge_hi[b];
      nb += ge_lo[b] - ge_hi[b];
    }
    int oa, ob;
    block_scan(na, oa, itmp);
    const int nbt = block_scan(nb, ob, itmp);
    (void)nbt;
    for (int b = rb0; b < rb1; ++b) {
      for (int j = 0; j < ge_hi[b]; ++j) fin[oa++] = b * k1 + j;
      if (!ties) {
        for (int j = ge_hi[b]; j < ge_lo[b]; ++j) between[ob++] = b * k1 + j;
      }
    }
    if (ties) {
      // exact ties at one score: lowest flat index = ascending beam, then token
      int tie = 0;
      for (int b = rb0; b < rb1; ++b) tie += ge_lo[b] - ge_hi[b];
      int toff;
      block_scan(tie, toff, itmp);
      for (int b = rb0; b < rb1; ++b) {
        for (int j = ge_hi[b]; j < ge_lo[b]; ++j) {
          if (toff < q) fin[n_above + toff] = b * k1 + j;
          ++toff;
        }
      }
    }
  }
  __syncthreads();
  if (!ties && M > k) {
    const int nb = [&] {
      int s = 0;
      for (int b = 0; b < W; ++b) s += ge_lo[b] - ge_hi[b];
      return s;
    }();
    for (int i = tid; i < nb; i += PR_THREADS) {
      const int bi = between[i] / k1, ji = between[i] % k1;
      const double si = cand_score(m, bi, ji);
      const int64_t fi = cand_flat(m, bi, ji);
      int rank = 0;
      for (int u = 0; u < nb; ++u) {
        const int bu = between[u] / k1, ju = between[u] % k1;
        const double su = cand_score(m, bu, ju);
        rank += (su > si) || (su == si && cand_flat(m, bu, ju) < fi);
      }
      if (rank < q) fin[n_above + rank] = between[i];
    }
    __syncthreads();
  }
  // final order of the selected set: (score desc, flat asc)
  const int nsel = M < k ? M : k;
  for (int i = tid; i < k; i += PR_THREADS) {
    const int64_t o = (int64_t)r * k;
    if (i >= nsel) {
      a.parent[o + i] = -1;
      a.token[o + i] = -1;
      a.score[o + i] = -INFINITY;
    }
  }
  for (int i = tid; i < nsel; i += PR_THREADS) {
    const int bi = fin[i] / k1, ji = fin[i] % k1;
    const double si = cand_score(m, bi, ji);
    const int64_t fi = cand_flat(m, bi, ji);
    int rank = 0;
    for (int u = 0; u < nsel; ++u) {
      const int bu = fin[u] / k1, ju = fin[u] % k1;
      const double su = cand_score(m, bu, ju);
      rank += (su > si) || (su == si && cand_flat(m, bu, ju) < fi);
    }
    const int64_t o = (int64_t)r * k + rank;
    a.parent[o] = bi;
    a.token[o] = m.vs[bi * k1 + ji];
    a.score[o] = (float)si;
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace
}  // namespace gr

using namespace gr;

extern "C" size_t gr_beam_prune_workspace_size(int num_reqs, int beam_width, int vocab, int k) {
  if (num_reqs < 0 || beam_width < 1 || vocab < 1 || k < 1) return 0;
  const int k1 = k < vocab ? k : vocab;
  const size_t rows = (size_t)num_reqs * beam_width;
  return align256(rows * k1 * sizeof(float)) + align256(rows * k1 * sizeof(int32_t)) +
         align256(rows * sizeof(double));
}

extern "C" gr_status_t gr_beam_prune_topk(const float* logits, int64_t logits_row_stride, const float* cum,
                                          int num_reqs, int beam_width, int vocab, int k, int eos_token_id,
                                          int32_t* parent, int32_t* token, float* score, float* eos_score,
                                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (num_reqs < 0 || beam_width < 1 || vocab < 4 || vocab % 4 != 0 || k < 1 || k > PR_MAXK || k > vocab ||
      beam_width > PR_MAXW || logits_row_stride < vocab || logits_row_stride % 4 != 0)
    return GR_ERR_INVALID_ARG;
  if (num_reqs == 0) return GR_OK;
  if (!logits || !cum || !parent || !token || !score) return GR_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(logits) & 15) != 0) return GR_ERR_INVALID_ARG;
  const size_t need = gr_beam_prune_workspace_size(num_reqs, beam_width, vocab, k);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return GR_ERR_WORKSPACE;
  const int k1 = k;
  const size_t rows = (size_t)num_reqs * beam_width;
  PruneArgs a;
  a.logits = logits;
  a.row_stride = logits_row_stride;
  a.cum = cum;
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
  a.score = score;
  a.eos_score = eos_score;
  if (vocab <= PR_CHUNK * PR_REG_CHUNKS)
    hipLaunchKernelGGL(prune_rows<PR_REG_CHUNKS>, dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
  else
    hipLaunchKernelGGL(prune_rows<0>, dim3((unsigned)rows), dim3(PR_THREADS), 0, stream, a);
  gr_status_t st = launch_status();
  if (st != GR_OK) return st;
  const size_t list_bytes = (size_t)beam_width * k1 * 8;
  if (list_bytes <= 128 * 1024) {
    static bool attr_set = false;
    if (!attr_set) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(prune_merge<true>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
      attr_set = true;
    }
    hipLaunchKernelGGL(prune_merge<true>, dim3((unsigned)num_reqs), dim3(PR_THREADS), list_bytes, stream, a);
  } else {
    hipLaunchKernelGGL(prune_merge<false>, dim3((unsigned)num_reqs), dim3(PR_THREADS), 0, stream, a);
  }
  return launch_status();
}
