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

namespace gr {
namespace {

constexpr int PR_THREADS = 256;
constexpr int PR_VEC = 4;
constexpr int PR_CHUNK = PR_THREADS * PR_VEC;  // elements per chunk
constexpr int PR_REG_CHUNKS = 8;               // rows of up to 8192 stay in registers
constexpr int PR_MAXK = 1024;
constexpr int PR_MAXW = 1024;
constexpr int PR_BINS = 2048;                  // radix-select histogram bins (11-bit digits)
constexpr int MG_THREADS = 1024;               // merge workgroup

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

// block-wide exclusive scan of one int per thread (NT threads); returns the total
template <int NT = PR_THREADS>
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
  for (int w = 0; w < NT / 64; ++w) {
    base += (w < wave) ? tmp[w] : 0;
    total += tmp[w];
  }
  excl = base + incl - v;
  __syncthreads();
  return total;
}

// Radix select: the need-th largest (1-based) of the unsigned KBITS-bit keys
// that for_each(f) hands to f (each thread its own keys; at least `need` keys
// in total).  Digits of 11 bits from the top; a pass histograms the keys that
// match the digits fixed so far and walks the bins from the top.  Stops early
// once the bin holding the need-th key holds exactly the keys still needed.
// Result: keys with (key & mask) > prefix are above the boundary (k_need - need
// of them); the `need` remaining come from the eq keys with (key & mask) ==
// prefix -- all of them when eq == need, else (mask all ones) a choice among
// equal keys left to the caller.
template <typename K>
struct RadixSel {
  K prefix, mask;
  int need, eq;
};

template <int NT, typename K, int KBITS, typename ForEach>
__device__ RadixSel<K> radix_select(ForEach for_each, int need, int* hist, int* itmp, int* sel) {
  const int tid = threadIdx.x;
  RadixSel<K> rs{0, 0, need, 0};
  constexpr int NP = (KBITS + 10) / 11;
  constexpr int BPT = PR_BINS / NT;  // bins owned per thread in the top-down walk
#pragma unroll 1
  for (int pass = 0; pass < NP; ++pass) {
    const int hi_bit = KBITS - 11 * pass;
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

template <int MAXC>  // MAXC > 0: row held in registers (<= MAXC chunks); 0: re-read from memory
__global__ __launch_bounds__(PR_THREADS) void prune_rows(PruneArgs a) {
  __shared__ float sx[PR_MAXK];
  __shared__ int sv[PR_MAXK];
  __shared__ float ox[PR_MAXK];
  __shared__ int ov[PR_MAXK];
  __shared__ int hist[PR_BINS];
  __shared__ float wred[PR_THREADS / 64];
  __shared__ int itmp[PR_THREADS / 64];
  __shared__ int sel[3];
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

  // ---- stage 1: row top-k1 by (logit desc, token asc), radix select ----
  const RadixSel<uint32_t> rs = radix_select<PR_THREADS, uint32_t, 32>(
      [&](auto&& f) {
        PR_FOR_CHUNKS(c) {
          if (valid(c)) {
#pragma unroll
            for (int j = 0; j < PR_VEC; ++j) f(fkey(get(c, j)));
          }
        }
      },
      k1, hist, itmp, sel);
  const uint32_t T = rs.prefix, Tm = rs.mask;
  const int need = rs.need, eq_cnt = rs.eq;
  // keys above the boundary: k1 - need of them, all taken; keys at it: all
  // when eq_cnt == need, else the first `need` by token
  {
    int gt = 0, eq = 0;
    PR_FOR_CHUNKS(c) {
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          const uint32_t u = fkey(get(c, j)) & Tm;
          gt += u > T;
          eq += u == T;
        }
      }
    }
    int off;
    const int ngt = block_scan(gt, off, itmp);
    PR_FOR_CHUNKS(c) {
      if (valid(c)) {
#pragma unroll
        for (int j = 0; j < PR_VEC; ++j) {
          const float y = get(c, j);
          if ((fkey(y) & Tm) > T) {
            sx[off] = y;
            sv[off] = c * PR_CHUNK + PR_VEC * tid + j;
            ++off;
          }
        }
      }
    }
    if (eq_cnt == need) {  // every key equal to T is taken: order is irrelevant here
      int eoff;
      block_scan(eq, eoff, itmp);
      PR_FOR_CHUNKS(c) {
        if (valid(c)) {
#pragma unroll
          for (int j = 0; j < PR_VEC; ++j) {
            const float y = get(c, j);
            if ((fkey(y) & Tm) == T) {
              sx[ngt + eoff] = y;
              sv[ngt + eoff] = c * PR_CHUNK + PR_VEC * tid + j;
              ++eoff;
            }
          }
        }
      }
    } else {  // ties at T: ascending token order (chunk-major, then thread, then lane)
      int taken = 0;
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
              if (pos < need) {
                sx[ngt + pos] = get(c, j);
                sv[ngt + pos] = c * PR_CHUNK + PR_VEC * tid + j;
              }
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
      const float xi = sx[i];
      const int vi = sv[i];
      int rank = 0;
#pragma unroll 8
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

// ---- kernel 2: per-request top-k over the rows' candidate lists -----------
typedef int32_t i32x4_t __attribute__((__vector_size__(4 * sizeof(int32_t))));

template <bool LDS_LISTS>  // true: the request's W x k1 lists are staged in LDS
__global__ __launch_bounds__(MG_THREADS) void prune_merge(PruneArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  __shared__ double cs[PR_MAXW];
  // the radix histogram during the selection, then the selected scores / flats
  __shared__ __attribute__((aligned(16))) uint8_t work[PR_MAXK * 16];
  __shared__ int fin[PR_MAXK];
  __shared__ int itmp[MG_THREADS / 64];
  __shared__ int sel[3];
  int* hist = reinterpret_cast<int*>(work);
  double* fsc = reinterpret_cast<double*>(work);
  int64_t* ffl = reinterpret_cast<int64_t*>(work + PR_MAXK * 8);

  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int W = a.W, k1 = a.k1, k = a.k;
  const int n = W * k1;
  const int64_t rbase = (int64_t)r * W;
  const float* gx = a.cand_x + rbase * k1;
  const int32_t* gv = a.cand_v + rbase * k1;
  const float* xs = gx;
  const int32_t* vs = gv;
  if constexpr (LDS_LISTS) {
    float* xl = reinterpret_cast<float*>(dyn);
    int32_t* vl = reinterpret_cast<int32_t*>(dyn + sizeof(float) * (size_t)n);
    if ((n & 3) == 0) {  // the request's lists then start 16-byte aligned
      for (int i = 4 * tid; i < n; i += 4 * MG_THREADS) {
        *reinterpret_cast<f32x4_t*>(xl + i) = *reinterpret_cast<const f32x4_t*>(gx + i);
        *reinterpret_cast<i32x4_t*>(vl + i) = *reinterpret_cast<const i32x4_t*>(gv + i);
      }
    } else {
      for (int i = tid; i < n; i += MG_THREADS) {
        xl[i] = gx[i];
        vl[i] = gv[i];
      }
    }
    xs = xl;
    vs = vl;
  }
  for (int b = tid; b < W; b += MG_THREADS) cs[b] = a.row_c[rbase + b];
  __syncthreads();

  // candidate i = b * k1 + j (row b, list position j), score cum - lse + logit;
  // thread tid visits i = tid, tid + NT, ... with b stepped incrementally.
  // Padding entries (token -1) are no candidates.
  const int db = MG_THREADS / k1, dj = MG_THREADS - db * k1;
  auto for_cand = [&](auto&& f) {
    int b = tid / k1, j = tid - b * k1;
    for (int i = tid; i < n; i += MG_THREADS) {
      const int v = vs[i];
      if (v >= 0) {
        const double c = cs[b];
        const double sc = c == -INFINITY ? -INFINITY : ((double)xs[i] + c) + 0.0;  // -0 -> +0
        f(b, v, sc);
      }
      b += db;
      j += dj;
      if (j >= k1) {
        j -= k1;
        ++b;
      }
    }
  };
  int mv = 0;
  for_cand([&](int, int, double) { ++mv; });
  int excl;
  const int M = block_scan<MG_THREADS>(mv, excl, itmp);
  const int nsel = M < k ? M : k;

  // boundary score (k-th largest), then among exact ties at it the lowest flat
  // index b * V + v (key ~(b << 32 | v): the largest key is the lowest index)
  RadixSel<uint64_t> r1{0, 0, 0, 0}, r2{0, 0, 0, 0};
  bool ties = false;
  if (M > k) {
    r1 = radix_select<MG_THREADS, uint64_t, 64>(
        [&](auto&& f) { for_cand([&](int, int, double sc) { f(dkey(sc)); }); }, k, hist, itmp, sel);
    if (r1.eq != r1.need) {
      ties = true;
      r2 = radix_select<MG_THREADS, uint64_t, 64>(
          [&](auto&& f) {
            for_cand([&](int b, int v, double sc) {
              if (dkey(sc) == r1.prefix) f(~(((uint64_t)b << 32) | (uint32_t)v));
            });
          },
          r1.need, hist, itmp, sel);
    }
  }
  auto selected = [&](int b, int v, double sc) -> bool {
    if (M <= k) return true;
    const uint64_t u = dkey(sc) & r1.mask;
    if (u != r1.prefix) return u > r1.prefix;
    if (!ties) return true;
    return (~(((uint64_t)b << 32) | (uint32_t)v) & r2.mask) >= r2.prefix;
  };
  int cnt = 0;
  for_cand([&](int b, int v, double sc) { cnt += selected(b, v, sc); });
  int off;
  block_scan<MG_THREADS>(cnt, off, itmp);  // nsel in total; the histogram is dead from here
  for_cand([&](int b, int v, double sc) {
    if (selected(b, v, sc)) {
      fsc[off] = sc;
      ffl[off] = (int64_t)b * a.V + v;
      fin[off] = b;
      ++off;
    }
  });
  __syncthreads();
  // final order of the selected set: (score desc, flat asc)
  for (int i = tid; i < nsel; i += MG_THREADS) {
    const double si = fsc[i];
    const int64_t fi = ffl[i];
    int rank = 0;
#pragma unroll 8
    for (int u = 0; u < nsel; ++u) {
      const double su = fsc[u];
      rank += (su > si) || (su == si && ffl[u] < fi);
    }
    const int64_t o = (int64_t)r * k + rank;
    a.parent[o] = fin[i];
    a.token[o] = (int32_t)(fi - (int64_t)fin[i] * a.V);
    a.score[o] = (float)si;
  }
  for (int i = nsel + tid; i < k; i += MG_THREADS) {
    const int64_t o = (int64_t)r * k + i;
    a.parent[o] = -1;
    a.token[o] = -1;
    a.score[o] = -INFINITY;
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
    hipLaunchKernelGGL(prune_merge<true>, dim3((unsigned)num_reqs), dim3(MG_THREADS), list_bytes, stream, a);
  } else {
    hipLaunchKernelGGL(prune_merge<false>, dim3((unsigned)num_reqs), dim3(MG_THREADS), 0, stream, a);
  }
  return launch_status();
}
