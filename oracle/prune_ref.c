/*
 * CPU oracle for fused beam pruning.  TEST INFRASTRUCTURE ONLY: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Reference algorithm (vllm_gr/entrypoints/openai/serving_engine.py:457-592,
 * offline twin vllm_gr/entrypoints/llm.py:201-280):
 *   score(b, v) = cum_logprob[b] + log_softmax(logits[b])[v]        (:511)
 *   stage 1: per beam, the top-K tokens (K = beam width; the sampler's
 *            logprobs=W request, serving_engine.py:300-308)
 *   EOS:     candidates equal to eos go to `completed` and leave the pool
 *            (:541-562)
 *   stage 2: top-W over the union by score (np.argpartition, :566-567),
 *            fork_info = (flat // K, token) (:590).
 *
 * Build contract restated here (the reference leaves tie order unspecified
 * and composes the score in float64 on the host, :538-539):
 *   m     = max_v x[v]                                   (fp32, exact)
 *   e_v   = exp2_neg(fmaf(x[v], LOG2E_F, -(m * LOG2E_F))) (fp32, see below)
 *   S     = fp32 sum of e_v in the fixed order below
 *   lse   = (double)m + log_f64((double)S)               (fp64, see below)
 *   c_b   = (double)cum[b] - lse                         (fp64)
 *   s     = (double)x[v] + c_b                           (fp64)
 *   stage 1 order: (x desc, v asc); stage 2 order: (s desc, flat asc),
 *   flat = b * V + v.  A row whose max is -inf has lse = c = s = -inf.
 *
 * Fixed summation order for S (the HIP kernel's layout: 256 threads in 4
 * waves of 64, each thread owning float4 groups):
 *   thread t owns elements [c*1024 + 4t, c*1024 + 4t + 4) for c = 0, 1, ...;
 *   its partial is the left-to-right fp32 sum over its elements in index
 *   order; within each wave of 64 lanes, for mask = 32,16,8,4,2,1:
 *   a[l] = a[l] + a[l ^ mask]; finally S = (w0 + w1) + (w2 + w3).
 *
 * exp2_neg(t), t <= 0: t = fmaxf(t, -126) (so -inf and NaN give 2^-126, a
 *   normal float); k = rint(t), f = t - k (exact),
 *   p = Horner in f with fmaf over the degree-5 coefficients EXP2_C (the
 *   Remez minimax of the relative error of 2^f on [-1/2, 1/2] with p(0) = 1,
 *   rounded to float32, c3 and c5 then nudged; oracle/fit_exp2.py derives the
 *   fit and measures both sets: within 2.02 ulp), result =
 *   ldexpf(p, k).
 * log_f64(s), s >= 1: s = mant * 2^e with mant in [sqrt(1/2), sqrt(2));
 *   z = (mant - 1) / (mant + 1); w = z*z;
 *   q = Horner in w with fma over 1/(2j+1), j = 11..0 (atanh series,
 *   log(mant) = 2 atanh(z)); result = e*LN2_HI + (e*LN2_LO + (z + z) * q).
 *
 * Every operation is a single IEEE-754 operation (add, sub, mul, div, fma,
 * rint, ldexp, frexp) so the result is reproducible bit for bit on any
 * conforming machine.  Compile with -ffp-contract=off.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define PRUNE_THREADS 256
#define PRUNE_WAVE 64
#define PRUNE_VEC 4

static const float LOG2E_F = 0x1.715476p+0f;
static const float EXP2_C[6] = {
    0x1.000000p+0f, 0x1.62e42ap-1f, 0x1.ebf9bcp-3f, 0x1.c6b746p-5f, 0x1.3cea88p-7f, 0x1.5bbea6p-10f};
static const double LN2_HI = 0x1.62e42p-1;
static const double LN2_LO = 0x1.fdf473de6af28p-22;
static const double SQRT_HALF = 0x1.6a09e667f3bcdp-1;

float oracle_exp2_neg(float t) {
  t = fmaxf(t, -126.0f);
  float k = rintf(t);
  float f = t - k;
  float p = EXP2_C[5];
  for (int j = 4; j >= 0; --j) p = fmaf(p, f, EXP2_C[j]);
  return ldexpf(p, (int)k);
}

double oracle_log_f64(double s) {
  int e;
  double mant = frexp(s, &e); /* mant in [0.5, 1) */
  if (mant < SQRT_HALF) {
    mant = mant * 2.0;
    e -= 1;
  }
  double z = (mant - 1.0) / (mant + 1.0);
  double w = z * z;
  double q = 1.0 / 23.0;
  for (int j = 10; j >= 0; --j) q = fma(q, w, 1.0 / (double)(2 * j + 1));
  double de = (double)e;
  return de * LN2_HI + (de * LN2_LO + (z + z) * q);
}

/* Row statistics in the fixed order.  Returns m; writes S and lse. */
static float row_stats(const float* x, int V, float* S_out, double* lse_out) {
  float m = -INFINITY;
  for (int v = 0; v < V; ++v) m = x[v] > m ? x[v] : m;
  if (m == -INFINITY) {
    *S_out = 0.0f;
    *lse_out = -INFINITY;
    return m;
  }
  const float ml = m * LOG2E_F;
  float part[PRUNE_THREADS];
  for (int t = 0; t < PRUNE_THREADS; ++t) {
    float acc = 0.0f;
    for (int base = 0; base < V; base += PRUNE_THREADS * PRUNE_VEC) {
      for (int j = 0; j < PRUNE_VEC; ++j) {
        int v = base + PRUNE_VEC * t + j;
        if (v < V) {
          float tt = fmaf(x[v], LOG2E_F, -ml);
          acc = acc + oracle_exp2_neg(tt);
        }
      }
    }
    part[t] = acc;
  }
  float wsum[PRUNE_THREADS / PRUNE_WAVE];
  for (int w = 0; w < PRUNE_THREADS / PRUNE_WAVE; ++w) {
    float a[PRUNE_WAVE], b[PRUNE_WAVE];
    memcpy(a, part + w * PRUNE_WAVE, sizeof(a));
    for (int mask = PRUNE_WAVE / 2; mask >= 1; mask >>= 1) {
      for (int l = 0; l < PRUNE_WAVE; ++l) b[l] = a[l] + a[l ^ mask];
      memcpy(a, b, sizeof(a));
    }
    wsum[w] = a[0];
  }
  float S = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
  *S_out = S;
  *lse_out = (double)m + oracle_log_f64((double)S);
  return m;
}

void oracle_prune_row_stats(const float* logits, const double* cum, int rows, int V,
                            float* m_out, float* S_out, double* lse_out, double* c_out) {
  for (int r = 0; r < rows; ++r) {
    float S;
    double lse;
    float m = row_stats(logits + (size_t)r * V, V, &S, &lse);
    if (m_out) m_out[r] = m;
    if (S_out) S_out[r] = S;
    if (lse_out) lse_out[r] = lse;
    if (c_out) c_out[r] = (m == -INFINITY) ? -INFINITY : cum[r] - lse;
  }
}

/* ---- bounded selection with an explicit total order ------------------ */
typedef struct {
  double key; /* larger is better */
  int64_t idx; /* smaller is better on equal key */
} cand_t;

/* a strictly better than b */
static int better(const cand_t* a, const cand_t* b) {
  if (a->key != b->key) return a->key > b->key;
  return a->idx < b->idx;
}

/* min-heap on "better": root is the worst kept candidate */
static void sift_down(cand_t* h, int n, int i) {
  for (;;) {
    int l = 2 * i + 1, r = l + 1, w = i;
    if (l < n && better(&h[w], &h[l])) w = l;
    if (r < n && better(&h[w], &h[r])) w = r;
    if (w == i) return;
    cand_t t = h[i];
    h[i] = h[w];
    h[w] = t;
    i = w;
  }
}
static void sift_up(cand_t* h, int i) {
  while (i > 0) {
    int p = (i - 1) / 2;
    if (!better(&h[p], &h[i])) return;
    cand_t t = h[i];
    h[i] = h[p];
    h[p] = t;
    i = p;
  }
}
static int cmp_desc(const void* a, const void* b) {
  const cand_t* x = (const cand_t*)a;
  const cand_t* y = (const cand_t*)b;
  if (better(x, y)) return -1;
  if (better(y, x)) return 1;
  return 0;
}

typedef struct {
  cand_t* h;
  int n, cap;
} topk_t;

static void topk_push(topk_t* t, cand_t c) {
  if (t->n < t->cap) {
    t->h[t->n] = c;
    sift_up(t->h, t->n);
    t->n++;
  } else if (t->cap > 0 && better(&c, &t->h[0])) {
    t->h[0] = c;
    sift_down(t->h, t->n, 0);
  }
}

/*
 * Full prune.  logits [R*W, V] row-major, cum [R*W] float64 (a float32
 * cumulative score enters exactly, as its float64 value).  Outputs [R, k]:
 * parent (beam within request), token, score (fp32 of the fp64 score),
 * score64 (nullable); eos_score [R*W] float64 (nullable; -inf when the
 * beam's top-k holds no EOS).  Slots past the available candidates get
 * -1/-1/-inf.  cand_token / cand_logprob [R*W, k1] (nullable): each row's
 * top-k1 by (x desc, v asc) before EOS / catalog removal, with logprob =
 * (float)((double)x - lse) (-inf for a row of -inf logits).
 * allowed [R*W, V] (nullable): the catalog mask -- a stage-1 candidate whose
 * token is not allowed for its beam leaves the pool (the reference sets its
 * logprob to -inf after the per-beam top-K, serving_engine.py:504-506); EOS
 * reports a score only when allowed.
 * Returns 0, or -1 on bad arguments.
 */
int oracle_prune_topk(const float* logits, const double* cum, int R, int W, int V, int k,
                      int eos, int32_t* parent, int32_t* token, float* score,
                      double* score64, double* eos_score, const uint8_t* allowed,
                      int32_t* cand_token, float* cand_logprob) {
  if (R < 0 || W <= 0 || V <= 0 || k <= 0) return -1;
  int k1 = k < V ? k : V;
  cand_t* row_heap = (cand_t*)malloc(sizeof(cand_t) * (size_t)k1);
  cand_t* req_heap = (cand_t*)malloc(sizeof(cand_t) * (size_t)k);
  for (int r = 0; r < R; ++r) {
    topk_t req = {req_heap, 0, k};
    for (int b = 0; b < W; ++b) {
      const float* x = logits + ((size_t)r * W + b) * V;
      float S;
      double lse;
      float m = row_stats(x, V, &S, &lse);
      double c = (m == -INFINITY) ? -INFINITY : cum[r * W + b] - lse;
      /* stage 1: per-row top-k1 by (x desc, v asc) */
      topk_t row = {row_heap, 0, k1};
      for (int v = 0; v < V; ++v) {
        cand_t cd = {(double)x[v], v};
        topk_push(&row, cd);
      }
      if (cand_token) {
        /* the row's list in order: a copy of the heap, sorted */
        cand_t* sorted = (cand_t*)malloc(sizeof(cand_t) * (size_t)k1);
        memcpy(sorted, row.h, sizeof(cand_t) * (size_t)row.n);
        qsort(sorted, row.n, sizeof(cand_t), cmp_desc);
        for (int i = 0; i < k1; ++i) {
          size_t o = ((size_t)r * W + b) * k1 + i;
          cand_token[o] = i < row.n ? (int32_t)sorted[i].idx : -1;
          cand_logprob[o] = i < row.n ? (m == -INFINITY ? -INFINITY : (float)(sorted[i].key - lse)) : -INFINITY;
        }
        free(sorted);
      }
      if (eos_score) eos_score[r * W + b] = -INFINITY;
      for (int i = 0; i < row.n; ++i) {
        int v = (int)row.h[i].idx;
        if (allowed && !allowed[((size_t)r * W + b) * V + v]) continue;
        double s = (m == -INFINITY) ? -INFINITY : (double)x[v] + c;
        if (v == eos) {
          if (eos_score) eos_score[r * W + b] = s;
          continue;
        }
        cand_t cd = {s, (int64_t)b * V + v};
        topk_push(&req, cd);
      }
    }
    qsort(req.h, req.n, sizeof(cand_t), cmp_desc);
    for (int i = 0; i < k; ++i) {
      size_t o = (size_t)r * k + i;
      if (i < req.n) {
        parent[o] = (int32_t)(req.h[i].idx / V);
        token[o] = (int32_t)(req.h[i].idx % V);
        score[o] = (float)req.h[i].key;
        if (score64) score64[o] = req.h[i].key;
      } else {
        parent[o] = -1;
        token[o] = -1;
        score[o] = -INFINITY;
        if (score64) score64[o] = -INFINITY;
      }
    }
  }
  free(row_heap);
  free(req_heap);
  return 0;
}
