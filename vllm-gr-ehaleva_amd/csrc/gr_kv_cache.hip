// Beam KV fork / append and slot scatter for gfx950.
//
// All three kernels move K/V rows of head_dim elements in 16-byte vectors;
// they are pure HBM copy work (no arithmetic), so the design goal is wide
// coalesced accesses, balanced work and no serialisation:
//  * beam_fork: one workgroup per two children (W/2 per request; one per
//    child when W is odd).  Every workgroup works out its request's whole plan
//    in LDS from the read-only input tables: each parent's lowest child (kept
//    in place), the copying children and their ranks, the childless parents
//    they take over (the owners), and the prefix sums of the copy lengths.
//    The request's copy-on-write tokens, concatenated, are then split evenly
//    over its workgroups, so the copy work is spread over every workgroup
//    whichever children copy; each token's rows are resolved once.  Copy
//    destinations are rows of childless parents, which nobody reads; sources
//    are rows of parents with children, which nobody writes below their
//    length; each child's own append goes to a position past every copied
//    range of its row; the new tables are written out of place -- so the
//    single launch is race-free with no inter-workgroup dependency.
//  * beam_append / reshape_and_cache: one wave per beam / token.
#include "gr_common.h"

#include <algorithm>

namespace gr {
namespace {

typedef uint32_t u32x4_t __attribute__((__vector_size__(4 * sizeof(uint32_t))));

constexpr int FORK_THREADS = 256;
constexpr int FORK_MAX_W = 1024;
constexpr int FORK_STAGE_BT = 2048;  // a request's whole block table is staged in LDS up to this many entries

// Copy-on-write tokens a workgroup resolves per round: each token's source
// and destination row offsets are worked out once (one search of the copy
// prefix sums per token, not per vector) and staged in LDS.
constexpr int FORK_TOK_CHUNK = 64;

// the fork kernel's LDS, sized by the request width W (ints; the 64-bit words
// first): cow and free masks, the staged token offsets, par,
// first (later the copy lengths), cnt, lens, owner_of, cpre (W + 1), the scan
// scratch, the staged block table
__host__ __device__ inline int fork_lds_ints(int W, int S) {
  const int ng = (W + 63) >> 6;
  return 4 * ng + 4 * FORK_TOK_CHUNK + 6 * W + 1 + 8 + 1 + (W * S <= FORK_STAGE_BT ? W * S : 0);
}
constexpr int FORK_BATCH = 2;        // 16-byte K and V vectors per thread in flight
constexpr int FORK_MAX_LAYERS = 32;  // layers one fork launch moves (more take further launches)

// Base addresses of the layers a fork launch moves (every layer has the same
// geometry); layer 0 is also the KvGeom's cache.
struct KvLayers {
  uint8_t* k[FORK_MAX_LAYERS];
  uint8_t* v[FORK_MAX_LAYERS];
};

struct KvGeom {
  void* k_cache;
  void* v_cache;
  int64_t num_blocks, block_stride, tok_stride, head_stride;
  int Hkv, D, bs, esize;
};

// byte offset of (block, offset, head) in the cache
__device__ inline int64_t kv_byte_off(const KvGeom& g, int64_t blk, int off, int h) {
  return (blk * g.block_stride + (int64_t)off * g.tok_stride + (int64_t)h * g.head_stride) * g.esize;
}

// exclusive prefix sum of v[0 .. n) into out[0 .. n] (out[n] = total) by a
// 256-thread workgroup, n <= FORK_MAX_W; tmp: 8 ints
// Position of the k-th (0-based) set bit of x (k below the popcount).
__device__ inline int select_bit(uint64_t x, int k) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const uint64_t lo = x & ((1ull << w) - 1);
    const int c = __builtin_popcountll(lo);
    if (k >= c) {
      k -= c;
      x >>= w;
      pos += w;
    } else {
      x = lo;
    }
  }
  return pos;
}

__device__ inline void block_scan(const int* v, int* out, int n, int* tmp) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int PER = FORK_MAX_W / FORK_THREADS;
  int x[PER], s = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u) {  // thread tid owns entries PER*tid .. PER*tid + PER-1
    const int i = PER * tid + u;
    x[u] = i < n ? v[i] : 0;
    s += x[u];
  }
  const int incl = wave_incl_scan(s);
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = incl - s;
  for (int w = 0; w < wave; ++w) base += tmp[w];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = PER * tid + u;
    if (i < n) out[i] = base;
    base += x[u];
  }
  if (tid == FORK_THREADS - 1) out[n] = base;
  __syncthreads();
}

// beam_fork's argument list as one struct (same types in the same order, so
// the same layout): its size is the span of argument lines the kernel touches.
struct ForkKernargs {
  const int32_t* parent;
  int R, W, cpw;
  const int32_t *bt_in, *len_in;
  int32_t *bt_out, *len_out;
  int S;
  KvGeom g;
  int L;
  KvLayers layers;
  const uint8_t *k_new, *v_new;
  int64_t new_tok_stride;
  int32_t* dev_status;
};

// 8 waves per SIMD: every workgroup of a 2048-child batch resident at once.
// Workgroup cg of request r owns children cg*cpw .. cg*cpw + cpw-1.
// MULTI: L layers (their bases in `layers`); otherwise the one layer of g.
template <bool MULTI>
__global__ __launch_bounds__(FORK_THREADS, 8) void beam_fork(
    const int32_t* __restrict__ parent, int R, int W, int cpw, const int32_t* __restrict__ bt_in,
    const int32_t* __restrict__ len_in, int32_t* __restrict__ bt_out, int32_t* __restrict__ len_out,
    int S, KvGeom g, int L, KvLayers layers, const uint8_t* k_new, const uint8_t* v_new, int64_t new_tok_stride,
    int32_t* dev_status) {
  kernarg_lines<kernarg_line_count<ForkKernargs>()>();
  extern __shared__ __attribute__((aligned(8))) int fork_lds[];
  __shared__ uint8_t* lay_k[FORK_MAX_LAYERS];  // the layers' bases, indexed per lane by the copy loop
  __shared__ uint8_t* lay_v[FORK_MAX_LAYERS];
  if (MULTI && threadIdx.x < L) {
    lay_k[threadIdx.x] = layers.k[threadIdx.x];
    lay_v[threadIdx.x] = layers.v[threadIdx.x];
  }
  const int ngroups = (W + 63) >> 6;
  uint64_t* cow_mask = reinterpret_cast<uint64_t*>(fork_lds);
  uint64_t* free_mask = cow_mask + ngroups;
  int64_t* tok_src = reinterpret_cast<int64_t*>(free_mask + ngroups);  // byte offset of a token's head-0 row, -1: skip
  int64_t* tok_dst = tok_src + FORK_TOK_CHUNK;
  int* par = reinterpret_cast<int*>(tok_dst + FORK_TOK_CHUNK);
  int* first = par + W;
  int* cnt = first + W;
  int* lens = cnt + W;
  int* owner_of = lens + W;
  int* cpre = owner_of + W;
  int* scan_tmp = cpre + W + 1;
  int& bad = scan_tmp[8];
  int* bts = scan_tmp + 9;
  int* cplen = first;  // once the masks are built
  const int wpr = W / cpw;  // workgroups per request
  const int r = blockIdx.x / wpr;
  const int cg = blockIdx.x - r * wpr;  // this workgroup's group of children
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (r >= R) return;
  const int row_vecs = g.D * g.esize / 16;  // 16-byte vectors per (token, head) row
  const int tv = g.Hkv * row_vecs;          // 16-byte vectors per token, all heads
  // the request's parents, lengths and (when small) block table first, then
  // the appended tokens' vectors: the tables' wait does not include those
  constexpr int PER = FORK_MAX_W / FORK_THREADS;
  constexpr int BT_PER = FORK_STAGE_BT / FORK_THREADS;
  const bool all_staged = W * S <= FORK_STAGE_BT;
  int pv[PER], lv[PER], bv[BT_PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid + u * FORK_THREADS;
    pv[u] = i < W ? parent[(int64_t)r * W + i] : 0;
    lv[u] = i < W ? len_in[(int64_t)r * W + i] : 0;
  }
#pragma unroll
  for (int u = 0; u < BT_PER; ++u) {
    const int j = tid + u * FORK_THREADS;
    bv[u] = all_staged && j < W * S ? bt_in[(int64_t)r * W * S + j] : 0;
  }
  __builtin_amdgcn_sched_barrier(0);
  // thread tid appends vector tid % tv of child cg*cpw + tid / tv (when the
  // group's appended tokens fit one vector per thread)
  const bool pre_new = k_new && tv * cpw <= FORK_THREADS && tid < tv * cpw;
  const int aq = tid / tv, ae = tid - (tid / tv) * tv;
  const int nh = ae / row_vecs, nvec = ae - (ae / row_vecs) * row_vecs;
  u32x4_t knew{}, vnew{};
  if (pre_new) {
    const int64_t src = (((int64_t)r * W + cg * cpw + aq) * new_tok_stride + (int64_t)nh * g.D) * g.esize + nvec * 16;
    knew = *reinterpret_cast<const u32x4_t*>(k_new + src);
    vnew = *reinterpret_cast<const u32x4_t*>(v_new + src);
  }
  if (tid == 0) bad = 0;
  for (int i = tid; i < W; i += FORK_THREADS) {
    first[i] = W;
    cnt[i] = 0;
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid + u * FORK_THREADS;
    if (i < W) lens[i] = lv[u];
  }
  if (all_staged) {
#pragma unroll
    for (int u = 0; u < BT_PER; ++u) {
      const int j = tid + u * FORK_THREADS;
      if (j < W * S) bts[j] = bv[u];
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid + u * FORK_THREADS;
    if (i < W) {
      int p = pv[u];
      if (p < 0 || p >= W) {
        bad = 1;
        p = i;
      }
      par[i] = p;
      atomicMin(&first[p], i);
      atomicAdd(&cnt[p], 1);
    }
  }
  __syncthreads();
  const bool req_bad = bad != 0;
  if (req_bad) {  // a request with a bad parent keeps its tables
    if (cg == 0 && tid == 0) flag_status(dev_status, GR_DEV_BAD_PARENT);
    for (int q = 0; q < cpw; ++q) {
      const int64_t n_c = (int64_t)r * W + cg * cpw + q;
      for (int j = tid; j < S; j += FORK_THREADS) bt_out[n_c * S + j] = bt_in[n_c * S + j];
      if (tid == 0) len_out[n_c] = lens[cg * cpw + q];
    }
    return;
  }
  // per 64-entry group: the children that copy (not their parent's lowest
  // child) and the parents without children
  for (int base = 0; base < W; base += FORK_THREADS) {
    const int i = base + tid;
    const bool in = i < W;
    const bool cw = in && first[par[in ? i : 0]] != i;
    const bool fr = in && cnt[in ? i : 0] == 0;
    const uint64_t cm = __builtin_amdgcn_ballot_w64(cw);
    const uint64_t fm = __builtin_amdgcn_ballot_w64(fr);
    if (lane == 0 && base + 64 * wave < W) {
      cow_mask[(base >> 6) + wave] = cm;
      free_mask[(base >> 6) + wave] = fm;
    }
  }
  __syncthreads();
  // the k-th childless parent (ascending) goes to the k-th copying child
  // (ascending; the two counts are equal): a copying child takes its rank
  // from the copy masks and selects that set bit of the childless masks
  const int cap = S * g.bs;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid + u * FORK_THREADS;
    if (i < W) {
      const uint64_t cm = cow_mask[i >> 6];
      const bool cw = (cm >> (i & 63)) & 1;
      int own = par[i];
      if (cw) {
        int k = __builtin_popcountll(cm & ((1ull << (i & 63)) - 1));
        for (int gi = 0; gi < (i >> 6); ++gi) k += __builtin_popcountll(cow_mask[gi]);
        int gw = 0;
        uint64_t fm = free_mask[0];
        int cnt_w = __builtin_popcountll(fm);
        while (k >= cnt_w && gw + 1 < ngroups) {
          k -= cnt_w;
          fm = free_mask[++gw];
          cnt_w = __builtin_popcountll(fm);
        }
        own = min(64 * gw + select_bit(fm, k), W - 1);
      }
      owner_of[i] = own;
      const int len = lens[par[i]];
      cplen[i] = cw ? (len < 0 ? 0 : len > cap ? cap : len) : 0;
    }
  }
  __syncthreads();
  block_scan(cplen, cpre, W, scan_tmp);  // (its barriers publish owner_of too)
  auto row_blk = [&](int row, int bi) -> int {
    return all_staged ? bts[row * S + bi] : bt_in[((int64_t)r * W + row) * S + bi];
  };
  uint8_t* kc = static_cast<uint8_t*>(g.k_cache);
  uint8_t* vc = static_cast<uint8_t*>(g.v_cache);
  // ---- each child of the group: its new table row, its appended token at
  // its row's length (past every copied range of the row), its new length
  for (int q = 0; q < cpw; ++q) {
    const int c = cg * cpw + q;
    const int64_t n_c = (int64_t)r * W + c;
    const int owner = owner_of[c];  // beam whose old row child c receives
    const int64_t n_o = (int64_t)r * W + owner;
    for (int j = tid; j < S; j += FORK_THREADS) bt_out[n_c * S + j] = all_staged ? bts[owner * S + j] : bt_in[n_o * S + j];
    int len = lens[par[c]];
    if (len < 0 || len > cap) {
      if (tid == 0) flag_status(dev_status, GR_DEV_BAD_LENGTH);
      len = len < 0 ? 0 : cap;
    }
    int new_len = len;
    if (k_new) {
      if (len < cap) {
        const int bdst = row_blk(owner, len / g.bs);
        if (bdst >= 0 && bdst < g.num_blocks) {
          if (tv * cpw <= FORK_THREADS) {
            if (pre_new && aq == q) {
              const int64_t dof = kv_byte_off(g, bdst, len % g.bs, nh) + nvec * 16;
              *reinterpret_cast<u32x4_t*>(kc + dof) = knew;
              *reinterpret_cast<u32x4_t*>(vc + dof) = vnew;
            }
          } else {
            for (int e = tid; e < tv; e += FORK_THREADS) {
              const int h = e / row_vecs, vec = e - h * row_vecs;
              const int64_t src = (n_c * new_tok_stride + (int64_t)h * g.D) * g.esize + vec * 16;
              const int64_t dof = kv_byte_off(g, bdst, len % g.bs, h) + vec * 16;
              *reinterpret_cast<u32x4_t*>(kc + dof) = *reinterpret_cast<const u32x4_t*>(k_new + src);
              *reinterpret_cast<u32x4_t*>(vc + dof) = *reinterpret_cast<const u32x4_t*>(v_new + src);
            }
          }
          new_len = len + 1;
        } else if (tid == 0) {
          flag_status(dev_status, GR_DEV_BAD_BLOCK);
        }
      } else if (tid == 0) {
        flag_status(dev_status, GR_DEV_SUFFIX_FULL);
      }
    }
    if (tid == 0) len_out[n_c] = new_len;
  }
  // ---- this workgroup's share of the request's copy-on-write tokens, in
  // rounds of FORK_TOK_CHUNK tokens: one thread per token finds its copying
  // child and block ids, then the round's vectors move
  const int total = cpre[W];
  const int e0 = (int)((int64_t)total * cg / wpr), e1 = (int)((int64_t)total * (cg + 1) / wpr);
  if (g.num_blocks > 0) {
#pragma unroll 1
    for (int t0 = e0; t0 < e1; t0 += FORK_TOK_CHUNK) {
      const int nt = min(FORK_TOK_CHUNK, e1 - t0);
      __syncthreads();  // the previous round's readers of tok_src / tok_dst are done
      if (tid < nt) {
        const int e = t0 + tid;
        int lo = 0, hi = W - 1;  // the copying child whose range holds e (skips empty ranges)
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (cpre[mid] <= e) lo = mid; else hi = mid - 1;
        }
        const int pos = e - cpre[lo];
        const int bi = pos / g.bs, off = pos - bi * g.bs;
        const int bsrc = row_blk(par[lo], bi), bdst = row_blk(owner_of[lo], bi);
        const bool valid = bsrc >= 0 && bsrc < g.num_blocks && bdst >= 0 && bdst < g.num_blocks;
        if (!valid) flag_status(dev_status, GR_DEV_BAD_BLOCK);
        tok_src[tid] = valid ? kv_byte_off(g, bsrc, off, 0) : -1;
        tok_dst[tid] = valid ? kv_byte_off(g, bdst, off, 0) : -1;
      }
      __syncthreads();
      // the round's vectors of every layer, one flat range: item it is layer
      // it / items, vector it % items of the round
      const int items = nt * tv;
      const int all_items = (MULTI ? L : 1) * items;
#pragma unroll 1
      for (int i0 = tid; i0 < all_items; i0 += FORK_THREADS * FORK_BATCH) {
        u32x4_t kb[FORK_BATCH], vb[FORK_BATCH];
        uint8_t* kd[FORK_BATCH];
        uint8_t* vd[FORK_BATCH];
        bool ok[FORK_BATCH];
#pragma unroll
        for (int u = 0; u < FORK_BATCH; ++u) {
          const int it = i0 + u * FORK_THREADS;
          const int l = MULTI && it < all_items ? it / items : 0;
          const int li = it - l * items;
          const int tk = li / tv, rem = li - (li / tv) * tv;
          const int h = rem / row_vecs, vec = rem - (rem / row_vecs) * row_vecs;
          const int64_t so = it < all_items ? tok_src[tk] : -1;
          ok[u] = so >= 0;
          const int64_t hoff = (int64_t)h * g.head_stride * g.esize + vec * 16;
          const int64_t dof = ok[u] ? tok_dst[tk] + hoff : 0;
          const int64_t sof = ok[u] ? so + hoff : 0;
          uint8_t* kl = MULTI ? lay_k[l] : kc;
          uint8_t* vl = MULTI ? lay_v[l] : vc;
          kd[u] = kl + dof;
          vd[u] = vl + dof;
          kb[u] = *reinterpret_cast<const u32x4_t*>(kl + sof);
          vb[u] = *reinterpret_cast<const u32x4_t*>(vl + sof);
        }
#pragma unroll
        for (int u = 0; u < FORK_BATCH; ++u) {
          if (ok[u]) {
            *reinterpret_cast<u32x4_t*>(kd[u]) = kb[u];
            *reinterpret_cast<u32x4_t*>(vd[u]) = vb[u];
          }
        }
      }
    }
  }
}

// One 64-lane wave per beam: append its token at suffix_len[n], then bump it.
__global__ __launch_bounds__(64) void beam_append(const uint8_t* k_new, const uint8_t* v_new,
                                                  int64_t new_tok_stride, KvGeom g,
                                                  const int32_t* __restrict__ bt, int S,
                                                  int32_t* __restrict__ len, int N, int32_t* dev_status) {
  const int n = blockIdx.x;
  if (n >= N) return;
  const int cur = len[n];
  const int cap = S * g.bs;
  const int row_vecs = g.D * g.esize / 16;
  bool ok = cur >= 0 && cur < cap;
  int blk = ok ? bt[(int64_t)n * S + cur / g.bs] : -1;
  ok = ok && blk >= 0 && blk < g.num_blocks;
  if (ok) {
    uint8_t* kc = static_cast<uint8_t*>(g.k_cache);
    uint8_t* vc = static_cast<uint8_t*>(g.v_cache);
    for (int e = threadIdx.x; e < g.Hkv * row_vecs; e += 64) {
      const int vec = e % row_vecs, h = e / row_vecs;
      const int64_t src = ((int64_t)n * new_tok_stride + (int64_t)h * g.D) * g.esize + vec * 16;
      const int64_t dof = kv_byte_off(g, blk, cur % g.bs, h) + vec * 16;
      *reinterpret_cast<u32x4_t*>(kc + dof) = *reinterpret_cast<const u32x4_t*>(k_new + src);
      *reinterpret_cast<u32x4_t*>(vc + dof) = *reinterpret_cast<const u32x4_t*>(v_new + src);
    }
  }
  __syncthreads();  // every lane has read len[n] before it changes
  if (threadIdx.x == 0) {
    if (ok) len[n] = cur + 1;
    else flag_status(dev_status, (cur >= cap) ? GR_DEV_SUFFIX_FULL : (cur < 0 ? GR_DEV_BAD_LENGTH : GR_DEV_BAD_BLOCK));
  }
}

__global__ __launch_bounds__(64) void reshape_and_cache_k(const uint8_t* key, int64_t key_stride,
                                                          const uint8_t* value, int64_t value_stride,
                                                          KvGeom g, const int64_t* __restrict__ slots,
                                                          int T, int32_t* dev_status) {
  const int t = blockIdx.x;
  if (t >= T) return;
  const int64_t slot = slots[t];
  if (slot < 0) return;
  const int64_t blk = slot / g.bs;
  const int off = (int)(slot % g.bs);
  if (blk >= g.num_blocks) {
    if (threadIdx.x == 0) flag_status(dev_status, GR_DEV_BAD_BLOCK);
    return;
  }
  const int row_vecs = g.D * g.esize / 16;
  uint8_t* kc = static_cast<uint8_t*>(g.k_cache);
  uint8_t* vc = static_cast<uint8_t*>(g.v_cache);
  for (int e = threadIdx.x; e < g.Hkv * row_vecs; e += 64) {
    const int vec = e % row_vecs, h = e / row_vecs;
    const int64_t dof = kv_byte_off(g, blk, off, h) + vec * 16;
    *reinterpret_cast<u32x4_t*>(kc + dof) =
        *reinterpret_cast<const u32x4_t*>(key + ((int64_t)t * key_stride + (int64_t)h * g.D) * g.esize + vec * 16);
    *reinterpret_cast<u32x4_t*>(vc + dof) =
        *reinterpret_cast<const u32x4_t*>(value + ((int64_t)t * value_stride + (int64_t)h * g.D) * g.esize + vec * 16);
  }
}

// Quantising scatter into an fp8 e4m3 cache: one workgroup per token, four
// elements (one 32-bit word of the cache) per thread and step.
template <int DT>
__global__ __launch_bounds__(256) void reshape_and_cache_fp8_k(const void* key, int64_t key_stride, const void* value,
                                                               int64_t value_stride, KvGeom g,
                                                               const int64_t* __restrict__ slots, int T,
                                                               const float* k_scale, const float* v_scale,
                                                               int32_t* dev_status) {
  using E = Elem<DT>;
  using S = typename E::storage;
  const int t = blockIdx.x;
  if (t >= T) return;
  const int64_t slot = slots[t];
  if (slot < 0) return;
  const int64_t blk = slot / g.bs;
  const int off = (int)(slot % g.bs);
  if (blk >= g.num_blocks) {
    if (threadIdx.x == 0) flag_status(dev_status, GR_DEV_BAD_BLOCK);
    return;
  }
  const float ks = k_scale ? k_scale[0] : 1.0f, vs = v_scale ? v_scale[0] : 1.0f;
  const int words = g.D / 4;
  uint8_t* kc = static_cast<uint8_t*>(g.k_cache);
  uint8_t* vc = static_cast<uint8_t*>(g.v_cache);
  for (int e = threadIdx.x; e < g.Hkv * words; e += 256) {
    const int h = e / words, d0 = (e - h * words) * 4;
    const S* kp = static_cast<const S*>(key) + (int64_t)t * key_stride + (int64_t)h * g.D + d0;
    const S* vp = static_cast<const S*>(value) + (int64_t)t * value_stride + (int64_t)h * g.D + d0;
    uint32_t kw = 0, vw = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kw |= float_to_fp8e4m3(E::to_float(kp[j]) / ks) << (8 * j);
      vw |= float_to_fp8e4m3(E::to_float(vp[j]) / vs) << (8 * j);
    }
    const int64_t dof = kv_byte_off(g, blk, off, h) + d0;
    *reinterpret_cast<uint32_t*>(kc + dof) = kw;
    *reinterpret_cast<uint32_t*>(vc + dof) = vw;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 16-byte vector moves need every row start 16-byte aligned.
gr_status_t check_geom(const KvGeom& g) {
  if (!g.k_cache || !g.v_cache || g.num_blocks < 0 || g.Hkv < 1 || g.bs < 1 || g.D < 8)
    return GR_ERR_INVALID_ARG;
  if ((g.D * g.esize) % 16 || !aligned16(g.k_cache) || !aligned16(g.v_cache)) return GR_ERR_INVALID_ARG;
  if ((g.block_stride * g.esize) % 16 || (g.tok_stride * g.esize) % 16 || (g.head_stride * g.esize) % 16)
    return GR_ERR_INVALID_ARG;
  if (g.block_stride < 1 || g.tok_stride < 1 || g.head_stride < 1) return GR_ERR_INVALID_ARG;
  return GR_OK;
}

KvGeom make_geom(void* k_cache, void* v_cache, int64_t num_blocks, int64_t bstr, int64_t tstr,
                 int64_t hstr, int Hkv, int D, int bs, int dtype) {
  KvGeom g;
  g.k_cache = k_cache;
  g.v_cache = v_cache;
  g.num_blocks = num_blocks;
  g.block_stride = bstr;
  g.tok_stride = tstr;
  g.head_stride = hstr;
  g.Hkv = Hkv;
  g.D = D;
  g.bs = bs;
  g.esize = dtype_size(dtype);
  return g;
}

}  // namespace
}  // namespace gr

using namespace gr;

namespace gr {
namespace {

// Checks shared by both fork entry points, then one launch per group of up to
// FORK_MAX_LAYERS layers (each launch derives the same tables from the inputs).
gr_status_t fork_launch(const int32_t* parent, int num_reqs, int beam_width, const int32_t* bt_in,
                        const int32_t* len_in, int32_t* bt_out, int32_t* len_out, int bt_stride, int num_layers,
                        void* const* k_caches, void* const* v_caches, int64_t num_blocks, int64_t kv_block_stride,
                        int64_t kv_tok_stride, int64_t kv_head_stride, const void* k_new, const void* v_new,
                        int64_t new_tok_stride, int num_kv_heads, int head_dim, int block_size, int dtype,
                        int32_t* dev_status, hipStream_t stream) {
  if (!cache_dtype_valid(dtype) || num_reqs < 0 || beam_width < 1 || bt_stride < 1 || num_layers < 1)
    return GR_ERR_INVALID_ARG;
  if (beam_width > FORK_MAX_W) return GR_ERR_UNSUPPORTED;
  if (!k_caches || !v_caches) return GR_ERR_INVALID_ARG;
  if (num_reqs == 0) return GR_OK;
  if (!parent || !bt_in || !len_in || !bt_out || !len_out) return GR_ERR_INVALID_ARG;
  if (bt_in == bt_out || len_in == len_out) return GR_ERR_INVALID_ARG;  // tables are written out of place
  if ((k_new == nullptr) != (v_new == nullptr)) return GR_ERR_INVALID_ARG;
  if (k_new && num_layers != 1) return GR_ERR_INVALID_ARG;  // the fused append is per layer
  for (int l = 0; l < num_layers; ++l) {
    KvGeom gl = make_geom(k_caches[l], v_caches[l], num_blocks, kv_block_stride, kv_tok_stride, kv_head_stride,
                          num_kv_heads, head_dim, block_size, dtype);
    const gr_status_t st = check_geom(gl);
    if (st != GR_OK) return st;
  }
  if (k_new && (!aligned16(k_new) || !aligned16(v_new) || (new_tok_stride * dtype_size(dtype)) % 16 ||
                new_tok_stride < (int64_t)num_kv_heads * head_dim))
    return GR_ERR_INVALID_ARG;
  if ((int64_t)num_reqs * beam_width > INT32_MAX) return GR_ERR_INVALID_ARG;
  const size_t lds = sizeof(int) * (size_t)fork_lds_ints(beam_width, bt_stride);
  // children per workgroup: two when the width allows and both appended
  // tokens fit one 16-byte vector per thread (half the workgroups to launch,
  // half the plans worked out)
  const int tv = num_kv_heads * (head_dim * dtype_size(dtype) / 16);
  const int cpw = beam_width % 2 == 0 && 2 * tv <= FORK_THREADS ? 2 : 1;
  for (int l0 = 0; l0 < num_layers; l0 += FORK_MAX_LAYERS) {
    const int L = std::min(FORK_MAX_LAYERS, num_layers - l0);
    KvLayers layers{};
    for (int l = 0; l < L; ++l) {
      layers.k[l] = static_cast<uint8_t*>(k_caches[l0 + l]);
      layers.v[l] = static_cast<uint8_t*>(v_caches[l0 + l]);
    }
    const KvGeom g = make_geom(k_caches[l0], v_caches[l0], num_blocks, kv_block_stride, kv_tok_stride,
                               kv_head_stride, num_kv_heads, head_dim, block_size, dtype);
    const dim3 grid((unsigned)(num_reqs * (beam_width / cpw)));
    if (num_layers == 1)
      hipLaunchKernelGGL(beam_fork<false>, grid, dim3(FORK_THREADS), lds, stream, parent, num_reqs, beam_width, cpw,
                         bt_in, len_in, bt_out, len_out, bt_stride, g, L, layers, static_cast<const uint8_t*>(k_new),
                         static_cast<const uint8_t*>(v_new), new_tok_stride, dev_status);
    else
      hipLaunchKernelGGL(beam_fork<true>, grid, dim3(FORK_THREADS), lds, stream, parent, num_reqs, beam_width, cpw,
                         bt_in, len_in, bt_out, len_out, bt_stride, g, L, layers, static_cast<const uint8_t*>(k_new),
                         static_cast<const uint8_t*>(v_new), new_tok_stride, dev_status);
    const gr_status_t st = launch_status();
    if (st != GR_OK) return st;
  }
  return GR_OK;
}

}  // namespace
}  // namespace gr

extern "C" gr_status_t gr_beam_kv_fork(const int32_t* parent, int num_reqs, int beam_width,
                                       const int32_t* bt_in, const int32_t* len_in, int32_t* bt_out,
                                       int32_t* len_out, int bt_stride, void* k_cache, void* v_cache,
                                       int64_t num_blocks, int64_t kv_block_stride, int64_t kv_tok_stride,
                                       int64_t kv_head_stride, const void* k_new, const void* v_new,
                                       int64_t new_tok_stride, int num_kv_heads, int head_dim,
                                       int block_size, int dtype, int32_t* dev_status, hipStream_t stream) {
  void* kc[1] = {k_cache};
  void* vc[1] = {v_cache};
  return fork_launch(parent, num_reqs, beam_width, bt_in, len_in, bt_out, len_out, bt_stride, 1, kc, vc, num_blocks,
                     kv_block_stride, kv_tok_stride, kv_head_stride, k_new, v_new, new_tok_stride, num_kv_heads,
                     head_dim, block_size, dtype, dev_status, stream);
}

extern "C" gr_status_t gr_beam_kv_fork_layers(const int32_t* parent, int num_reqs, int beam_width,
                                              const int32_t* bt_in, const int32_t* len_in, int32_t* bt_out,
                                              int32_t* len_out, int bt_stride, int num_layers,
                                              void* const* k_caches, void* const* v_caches, int64_t num_blocks,
                                              int64_t kv_block_stride, int64_t kv_tok_stride,
                                              int64_t kv_head_stride, int num_kv_heads, int head_dim,
                                              int block_size, int dtype, int32_t* dev_status, hipStream_t stream) {
  return fork_launch(parent, num_reqs, beam_width, bt_in, len_in, bt_out, len_out, bt_stride, num_layers, k_caches,
                     v_caches, num_blocks, kv_block_stride, kv_tok_stride, kv_head_stride, nullptr, nullptr, 0,
                     num_kv_heads, head_dim, block_size, dtype, dev_status, stream);
}

extern "C" gr_status_t gr_beam_kv_append(const void* k_new, const void* v_new, int64_t new_tok_stride,
                                         void* k_cache, void* v_cache, int64_t num_blocks,
                                         int64_t kv_block_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
                                         const int32_t* suffix_bt, int bt_stride, int32_t* suffix_len,
                                         int num_beams, int num_kv_heads, int head_dim, int block_size, int dtype,
                                         int32_t* dev_status, hipStream_t stream) {
  if (!cache_dtype_valid(dtype) || num_beams < 0 || bt_stride < 1) return GR_ERR_INVALID_ARG;
  if (num_beams == 0) return GR_OK;
  if (!k_new || !v_new || !suffix_bt || !suffix_len) return GR_ERR_INVALID_ARG;
  KvGeom g = make_geom(k_cache, v_cache, num_blocks, kv_block_stride, kv_tok_stride, kv_head_stride,
                       num_kv_heads, head_dim, block_size, dtype);
  gr_status_t st = check_geom(g);
  if (st != GR_OK) return st;
  if (!aligned16(k_new) || !aligned16(v_new) || (new_tok_stride * g.esize) % 16 ||
      new_tok_stride < (int64_t)num_kv_heads * head_dim)
    return GR_ERR_INVALID_ARG;
  hipLaunchKernelGGL(beam_append, dim3((unsigned)num_beams), dim3(64), 0, stream,
                     static_cast<const uint8_t*>(k_new), static_cast<const uint8_t*>(v_new), new_tok_stride, g,
                     suffix_bt, bt_stride, suffix_len, num_beams, dev_status);
  return launch_status();
}

extern "C" gr_status_t gr_reshape_and_cache(const void* key, int64_t key_tok_stride, const void* value,
                                            int64_t value_tok_stride, void* k_cache, void* v_cache,
                                            int64_t num_blocks, int64_t kv_block_stride, int64_t kv_tok_stride,
                                            int64_t kv_head_stride, const int64_t* slot_mapping, int num_tokens,
                                            int num_kv_heads, int head_dim, int block_size, int dtype,
                                            int32_t* dev_status, hipStream_t stream) {
  if (!dtype_valid(dtype) || num_tokens < 0) return GR_ERR_INVALID_ARG;
  if (num_tokens == 0) return GR_OK;
  if (!key || !value || !slot_mapping) return GR_ERR_INVALID_ARG;
  KvGeom g = make_geom(k_cache, v_cache, num_blocks, kv_block_stride, kv_tok_stride, kv_head_stride,
                       num_kv_heads, head_dim, block_size, dtype);
  gr_status_t st = check_geom(g);
  if (st != GR_OK) return st;
  if (!aligned16(key) || !aligned16(value) || (key_tok_stride * g.esize) % 16 ||
      (value_tok_stride * g.esize) % 16 || key_tok_stride < (int64_t)num_kv_heads * head_dim ||
      value_tok_stride < (int64_t)num_kv_heads * head_dim)
    return GR_ERR_INVALID_ARG;
  hipLaunchKernelGGL(reshape_and_cache_k, dim3((unsigned)num_tokens), dim3(64), 0, stream,
                     static_cast<const uint8_t*>(key), key_tok_stride, static_cast<const uint8_t*>(value),
                     value_tok_stride, g, slot_mapping, num_tokens, dev_status);
  return launch_status();
}

extern "C" gr_status_t gr_reshape_and_cache_fp8(const void* key, int64_t key_tok_stride, const void* value,
                                                int64_t value_tok_stride, void* k_cache, void* v_cache,
                                                int64_t num_blocks, int64_t kv_block_stride, int64_t kv_tok_stride,
                                                int64_t kv_head_stride, const int64_t* slot_mapping,
                                                int num_tokens, int num_kv_heads, int head_dim, int block_size,
                                                int dtype, const float* k_scale, const float* v_scale,
                                                int32_t* dev_status, hipStream_t stream) {
  if (!dtype_valid(dtype) || num_tokens < 0) return GR_ERR_INVALID_ARG;
  if (num_tokens == 0) return GR_OK;
  if (!key || !value || !slot_mapping) return GR_ERR_INVALID_ARG;
  KvGeom g = make_geom(k_cache, v_cache, num_blocks, kv_block_stride, kv_tok_stride, kv_head_stride,
                       num_kv_heads, head_dim, block_size, GR_DTYPE_FP8_E4M3);
  gr_status_t st = check_geom(g);  // cache rows 16-byte aligned: head_dim a multiple of 16
  if (st != GR_OK) return st;
  if (key_tok_stride < (int64_t)num_kv_heads * head_dim || value_tok_stride < (int64_t)num_kv_heads * head_dim)
    return GR_ERR_INVALID_ARG;
  switch (dtype) {
    case GR_DTYPE_F32:
      hipLaunchKernelGGL((reshape_and_cache_fp8_k<GR_DTYPE_F32>), dim3((unsigned)num_tokens), dim3(256), 0, stream,
                         key, key_tok_stride, value, value_tok_stride, g, slot_mapping, num_tokens, k_scale,
                         v_scale, dev_status);
      break;
    case GR_DTYPE_F16:
      hipLaunchKernelGGL((reshape_and_cache_fp8_k<GR_DTYPE_F16>), dim3((unsigned)num_tokens), dim3(256), 0, stream,
                         key, key_tok_stride, value, value_tok_stride, g, slot_mapping, num_tokens, k_scale,
                         v_scale, dev_status);
      break;
    default:
      hipLaunchKernelGGL((reshape_and_cache_fp8_k<GR_DTYPE_BF16>), dim3((unsigned)num_tokens), dim3(256), 0, stream,
                         key, key_tok_stride, value, value_tok_stride, g, slot_mapping, num_tokens, k_scale,
                         v_scale, dev_status);
      break;
  }
  return launch_status();
}

extern "C" const char* gr_status_string(gr_status_t s) {
  switch (s) {
    case GR_OK: return "ok";
    case GR_ERR_INVALID_ARG: return "invalid argument";
    case GR_ERR_UNSUPPORTED: return "unsupported configuration";
    case GR_ERR_LAUNCH: return "kernel launch failed";
    case GR_ERR_WORKSPACE: return "workspace missing or too small";
    default: return "unknown status";
  }
}

extern "C" int gr_version(void) { return GR_VERSION_CODE; }
