// BeamAttention decode on gfx950 matrix cores (bf16/fp16, head_dim 128).
//
// Work decomposition.  For request r and KV head h the query rows of all its
// beams form one dense M x 128 matrix (M = beams * q_per_beam * GQA group):
// the shared prefix contraction is a plain GEMM-shaped problem, which is why
// it runs on MFMA.  A workgroup owns 128 of those rows (8 waves: 4 row groups
// of 32 rows x 2 key halves, two waves per SIMD so one wave's matrix work
// overlaps the other's softmax and loads) and streams the request's prefix
// K/V through LDS in 64-key super-tiles, each loaded once for all 128 rows,
// straight from global memory into LDS (global_load_lds_dwordx4: no register
// staging, no LDS store instructions) two tiles ahead of the one computed.
// Workgroups that share (r, h) are placed on the same XCD (blockIdx % 8 is
// the XCD under round-robin dispatch) so their prefix re-reads hit that
// XCD's L2.  Each beam's short suffix is read from its own paged blocks into
// masked 32-key tiles after the prefix, with the same online softmax; the two
// waves of a row group (two partial states) are merged in LDS at the end.
// One launch, no gather/merge passes over HBM (contrast beam_attn.py:656-699).
//
// MFMA formulation and tile layouts: gr_mfma_tile.h.
#include <algorithm>

#include "gr_mfma_tile.h"

namespace gr {
namespace {

constexpr int MF_THREADS = 512;
constexpr int MF_ROWS = 128;   // query rows per workgroup
constexpr int PBT_WIN = 2048;  // prefix block-table entries staged in LDS
constexpr int NBUF = 4;        // tile buffers: prefix tile t in buffer t % 4 (V of t and K of t+1 read during
                               // step t while tiles t+2 and t+3 land); a suffix tile pair takes all four
constexpr int LOADS_PER_TILE = 4;  // direct-to-LDS loads each wave issues per prefix tile
constexpr int SB_STAGE = 2;    // suffix block ids staged in LDS per beam (more are read from HBM)

// Workgroup barrier once this wave's LDS reads are done and all but its newest
// INFLIGHT direct-to-LDS tile loads have landed (the compiler does not see
// those loads: the count is explicit).
template <int INFLIGHT>
__device__ inline void tile_barrier() {
  static_assert(INFLIGHT == 0 || INFLIGHT == 2 || INFLIGHT == LOADS_PER_TILE, "one tile in flight at most");
  if constexpr (INFLIGHT == LOADS_PER_TILE) __asm__ volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else if constexpr (INFLIGHT == 2) __asm__ volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}


// PREFILL: the varlen causal mode (gr_paged_attn_prefill).  The argument
// block is read as: prefix_bt = block table, prefix_len = sequence length,
// beam_start = query start per request, num_beams = query tokens, T = the
// largest query count; a request's rows are its query tokens x GQA group,
// query i sees keys 0 .. seq - ql + i, all read through the prefix machinery
// (fully visible tiles pipelined, the causal edge masked per row), no suffix.
// SPLIT: a.nsplit workgroups per row tile, each over a contiguous share of
// the prefix's 64-key tiles (the last one also takes the suffix), writing its
// normalised partial O (in the query dtype, as the two passes of a cascade
// hand over their outputs) and fp32 LSE to the workspace; split_merge
// combines them in fp32.
// OPT (decode only): a left window and/or ALiBi.  Window a.win_left >= 0:
// row r sees key k iff k >= qpos_r - win_left, qpos_r its query token's index
// in [prefix ; suffix]; the prefix range starts at the first tile any row can
// see, its first tiles (up to the WG's highest lower bound) take masked
// steps, the rest the fast loop.  ALiBi (a.alibi): each weight's exponent
// gains slope * (k - qpos_r) (log2 units: times log2 e), a linear function
// of the key in each tile (LinBias); the softmax reference follows the raw
// scores.  Sinks (a.sinks, any mode) join each row's softmax in the epilogue
// (in split_merge for the split mode).
// KV8: the caches hold OCP e4m3 bytes (read as e4m3 * k_scale / v_scale).
// Tiles land as bytes in a three-slot staging ring after three tile buffers;
// each wave converts the rows it loaded into a tile buffer one step ahead of
// their use, so the matrix-core steps read bf16 / fp16 tiles as usual.  The K
// scale folds into the softmax constant, the V scale into the output.
// PAIR: head_dim 64 as pairs of adjacent KV heads (a.pair; see mfma_pair_args).
template <int DT, bool SOFTCAP, bool PREFILL = false, bool SPLIT = false, bool OPT = false, bool KV8 = false,
          bool PAIR = false>
__global__ __launch_bounds__(MF_THREADS, 1) void decode_mfma(DecodeArgs a, int units, int mtiles) {
  static_assert(!(PAIR && SPLIT), "head pairs are never split");
  constexpr int NB = KV8 ? 3 : NBUF;       // tile buffers
  constexpr int STG = 16384;               // bytes per fp8 staging slot: 64 rows x 128 B of K, then of V
  __shared__ __attribute__((aligned(1024))) uint16_t lds[KV8 ? 3 * BUF + 3 * STG / 2 : NBUF * BUF];
  __shared__ int suf_cum[4][34];         // per row group: cumulative suffix lengths of its beams
  __shared__ int suf_info[2][4][32];     // per suffix tile and row group slot: (beam << 16) | j, or -1
  __shared__ int suf_s0[4][32];          // per row group beam: first suffix position
  __shared__ int suf_blk[4][32][SB_STAGE];  // per row group beam: its first suffix block ids
  __shared__ int64_t suf_off[4][64];     // per row group: element offset of its first 64 suffix slots (-1: none)
  __shared__ int suf_tab_bad[4];         // per row group: its slot table is not built (unstaged block ids)
  __shared__ int pbt_s[PBT_WIN];         // staged prefix block ids (-1 = invalid)
  __shared__ int hot_flag;               // a tile of the fast loop needed the exact path
  __shared__ int win_hi[8];              // per wave: the highest window lower bound of its rows

  // the arguments' five scalar-cache lines at once (DecodeArgs, units, mtiles)
  kernarg_lines<kernarg_line_count<DecodeArgs>(8)>();
  // ---- XCD-aware tile placement: all m-tiles of a (request, KV head) land on
  // the same XCD (round-robin dispatch puts workgroup i on XCD i % 8)
  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  // prefill: tile rank is the slow index and runs last-token-first, so every
  // (request, head)'s longest causal range is dispatched in the first wave
  const int ugroups = (units + 7) >> 3;
  // split: the splits of a row tile are adjacent in dispatch order, on one XCD
  const int nsplit = SPLIT ? a.nsplit : 1;
  const int split = SPLIT ? local % nsplit : 0;
  const int lt = SPLIT ? local / nsplit : local;
  const int unit = PREFILL ? (lt % ugroups) * 8 + xcd : (lt / mtiles) * 8 + xcd;
  const int mt = PREFILL ? mtiles - 1 - lt / ugroups : lt % mtiles;
  if (unit >= units) return;
  const int r = unit / a.Hkv, hk = unit % a.Hkv;
  const int G = a.Hq / a.Hkv;
  const int tid = threadIdx.x;
  // ---- prologue, two memory round trips.  First the reads that need only the
  // arguments -- the request's beam range, its prefix length and the first
  // window of its prefix block table; then, with the window staged in LDS, the
  // suffix metadata, Q and the first two prefix tiles, all in flight together.
  const int32_t* pbt = a.prefix_bt + (int64_t)r * a.prefix_bt_stride;
  constexpr int WIN_PER_THREAD = PBT_WIN / MF_THREADS;
  static_assert(PBT_WIN % MF_THREADS == 0, "window split");
  // (prologue loads are branch-free -- an unused lane reads a zero source --
  // so the compiler's wait counts stay exact and later loads stay in flight)
  const int* zint = reinterpret_cast<const int*>(g_zero16);
  int raw_blk[WIN_PER_THREAD];
#pragma unroll
  for (int i = 0; i < WIN_PER_THREAD; ++i) {
    const int bi = tid + i * MF_THREADS;
    raw_blk[i] = *(bi < a.prefix_bt_stride ? pbt + bi : zint);
  }
  const int P_arg = PREFILL ? 0 : a.prefix_len[r];
  __asm__ volatile("" ::"s"(P_arg));  // read with the beam range, not after its checks
  const int nb0 = a.beam_start[r];  // prefill: first query token of the request
  int W, TG, rows_r, ctx = 0;
  if constexpr (PREFILL) {
    const int ql = a.beam_start[r + 1] - nb0;
    const int seq = a.prefix_len[r];
    ctx = seq - ql;  // keys before the request's first query token
    if (nb0 < 0 || ql < 0 || nb0 + ql > a.num_beams || ql > a.T || ctx < 0 ||
        seq > a.prefix_bt_stride * a.bs) {
      if (threadIdx.x == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
      return;
    }
    W = 1;
    TG = G;
    rows_r = ql * G;
  } else {
    W = a.beam_start[r + 1] - nb0;
    TG = a.T * G;
    rows_r = W * TG;
    // beam_start is device data: never trust it (a request past max_beams
    // would leave rows no workgroup computes)
    if (nb0 < 0 || W < 0 || nb0 + W > a.num_beams || W > a.max_beams) {
      if (threadIdx.x == 0 && mt == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
      return;
    }
  }
  const int row_base = mt * MF_ROWS;
  if (row_base >= rows_r) return;

  const int wave = tid >> 6, lane = tid & 63;
  const int rg = wave >> 1, ks = wave & 1;  // row group (32 rows), key half
  const int lrow = lane & 31, lhalf = lane >> 5;
  using S = uint16_t;
  const S* qp = static_cast<const S*>(a.q);
  const S* kc = static_cast<const S*>(a.k_cache);
  const S* vc = static_cast<const S*>(a.v_cache);
  const int64_t head_off = (int64_t)hk * a.kv_head_stride;

  // ---- Q fragments (B operand of S^T): this lane's query row ----
  const int my_rho = row_base + rg * 32 + lrow;
  const bool row_ok = my_rho < rows_r;
  const int my_b = PREFILL ? 0 : my_rho / TG;
  const int my_qi = PREFILL ? my_rho / G : (my_rho / G) % a.T, my_g = my_rho % G;
  const int64_t my_tok = PREFILL ? (int64_t)(nb0 + my_qi) : (int64_t)((nb0 + my_b) * a.T + my_qi);
  u32x4_t qf[8];
  // an fp8 cache's K scale multiplies every score: it folds into c
  const float ksc = KV8 && a.k_scale ? a.k_scale[0] : 1.f;
  const float vsc = KV8 && a.v_scale ? a.v_scale[0] : 1.f;
  const float c = (SOFTCAP ? a.scale / a.softcap : a.scale * LOG2E) * ksc;
  const float cap = a.softcap;

  f32x16_t o[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) o[mb] = f32x16_t{};
  RowState st = {-INFINITY, 0.f};

  const int pre_cap = a.prefix_bt_stride * a.bs;
  // prefill: the workgroup reads keys up to its last query token's
  int P = PREFILL ? ctx + (min(row_base + MF_ROWS, rows_r) - 1) / G + 1 : P_arg;
  if (P < 0 || P > pre_cap) {
    if (tid == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
    P = P < 0 ? 0 : pre_cap;
  }
  const int n_all = (P + ST_KEYS - 1) / ST_KEYS;
  // window: no row sees keys below P - T - win_left (its query sits at P - T or later)
  const int wl = OPT ? a.win_left : -1;
  const int tw0 = wl >= 0 ? max(0, P - a.T - wl) / ST_KEYS : 0;
  const int n_rng = n_all - tw0;
  // split: the last split also runs the suffix phase (about three prefix
  // steps), so the others share up to three of its tiles
  const int sb = SPLIT ? min(3, n_rng / (2 * nsplit)) : 0;
  auto split_bound = [&](int s) {
    return s >= nsplit ? n_rng : min(n_rng, s * (n_rng + sb) / nsplit);  // < 2^30: n_rng < 2^25, s <= 16
  };
  const int ts0 = tw0 + (SPLIT ? split_bound(split) : 0);  // first tile of this workgroup
  const int n_st = SPLIT ? tw0 + split_bound(split + 1) - ts0 : n_rng;
  const int kb = ts0 * ST_KEYS;  // first key of this workgroup's prefix range
  const int bsh = a.bs_shift;

  // The request's prefix block-table row is staged in LDS (a window of
  // PBT_WIN entries), validated once; invalid ids become -1 and read as zeros.
  // Tile loads then need no dependent global reads and no atomics.
  const int nblk = (P + a.bs - 1) >> bsh;
  int win0 = 0;
  auto load_window = [&](int w0) {
    for (int i = tid; i < PBT_WIN; i += MF_THREADS) {
      const int bi = w0 + i;
      int blk = -1;
      if (bi < nblk) {
        blk = pbt[bi];
        if (blk < 0 || blk >= a.num_blocks) {
          flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
          blk = -1;
        }
      }
      pbt_s[i] = blk;
    }
  };
  int bad_blk = 0;
#pragma unroll
  for (int i = 0; i < WIN_PER_THREAD; ++i) {
    const int bi = tid + i * MF_THREADS;
    int blk = -1;
    if (bi < nblk) {
      blk = tid + i * MF_THREADS < a.prefix_bt_stride ? raw_blk[i] : -1;
      if (blk < 0 || blk >= a.num_blocks) {
        flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
        blk = -1;
        bad_blk = 1;
      }
    }
    pbt_s[tid + i * MF_THREADS] = blk;
  }
  if (tid == 0) hot_flag = 0;
  // a flagged block id in the first window: its keys read the zero source,
  // which only the general tile loads do (the lean loads below assume none)
  const bool win_bad = __syncthreads_or(bad_blk) != 0;

  // keep the window over [k0, k0 + 64); switching costs two barriers and
  // happens once per PBT_WIN blocks
  auto ensure_window = [&](int k0) {
    const int last = min(k0 + ST_KEYS, P) - 1;
    if ((k0 >> bsh) < win0 || (last >> bsh) >= win0 + PBT_WIN) {
      __syncthreads();
      win0 = k0 >> bsh;
      load_window(win0);
      __syncthreads();
    }
  };
  // zero source of loads past the prefix or the suffix
  const S* zsrc = reinterpret_cast<const S*>(g_zero16);
  // ---- prefix tile loads, straight from global memory into LDS
  // (global_load_lds_dwordx4: no registers, no LDS store instructions).  Wave
  // wv moves rows 8 wv .. 8 wv + 7 of a tile's K and of its V, four rows (1 KB
  // of LDS) per instruction: lane i lands on row 8 wv + 4 j + (i >> 4),
  // physical chunk i & 15, and fetches the logical chunk the swizzles put
  // there.  Four rows never straddle a block (power-of-two block size >= 4),
  // so each instruction has one wave-uniform base address.  Every wave issues
  // exactly LOADS_PER_TILE loads per tile, tiles in order: the waits count on it.
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4, pch = lane & 15;
  const int ck = pch ^ (q4 | ((wv & 1) << 2));          // kchunk of rows 8 wv + 4 j + q4
  const int cv = (((pch >> 2) ^ q4) << 2) | (pch & 3);  // vchunk of the same rows
  const int64_t tok = a.kv_tok_stride;
  const uint32_t vo_k = (uint32_t)((q4 * tok + ck * 8) * 2);
  const uint32_t vo_v = (uint32_t)((q4 * tok + cv * 8) * 2);
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(lds);
  const uint32_t blk_stride = (uint32_t)a.kv_block_stride;
  // Prefix tile t of this workgroup's range into buffer buf: the wave-uniform
  // addresses of its four loads (prep_tile, which may move the block-table
  // window), then the loads one at a time (issue_load n: K of rows 8 wv + 4 j,
  // then their V, j = n >> 1).  Rows of an invalid block (flagged when the
  // window was staged) and rows past the prefix read the zero source.
  struct TileLoads {
    int64_t el[2];  // element offset of rows 8 wv + 4 j in the K and V caches
    int key[2], blk[2];
    uint32_t dst;  // LDS byte address of the wave's first K row
  };
  auto prep_tile = [&](int t, int buf) {
    const int k0 = kb + t * ST_KEYS;
    ensure_window(k0);
    TileLoads L;
    L.dst = lds0 + (uint32_t)(buf * BUF * 2) + (uint32_t)(wv * 8 * KS_PITCH * 2);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int key = k0 + 8 * wv + 4 * j;
      const int blk = __builtin_amdgcn_readfirstlane(key < P ? pbt_s[(key >> bsh) - win0] : -1);
      L.key[j] = key;
      L.blk[j] = blk;
      L.el[j] = (int64_t)((uint64_t)(uint32_t)max(blk, 0) * blk_stride) + (int64_t)(key & (a.bs - 1)) * tok + head_off;
    }
    return L;
  };
  auto issue_load = [&](const TileLoads& L, int n) {
    const int j = n >> 1;
    const bool isv = n & 1;
    const uint32_t d = L.dst + (isv ? K_TILE * 2 : 0) + j * 1024;
    const S* base = (isv ? vc : kc) + L.el[j];
    if (L.key[j] + 4 <= P && L.blk[j] >= 0) {
      dma_s(d, base, isv ? vo_v : vo_k);
    } else {
      const bool ok = L.blk[j] >= 0 && L.key[j] + q4 < P;
      dma_v(d, ok ? base + q4 * tok + (isv ? cv : ck) * 8 : zsrc);
    }
  };
  auto issue_tile = [&](int t, int buf) {
    const TileLoads L = prep_tile(t, buf);
#pragma unroll
    for (int n = 0; n < LOADS_PER_TILE; ++n) issue_load(L, n);
  };
  // second round trip: suffix metadata (needed first, by the slot table), Q,
  // then the first two tiles.  Suffix metadata: lane l < nbeams of the
  // key-half-0 wave of row group rg owns beam b_lo + l of the group.
  const int suf_cap = a.suffix_bt_stride * a.bs;
  const int rlo = row_base + rg * 32;
  const int b_lo = rlo / TG;
  const int nbeams = !PREFILL && rlo < rows_r ? min((rlo + 31) / TG, W - 1) - b_lo + 1 : 0;  // <= 32
  const bool meta_lane = ks == 0 && lane < nbeams;
  int sL, sS0, sBlk[SB_STAGE];
  {
    const int n = nb0 + b_lo + lane;
    sL = *(meta_lane ? a.suffix_len + n : zint);
    sS0 = *(meta_lane && a.suffix_start ? a.suffix_start + n : zint);
#pragma unroll
    for (int j = 0; j < SB_STAGE; ++j)
      sBlk[j] = *(meta_lane && j < a.suffix_bt_stride ? a.suffix_bt + (int64_t)n * a.suffix_bt_stride + j : zint);
  }
  const int my_len = *(!PREFILL && row_ok ? a.suffix_len + nb0 + my_b : zint);  // this lane's beam (causal limit)
  __builtin_amdgcn_sched_barrier(0);  // the metadata loads stay first: the slot table waits only for them
  {
    // head pairs: query head hq's 64 dims fill dims [64 half, 64 half + 64),
    // half = which KV head of the pair it reads; the other half stays zero
    const int hq = hk * G + my_g, half = PAIR ? my_g / (G >> 1) : 0;
    const S* src = qp + my_tok * a.q_tok_stride + (int64_t)hq * (PAIR ? HD / 2 : HD) + lhalf * 8 -
                   (PAIR ? half * (HD / 2) : 0);
    const S* zq = reinterpret_cast<const S*>(g_zero16);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[kk] = *reinterpret_cast<const u32x4_t*>(row_ok && (!PAIR || (kk >> 2) == half) ? src + kk * 16 : zq);
  }
  // ALiBi: this lane's row's slope (log2 units), read with Q
  const float alpha = OPT && a.alibi ? *(row_ok ? a.alibi + hk * G + my_g : reinterpret_cast<const float*>(zint)) * LOG2E
                                     : 0.f;

  // Lean loads of the loop's full tiles.  When every block id of the range sits
  // in the first staged window (which then never moves), a block holds at
  // least 8 keys (rows 8 wv .. 8 wv + 7 of a tile share one block) and the
  // range has at most 64 tiles, and no block id of the window was flagged,
  // lane t of toff_lo / toff_hi holds the byte offset of tile t's rows of this
  // wave: a tile's four loads then take two lane reads and scalar address
  // arithmetic, with no LDS round trip and no window check.  They move
  // exactly what issue_tile moves.
  const int k_end = min(kb + n_st * ST_KEYS, P);
  const bool lean = !win_bad && n_st <= 64 && a.bs >= 8 && (n_st == 0 || ((k_end - 1) >> bsh) < PBT_WIN);
  const bool last_full = kb + n_st * ST_KEYS <= P;
  // lane t: byte offset of tile t's rows 8 wv .. from the head's K (and V) base
  uint32_t toff_lo = 0, toff_hi = 0;
  {
    const int key = kb + lane * ST_KEYS + 8 * wv;
    if (lean && lane < n_st && key < P) {
      const int blk = max(pbt_s[key >> bsh], 0);
      const uint64_t e = (uint64_t)(uint32_t)blk * blk_stride + (uint64_t)(uint32_t)(key & (a.bs - 1)) * (uint64_t)tok;
      const uint64_t eb = KV8 ? e : e << 1;  // bytes
      toff_lo = (uint32_t)eb;
      toff_hi = (uint32_t)(eb >> 32);
    }
  }
  const char* kc_h = reinterpret_cast<const char*>(kc + head_off);
  const char* vc_h = reinterpret_cast<const char*>(vc + head_off);
  const uint32_t tok4b = (uint32_t)(8 * tok);  // bytes of four token rows
  const uint32_t dst_w = lds0 + (uint32_t)(wv * 8 * KS_PITCH * 2);
  auto issue_tile_lean = [&](int t, int buf) {
    const uint64_t toff = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)toff_hi, t) << 32) |
                         (uint32_t)__builtin_amdgcn_readlane((int)toff_lo, t);
    const char* kb0 = kc_h + toff;
    const char* vb0 = vc_h + toff;
    const uint32_t d = dst_w + (uint32_t)(buf * BUF * 2);
    const uint32_t dst[4] = {d, d + K_TILE * 2, d + 1024, d + K_TILE * 2 + 1024};
    const void* const src[4] = {kb0, vb0, kb0 + tok4b, vb0 + tok4b};
    const uint32_t off[4] = {vo_k, vo_v, vo_k, vo_v};
    dma_s4(dst, src, off);
  };
  // a prologue tile into its own buffer: lean when it can be
  auto issue_first = [&](int t) {
    if (lean && (t + 1 < n_st || last_full)) issue_tile_lean(t, t);
    else issue_tile(t, t);
  };
  // fp8: tile t's bytes into staging slot `slot`, this wave's rows 8 wv .. 8 wv
  // + 7 of K and of V (lane i: row 8 wv + (i >> 3), 16-byte chunk i & 7), one
  // 1 KB load each; lean tiles from the lane offsets, others row by row
  // through the staged window (rows past the prefix or in an invalid block
  // read the zero source)
  const uint8_t* kc8 = static_cast<const uint8_t*>(a.k_cache);
  const uint8_t* vc8 = static_cast<const uint8_t*>(a.v_cache);
  const int r8 = lane >> 3, c8 = lane & 7;
  const uint32_t vo8 = (uint32_t)(r8 * tok + c8 * 16);
  const uint32_t stg_w = lds0 + (uint32_t)(3 * BUF * 2) + (uint32_t)(wv * 1024);
  auto dma8 = [&](int t, int slot) {
    const uint32_t d = stg_w + (uint32_t)(slot * STG);
    if (lean && (t + 1 < n_st || last_full)) {
      const uint64_t toff = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)toff_hi, t) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)toff_lo, t);
      dma_s(d, kc8 + head_off + toff, vo8);
      dma_s(d + 8192, vc8 + head_off + toff, vo8);
    } else {
      const int k0 = kb + t * ST_KEYS;
      ensure_window(k0);
      const int key = k0 + 8 * wv + r8;
      const int blk = key < P ? pbt_s[(key >> bsh) - win0] : -1;
      const int64_t off = (int64_t)((uint64_t)(uint32_t)max(blk, 0) * blk_stride) + (int64_t)(key & (a.bs - 1)) * tok +
                          head_off + c8 * 16;
      const bool ok = key < P && blk >= 0;
      dma_v(d, ok ? (const void*)(kc8 + off) : (const void*)zsrc);
      dma_v(d + 8192, ok ? (const void*)(vc8 + off) : (const void*)zsrc);
    }
  };
  // fp8: this wave's rows of staging slot `slot` as bf16 / fp16 into tile
  // buffer `buf`, in the swizzled layouts the fragment reads expect
  auto convert8 = [&](int slot, int buf) {
    const uint8_t* st8 = reinterpret_cast<const uint8_t*>(lds) + 3 * BUF * 2 + slot * STG;
    const int row = 8 * wv + r8;
    const u32x4_t rk = *reinterpret_cast<const u32x4_t*>(st8 + row * 128 + c8 * 16);
    const u32x4_t rv = *reinterpret_cast<const u32x4_t*>(st8 + 8192 + row * 128 + c8 * 16);
    uint16_t* bk = lds + buf * BUF + row * KS_PITCH;
    uint16_t* bvv = lds + buf * BUF + K_TILE + row * VS_PITCH;
    *reinterpret_cast<u32x4_t*>(bk + kchunk(row, 2 * c8) * 8) = Fp8Cvt<DT>::x8(rk[0], rk[1]);
    *reinterpret_cast<u32x4_t*>(bk + kchunk(row, 2 * c8 + 1) * 8) = Fp8Cvt<DT>::x8(rk[2], rk[3]);
    *reinterpret_cast<u32x4_t*>(bvv + vchunk(row, 2 * c8) * 8) = Fp8Cvt<DT>::x8(rv[0], rv[1]);
    *reinterpret_cast<u32x4_t*>(bvv + vchunk(row, 2 * c8 + 1) * 8) = Fp8Cvt<DT>::x8(rv[2], rv[3]);
  };
  // the first tiles: bf16 / fp16 tiles 0 and 1 into buffers 0 and 1; fp8
  // tiles 0, 1, 2 into staging slots 0, 1, 2 (0 and 1 converted below)
  if constexpr (KV8) {
    for (int t = 0; t < min(n_st, 3); ++t) dma8(t, t);
  } else {
    if (n_st > 0) issue_first(0);
    if (n_st > 1) issue_first(1);
  }
  int suf_len = 0, suf_incl = 0;  // this meta lane's validated suffix length, inclusive prefix sum
  if (ks == 0) {
    int len = 0;
    if (meta_lane) {
      len = (sL < 0 || sS0 < 0 || sS0 + sL > suf_cap) ? 0 : sL;
      if (len != sL) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
      suf_s0[rg][lane] = sS0;
#pragma unroll
      for (int j = 0; j < SB_STAGE; ++j) suf_blk[rg][lane][j] = j < a.suffix_bt_stride ? sBlk[j] : -1;
    }
    const int incl = wave_incl_scan<32>(len);  // inclusive scan over the first 32 lanes (and the last 32)
    if (lane < 32) suf_cum[rg][lane + 1] = incl;
    suf_len = len;
    suf_incl = incl;
    if (lane == 0) {
      suf_cum[rg][0] = 0;
      suf_cum[rg][33] = b_lo;  // first beam of the group
    }
  }
  // Slot table of each row group's first suffix tile pair (64 slots), built
  // while the first tiles' loads are in flight: the element offset of the
  // slot's token row (-1: empty or invalid block) and its tag (beam << 16 | j)
  // for the masks, so the suffix gathers need one LDS read per slot.  Only
  // the staged block ids are used (no memory reads here: a wait would also
  // wait for the tile loads); a group that needs others is flagged, and its
  // workgroup gathers the first pair the general way.
  if (!PREFILL && ks == 0) {
    const int tot = __shfl(suf_incl, 31, 64);
    const int c0 = suf_incl - suf_len;
    const int n_in = meta_lane && c0 < 64 ? min(suf_len, 64 - c0) : 0;
    const bool bad = __ballot(n_in > 0 && ((sS0 + n_in - 1) >> bsh) >= SB_STAGE) != 0;
    if (lane == 0) suf_tab_bad[rg] = bad ? 1 : 0;
    if (!bad && lane >= tot) {
      suf_off[rg][lane] = -1;
      suf_info[lane >> 5][rg][lane & 31] = -1;
    }
    if (!bad) {
      bool bad_blk = false;  // reported after the loop: a memory operation inside it makes the
                             // compiler wait for every load in flight before entering it
      for (int j = 0; j < n_in; ++j) {
        const int pos = sS0 + j;
        const int bi = pos >> bsh;
        int blk = -1;
#pragma unroll
        for (int q = 0; q < SB_STAGE; ++q) blk = bi == q && q < a.suffix_bt_stride ? sBlk[q] : blk;
        const bool ok = blk >= 0 && blk < a.num_blocks;
        bad_blk |= !ok;
        const int slot = c0 + j;
        suf_off[rg][slot] = ok ? (int64_t)blk * a.kv_block_stride + (int64_t)(pos & (a.bs - 1)) * a.kv_tok_stride + head_off : -1;
        suf_info[slot >> 5][rg][slot & 31] = ok ? ((b_lo + lane) << 16) | j : -1;
      }
      if (bad_blk) flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
    }
  }
  // Retire every prologue load (Q and the first two tiles) here, with a wait
  // the compiler sees: its own wait before the first read of qf would
  // otherwise be a full vector-memory wait placed after the next tile load.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  // window: this lane's row sees keys from lo_row on; the workgroup's highest
  // bound says how many of its first tiles need masks
  int lo_row = 0;
  // ALiBi: the bias of this lane's first key of a tile at key k0 is
  // alpha * (k0 + al_off) -- its keys sit at k0 + ks * 32 + 8 * lhalf + r'
  const int al_off = OPT ? ks * 32 + 8 * lhalf - (P + my_len - a.T + my_qi) : 0;
  if constexpr (OPT) {
    lo_row = wl >= 0 ? P + my_len - a.T + my_qi - wl : INT_MIN;
    int hi = row_ok ? lo_row : INT_MIN;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) hi = max(hi, __shfl_xor(hi, off, 64));
    if (lane == 0) win_hi[wave] = hi;
  }
  if constexpr (KV8) {
    if (n_st > 0) convert8(0, 0);
    if (n_st > 1) convert8(1, 1);
  }
  __syncthreads();
  int n_edge = 0;  // tiles [0, n_edge) of the range: some row's window starts inside or after them
  if constexpr (OPT) {
    int hi = win_hi[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) hi = max(hi, win_hi[w]);
    n_edge = hi > kb ? min(n_st, (int)(((int64_t)hi - kb + ST_KEYS - 1) / ST_KEYS)) : 0;
  }
  if constexpr (KV8) {
    if (n_st > 3) dma8(3, 0);  // into tile 0's slot, converted above
  } else {
    if (n_st > 2) issue_first(2);
  }
  f32x16_t s_cur = qk_half<DT>(lds, ks * 32, lane, qf);  // (stale LDS when n_st == 0: never used)
  // the exponent terms of prefix tile t's weights: ALiBi's linear bias, or none
  auto tb = [&](int t) {
    if constexpr (OPT) return LinBias{alpha, alpha * (float)(kb + t * ST_KEYS + al_off)};
    else return NoBias{};
  };
  // Suffix prefetch.  The first suffix tile pair (64 slots per row group: the
  // slot table's) is four pieces, piece i = 2 h + gp holding tile h of row
  // groups 2 gp and 2 gp + 1 (their 32 slots each, rows (g & 1) * 32 ..) in
  // buffer (n_st + i) % 4.  The last prefix steps free those buffers one by
  // one -- step t has no tile t + 3 to fetch once t + 3 >= n_st -- so pieces
  // 0, 1, 2 go out, as direct-to-LDS gathers of the slots' rows, at the tops
  // of steps n_st - 3, n_st - 2, n_st - 1, and piece 3 after the loop: the
  // gathers' latency hides behind the last prefix steps.
  int max_tot = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) max_tot = max(max_tot, suf_cum[g][32]);
  const int n_sit = PREFILL || (SPLIT && split != nsplit - 1) ? 0 : (max_tot + 31) / 32;
  const bool tab_ok = !(suf_tab_bad[0] | suf_tab_bad[1] | suf_tab_bad[2] | suf_tab_bad[3]);
  const int spf_n = !PREFILL && !KV8 && tab_ok && n_st >= 3 ? 2 * min(n_sit, 2) : 0;  // pieces prefetched
  const int sbase = n_st & 3;  // suffix tile h of row group g sits in buffer (sbase + 2 h + (g >> 1)) % 4
  auto suf_piece = [&](int i) {
    const int h = i >> 1, gp = i & 1;
    const uint32_t d = lds0 + (uint32_t)(((sbase + i) & 3) * BUF * 2) + (uint32_t)(wv * 8 * KS_PITCH * 2);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = 8 * wv + 4 * j + q4;  // row of the piece: group 2 gp + (row >> 5), slot row & 31
      const int64_t off = suf_off[2 * gp + (row >> 5)][h * 32 + (row & 31)];
      dma_v(d + j * 1024, off < 0 ? zsrc : kc + off + ck * 8);
      dma_v(d + K_TILE * 2 + j * 1024, off < 0 ? zsrc : vc + off + cv * 8);
    }
  };
  // One step over a fully visible tile `it` (not the last): consumes its S^T
  // from s_in, leaves that of tile it+1 in s_out.  Keys of an invalid block
  // read as zero rows (the block was flagged when the window was staged).
  // Tile t+3 goes out at the top of step t, into buffer (t+3) % 4: its
  // previous tile, t-1, was last read in step t-1, before the barrier that
  // ended it.
  // fp8: the top of step t converts tile t + 2 (staged since step t - 2) into
  // its buffer (tile t - 1's, read up to step t - 1) and loads tile t + 4 into
  // staging (tile t + 1's slot, converted in step t - 1).
  auto fetch_ahead = [&](int t) {
    if constexpr (KV8) {
      if (t + 2 < n_st) convert8((t + 2) % 3, (t + 2) % 3);
      if (t + 4 < n_st) dma8(t + 4, (t + 4) % 3);
      return;
    }
    const int tn = t + 3;
    if (tn < n_st) {
      if (lean && (tn + 1 < n_st || last_full)) issue_tile_lean(tn, tn % NB);
      else issue_tile(tn, tn % NB);
    } else if (tn - n_st < min(spf_n, 3)) {
      suf_piece(tn - n_st);
    }
  };
  // The end of step t: tile t+2 (read from the next step on) has landed; tile
  // t+3, or the suffix piece issued in its place, may still be in flight.
  auto step_barrier = [&](int t) {
    if constexpr (KV8) {  // tile t + 3's bytes (converted next step) have landed; t + 4's may not
      if (t + 4 < n_st) tile_barrier<2>();
      else tile_barrier<0>();
    } else {
      if (t + 3 < n_st || t + 3 - n_st < min(spf_n, 3)) tile_barrier<LOADS_PER_TILE>();
      else tile_barrier<0>();
    }
  };
  // (the step lambdas are forced inline: one left out of line -- the compiler
  // did that in the soft-capped prefill -- takes everything it captures by
  // reference, O and Q included, through a 1.7 KB per-lane stack in scratch)
  auto prefix_step = [&](int it, const f32x16_t& s_in, f32x16_t& s_out) __attribute__((always_inline)) {
    fetch_ahead(it);
    pipe_step<DT, SOFTCAP>(lds + (it % NB) * BUF, lds + ((it + 1) % NB) * BUF, ks * 32, lane, qf, s_in, s_out,
                           o, st, c, cap, tb(it));
    step_barrier(it);
  };
  // The last tile: no next tile; masked when only p_last of its keys exist.
  const int p_last = min(ST_KEYS, P - kb - (n_st - 1) * ST_KEYS);  // keys in the last tile (1 .. 64)
  auto last_step = [&](int it, const f32x16_t& s_in) __attribute__((always_inline)) {
    fetch_ahead(it);  // (a suffix piece, if any)
    // register r of lane half lhalf holds tile key ks*32 + 16*(r>>3) + 8*lhalf + (r&7)
    uint32_t v = 0;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) v |= (ks * 32 + 16 * (rr >> 3) + 8 * lhalf + (rr & 7) < p_last ? 1u : 0u) << rr;
    const uint32_t vis[1] = {v};
    const f32x16_t s1[1] = {s_in};
    u32x4_t pw[1][2];
    weights<DT, SOFTCAP, true, 1>(s1, vis, st, c, cap, pw, o, tb(it));
    pv<DT, 1>(lds + (it % NB) * BUF, ks * 32, lane, pw, o);
    __syncthreads();
  };
  f32x16_t s_alt;
  int it = 0;
  // Fully visible tiles run in a loop that never rescales O (a rescale in
  // the loop makes the compiler copy the accumulators every step).  The
  // workgroup's first tile (peeled: O is still zero) sets each row's
  // reference; a later tile with a score more than Rescale::THRESH above it --
  // never for ordinary inputs -- is only recorded, and the workgroup then
  // recomputes its prefix range exactly (after the masked tiles).
  bool hot_seen = false;
  u32x4_t p[1][2];
  auto finish_step = [&](int t) __attribute__((always_inline)) {
    phase_c1<DT>(lds + (t % NB) * BUF, ks * 32, lane, p, o);
    step_barrier(t);
  };
  // tile 0 (and S^T of tile 1): exact weights, O still zero
  auto peel = [&]() __attribute__((always_inline)) {
    fetch_ahead(0);
    phase_a1<DT, SOFTCAP>(lds + BUF, ks * 32, lane, qf, s_cur, s_alt, st, c, cap, p, tb(0));
    f32x16_t zo[4] = {};
    const uint32_t vis[1] = {0xFFFFu};
    const f32x16_t s1[1] = {s_cur};
    weights<DT, SOFTCAP, false, 1>(s1, vis, st, c, cap, p, zo, tb(0));
    finish_step(0);
    s_cur = s_alt;
    it = 1;
  };
  // One fast step over tile t (not the last): consumes its S^T from s_in and
  // leaves that of tile t+1 in s_out.  The exact-path test is deferred: each
  // lane records its own flag and the waves vote after the loop.
  auto fast_step = [&](int t, const f32x16_t& s_in, f32x16_t& s_out) __attribute__((always_inline)) {
    fetch_ahead(t);
    hot_seen |= phase_a1<DT, SOFTCAP, true>(lds + ((t + 1) % NB) * BUF, ks * 32, lane, qf, s_in, s_out, st, c, cap, p, tb(t));
    phase_c1<DT>(lds + (t % NB) * BUF, ks * 32, lane, p, o);
    step_barrier(t);
  };
  // The same step when tile t+3 exists and is full and the lean loads apply
  // (steps t < n_lean): no run-time choices.
  const int n_lean = !lean ? 0 : KV8 ? (last_full ? n_st - 4 : n_st - 5) : (last_full ? n_st - 3 : n_st - 4);
  auto lean_step = [&](int t, const f32x16_t& s_in, f32x16_t& s_out) __attribute__((always_inline)) {
    hot_seen |= phase_ac<DT, SOFTCAP>(lds + ((t + 1) % NB) * BUF, lds + (t % NB) * BUF, ks * 32, lane, qf, s_in,
                                      s_out, st, c, cap, o, [&]() {
                                        if constexpr (KV8) {
                                          convert8((t + 2) % 3, (t + 2) % 3);
                                          dma8(t + 4, (t + 4) % 3);
                                        } else {
                                          issue_tile_lean(t + 3, (t + 3) % NB);
                                        }
                                      }, tb(t));
    tile_barrier<KV8 ? 2 : LOADS_PER_TILE>();
  };
  // fast steps over tiles [it, t_end): S^T alternates between s_cur and s_alt
  auto fast_steps = [&](int t_end) {
    for (; it + 1 < min(t_end, n_lean); it += 2) {
      lean_step(it, s_cur, s_alt);
      lean_step(it + 1, s_alt, s_cur);
    }
    for (; it + 1 < t_end; it += 2) {
      fast_step(it, s_cur, s_alt);
      fast_step(it + 1, s_alt, s_cur);
    }
    if (it < t_end) {
      fast_step(it, s_cur, s_alt);
      s_cur = s_alt;
      ++it;
    }
  };
  // prefill: the last key this lane's row sees
  const int lim = PREFILL ? (row_ok ? ctx + my_qi : -1) : 0;
  if constexpr (PREFILL) {
    // tiles below the workgroup's first query token's position are visible to
    // every row: pipelined steps; the rest (the causal edge, at most three
    // tiles for 128 rows) step one at a time with a per-row mask
    const int n_pipe = min((ctx + row_base / G + 1) / ST_KEYS, n_st - 1);
    if (n_pipe >= 2) {
      peel();
      fast_steps(n_pipe);
    } else if (n_pipe == 1) {
      prefix_step(0, s_cur, s_alt);
      s_cur = s_alt;
      it = 1;
    }
    if (__ballot(hot_seen) != 0 && lane == 0) hot_flag = 1;
    for (; it < n_st; ++it) {
      fetch_ahead(it);
      uint32_t v = 0;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr)
        v |= (it * ST_KEYS + ks * 32 + 16 * (rr >> 3) + 8 * lhalf + (rr & 7) <= lim ? 1u : 0u) << rr;
      const uint32_t vis[1] = {v};
      const f32x16_t s1[1] = {s_cur};
      u32x4_t pw[1][2];
      weights<DT, SOFTCAP, true, 1>(s1, vis, st, c, cap, pw, o, tb(it));
      pv<DT, 1>(lds + (it % NB) * BUF, ks * 32, lane, pw, o);
      if (it + 1 < n_st) s_cur = qk_half<DT>(lds + ((it + 1) % NB) * BUF, ks * 32, lane, qf);
      step_barrier(it);
    }
  } else {
    if constexpr (OPT) {
      // the window's edge tiles, one at a time with each row's mask (the
      // prefill's causal-edge step with a lower bound instead of an upper)
      for (; it < n_edge; ++it) {
        fetch_ahead(it);
        const int nk = it == n_st - 1 ? p_last : ST_KEYS;
        uint32_t v = 0;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const int kl = ks * 32 + 16 * (rr >> 3) + 8 * lhalf + (rr & 7);
          v |= (kl < nk && kb + it * ST_KEYS + kl >= lo_row ? 1u : 0u) << rr;
        }
        const uint32_t vis[1] = {v};
        const f32x16_t s1[1] = {s_cur};
        u32x4_t pw[1][2];
        weights<DT, SOFTCAP, true, 1>(s1, vis, st, c, cap, pw, o, tb(it));
        pv<DT, 1>(lds + (it % NB) * BUF, ks * 32, lane, pw, o);
        if (it + 1 < n_st) s_cur = qk_half<DT>(lds + ((it + 1) % NB) * BUF, ks * 32, lane, qf);
        if (it + 1 < n_st) step_barrier(it);
        else __syncthreads();
      }
    }
    // the last two tiles take the general step
    if (it == 0 && n_st >= 3) peel();
    for (; it + 1 < n_lean; it += 2) {  // two steps per trip: S^T alternates between s_cur and s_alt
      lean_step(it, s_cur, s_alt);
      lean_step(it + 1, s_alt, s_cur);
    }
    for (; it + 2 < n_st; it += 2) {
      fast_step(it, s_cur, s_alt);
      fast_step(it + 1, s_alt, s_cur);
    }
    if (__ballot(hot_seen) != 0 && lane == 0) hot_flag = 1;
    if (it + 1 < n_st) {
      prefix_step(it, s_cur, s_alt);
      last_step(it + 1, s_alt);
    } else if (it < n_st) {
      last_step(it, s_cur);
    }
  }
  __syncthreads();
  // The lane's row indices again, worked out after the prefix loop instead of
  // being kept live through it (kept, they were spilled to scratch and the
  // epilogue waited on three dependent scratch reloads for its output address).
  // (the divisors too: the compiler would otherwise keep the prologue's
  // integer-division reciprocals live through the loop)
  int tid_e = tid, G_e = G, TG_e = TG, T_e = a.T;
  __asm__ volatile("" : "+v"(tid_e), "+v"(G_e), "+v"(TG_e), "+v"(T_e));
  const int rho_e = row_base + (tid_e >> 7) * 32 + (tid_e & 31);  // row group tid / 128, row tid % 32
  const bool ok_e = rho_e < rows_r;
  const int b_e = PREFILL ? 0 : rho_e / TG_e;
  const int qi_e = PREFILL ? rho_e / G_e : (rho_e / G_e) % T_e;
  const int g_e = rho_e % G_e;
  const int lane_e = tid_e & 63, lhalf_e = lane_e >> 5, lrow_e = lane_e & 31;
  // the row's beam's suffix length read again (an L2 hit) rather than kept
  // live through the loop
  const int len_e = *(!PREFILL && ok_e ? a.suffix_len + nb0 + b_e : zint);
  const bool hot = hot_flag != 0;
  if (hot) {
    // exact recomputation of the workgroup's prefix range, one tile at a time
    // through buffer 0, every tile on the exact (masked) path (after every
    // suffix piece has landed: their data is gathered again below)
    tile_barrier<0>();
    const int lo_e = wl >= 0 ? P + len_e - a.T + qi_e - wl : INT_MIN;  // the row's window bound
    st = RowState{-INFINITY, 0.f};
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) o[mb] = f32x16_t{};
    for (int t = 0; t < n_st; ++t) {
      if constexpr (KV8) {
        dma8(t, 0);
        tile_barrier<0>();
        convert8(0, 0);
        __syncthreads();
      } else {
        issue_tile(t, 0);
        tile_barrier<0>();
      }
      const int nk = t == n_st - 1 ? p_last : ST_KEYS;
      uint32_t v = 0;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int kl = ks * 32 + 16 * (rr >> 3) + 8 * lhalf_e + (rr & 7);  // key within the tile
        v |= (PREFILL ? t * ST_KEYS + kl <= lim : kl < nk && kb + t * ST_KEYS + kl >= lo_e) ? 1u << rr : 0u;
      }
      const uint32_t vis[1] = {v};
      const f32x16_t s1[1] = {qk_half<DT>(lds, ks * 32, lane_e, qf)};
      weights<DT, SOFTCAP, true, 1>(s1, vis, st, c, cap, p, o, tb(t));
      pv<DT, 1>(lds, ks * 32, lane_e, p, o);
      __syncthreads();
    }
  }

  // ---- suffix: each row group's beams' own tokens, masked 32-key tiles ----
  // (all threads load; the two waves of a row group compute a pair of tiles
  // side by side; the group's metadata was staged in the prologue)
  const bool spf_ok = spf_n > 0 && !hot;  // the prefetched pieces are in place
  // this lane's row's sink (log2 units), read now so its latency hides behind
  // the suffix (the split mode adds it in split_merge)
  const float sink_l2 = !SPLIT && a.sinks && ok_e ? a.sinks[hk * G + g_e] * LOG2E : -INFINITY;
  // loader: 4 row groups x 32 slots x 16 chunks per tile; row group g's slots
  // live in buffer g >> 1, rows / columns (g & 1) * 32 .. + 31; all loads of a
  // tile are issued before its first LDS store.
  constexpr int SUF_PER_THREAD = 4 * 32 * 16 / MF_THREADS;
  static_assert(4 * 32 * 16 % MF_THREADS == 0, "suffix loader split");
  // element el of the K / V cache (a byte of an fp8 cache), and one 16-byte
  // chunk of a bf16 / fp16 row loaded from there: eight fp8 bytes converted
  using gvec = const __attribute__((address_space(1))) u32x4_t*;  // global loads, not flat
  using gvec2 = const __attribute__((address_space(1))) u32x2_t*;
  auto kel = [&](int64_t el) { return KV8 ? reinterpret_cast<const S*>(kc8 + el) : kc + el; };
  auto vel = [&](int64_t el) { return KV8 ? reinterpret_cast<const S*>(vc8 + el) : vc + el; };
  auto ldchunk = [&](const S* p) -> u32x4_t {
    if constexpr (KV8) {
      const u32x2_t w = *(gvec2)(p);
      return Fp8Cvt<DT>::x8(w[0], w[1]);
    } else {
      return *(gvec)(p);
    }
  };
  auto suf_gather = [&](int it, int t, u32x4_t (&skv)[SUF_PER_THREAD], u32x4_t (&svv)[SUF_PER_THREAD],
                        int (&sinfo)[SUF_PER_THREAD]) {
    // Two passes: every address first, then all the loads back to back.  Any
    // wait on a global or scratch read in the first pass then has no K/V
    // load to wait for (the vector-memory counter retires in order).
    // Empty slots and invalid blocks read the zero source.
    const S* ksrc[SUF_PER_THREAD];
    const S* vsrc[SUF_PER_THREAD];
#pragma unroll
    for (int i = 0; i < SUF_PER_THREAD; ++i) {
      const int e = t + i * MF_THREADS;
      const int grp = e >> 9;
      const int slot = (e >> 4) & 31;
      const int ch = e & 15;
      const int gs = it * 32 + slot;
      ksrc[i] = zsrc;
      vsrc[i] = zsrc;
      sinfo[i] = -1;
      if (gs < suf_cum[grp][32]) {
        int lo = 0, hi = 31;  // largest beam index i with cum[i] <= gs (skips empty beams)
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (suf_cum[grp][mid] <= gs) lo = mid; else hi = mid - 1;
        }
        const int b = suf_cum[grp][33] + lo;
        const int j = gs - suf_cum[grp][lo];
        const int n = nb0 + b;
        const int pos = suf_s0[grp][lo] + j;
        const int bi = pos >> bsh;  // power-of-two block size on this path
        int blk;  // staged ids from LDS, later ones (long suffixes) from HBM
        if (bi < SB_STAGE) blk = suf_blk[grp][lo][bi];
        else blk = a.suffix_bt[(int64_t)n * a.suffix_bt_stride + bi];
        if (blk >= 0 && blk < a.num_blocks) {
          const int64_t base = (int64_t)blk * a.kv_block_stride + (int64_t)(pos & (a.bs - 1)) * a.kv_tok_stride +
                               head_off + ch * 8;
          ksrc[i] = kel(base);
          vsrc[i] = vel(base);
          sinfo[i] = (b << 16) | j;
        } else {
          flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < SUF_PER_THREAD; ++i) {
      skv[i] = ldchunk(ksrc[i]);
      svv[i] = ldchunk(vsrc[i]);
    }
  };
  // tile h (0 or 1) of a pair: row group g's slots in buffer 2h + (g >> 1),
  // rows (g & 1) * 32 .. + 31
  auto suf_store = [&](int t, int h, const u32x4_t (&skv)[SUF_PER_THREAD], const u32x4_t (&svv)[SUF_PER_THREAD]) {
#pragma unroll
    for (int i = 0; i < SUF_PER_THREAD; ++i) {
      const int e = t + i * MF_THREADS;
      const int grp = e >> 9;
      const int slot = (e >> 4) & 31;
      const int ch = e & 15;
      uint16_t* buf = lds + ((sbase + 2 * h + (grp >> 1)) & 3) * BUF;
      const int key = (grp & 1) * 32 + slot;
      *reinterpret_cast<u32x4_t*>(buf + key * KS_PITCH + kchunk(key, ch) * 8) = skv[i];
      *reinterpret_cast<u32x4_t*>(buf + K_TILE + key * VS_PITCH + vchunk(key, ch) * 8) = svv[i];
    }
  };
  auto suf_tag = [&](int t, int h, const int (&sinfo)[SUF_PER_THREAD]) {
#pragma unroll
    for (int i = 0; i < SUF_PER_THREAD; ++i) {
      const int e = t + i * MF_THREADS;
      if ((e & 15) == 0) suf_info[h][e >> 9][(e >> 4) & 31] = sinfo[i];
    }
  };
  // the first pair's slots come from the prologue's slot table (tags already
  // in suf_info): one LDS read per slot, then the loads
  auto suf_gather_tab = [&](int h, int t, u32x4_t (&skv)[SUF_PER_THREAD], u32x4_t (&svv)[SUF_PER_THREAD]) {
    const S* ksrc[SUF_PER_THREAD];
    const S* vsrc[SUF_PER_THREAD];
#pragma unroll
    for (int i = 0; i < SUF_PER_THREAD; ++i) {
      const int e = t + i * MF_THREADS;
      const int64_t off = suf_off[e >> 9][h * 32 + ((e >> 4) & 31)];
      const int ch = e & 15;
      ksrc[i] = off < 0 ? zsrc : kel(off + ch * 8);
      vsrc[i] = off < 0 ? zsrc : vel(off + ch * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < SUF_PER_THREAD; ++i) {
      skv[i] = ldchunk(ksrc[i]);
      svv[i] = ldchunk(vsrc[i]);
    }
  };
  // this wave's row group against tile h of the pair
  auto suf_compute = [&](int h) {
    // register r of this lane is slot 16*(r>>3) + 8*lhalf + (r&7) of the group's 32
    const int lim = ok_e ? len_e - a.T + qi_e : -1;
    // window: suffix token j sits at key P + j
    const int jlo = wl >= 0 ? len_e - a.T + qi_e - wl : 0;
    uint32_t vis = 0;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const int info = suf_info[h][rg][16 * (rr >> 3) + 8 * lhalf_e + (rr & 7)];
      const bool ok = info >= 0 && (info >> 16) == b_e && (info & 0xFFFF) <= lim && (info & 0xFFFF) >= jlo;
      vis |= (ok ? 1u : 0u) << rr;
    }
    const uint16_t* sbuf = lds + ((sbase + 2 * h + (rg >> 1)) & 3) * BUF;
    const f32x16_t s1[1] = {qk_half<DT>(sbuf, (rg & 1) * 32, lane_e, qf)};
    const uint32_t vis1[1] = {vis};
    u32x4_t pw[1][2];
    if constexpr (OPT) {
      // ALiBi of suffix token j (key P + j): alpha * (j - (len - T + qi))
      float bb[16];
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int info = suf_info[h][rg][16 * (rr >> 3) + 8 * lhalf_e + (rr & 7)];
        bb[rr] = alpha * (float)((info & 0xFFFF) - (len_e - a.T + qi_e));
      }
      weights<DT, SOFTCAP, true, 1>(s1, vis1, st, c, cap, pw, o, ArrBias{bb});
    } else {
      weights<DT, SOFTCAP, true, 1>(s1, vis1, st, c, cap, pw, o);
    }
    pv<DT, 1>(sbuf, (rg & 1) * 32, lane_e, pw, o);
  };
  // Tiles in pairs: the key-half-0 wave of each row group takes the first
  // tile, the key-half-1 wave the second, at the same time (each adds to its
  // own partial state; the halves merge below).
  if (spf_ok && spf_n > 3) suf_piece(3);  // its buffer held the last prefix tile
  for (int it = 0; it < n_sit; it += 2) {
    // a fresh copy of the thread index each trip: the slot addresses derived
    // from it are recomputed in registers rather than hoisted out of the loop
    // and spilled to scratch (whose reloads would wait on every load)
    int t = tid;
    __asm__ volatile("" : "+v"(t));
    const bool two = it + 1 < n_sit;
    if (it == 0 && spf_ok) {
      // the pair is in LDS (prefetched pieces, tags from the slot table)
    } else if (it == 0 && tab_ok) {
      // both tiles' loads in flight at once (a missing second tile's slots are
      // empty and read the zero source)
      u32x4_t skv0[SUF_PER_THREAD], svv0[SUF_PER_THREAD], skv1[SUF_PER_THREAD], svv1[SUF_PER_THREAD];
      suf_gather_tab(0, t, skv0, svv0);
      suf_gather_tab(1, t, skv1, svv1);
      suf_store(t, 0, skv0, svv0);
      suf_store(t, 1, skv1, svv1);
    } else {
      {
        u32x4_t skv0[SUF_PER_THREAD], svv0[SUF_PER_THREAD];
        int sinfo0[SUF_PER_THREAD];
        suf_gather(it, t, skv0, svv0, sinfo0);
        suf_store(t, 0, skv0, svv0);
        suf_tag(t, 0, sinfo0);
      }
      if (two) {
        u32x4_t skv1[SUF_PER_THREAD], svv1[SUF_PER_THREAD];
        int sinfo1[SUF_PER_THREAD];
        suf_gather(it + 1, t, skv1, svv1, sinfo1);
        suf_store(t, 1, skv1, svv1);
        suf_tag(t, 1, sinfo1);
      }
    }
    if (it == 0 && spf_ok) tile_barrier<0>();  // every piece has landed
    else __syncthreads();
    if (ks == 0 || two) suf_compute(ks);
    __syncthreads();
  }

  // ---- merge the two key halves and write O, LSE --------------------------
  // (the row indices once more, from a fresh copy of the thread index, so
  // none of them lives through the suffix phase)
  int tid_f = tid, G_f = G, TG_f = TG, T_f = a.T;
  __asm__ volatile("" : "+v"(tid_f), "+v"(G_f), "+v"(TG_f), "+v"(T_f));
  const int rho_f = row_base + (tid_f >> 7) * 32 + (tid_f & 31);
  const bool ok_f = rho_f < rows_r;
  const int b_f = PREFILL ? 0 : rho_f / TG_f;
  const int qi_f = PREFILL ? rho_f / G_f : (rho_f / G_f) % T_f;
  const int g_f = rho_f % G_f;
  const int lane_f = tid_f & 63, lhalf_f = lane_f >> 5, lrow_f = lane_f & 31;
  // [rg][lane][64 accumulators, padded to 68]: 16-byte writes and reads, the
  // padding spreads a row of lanes over every bank
  constexpr int XO_PITCH = 68;
  float* xo = reinterpret_cast<float*>(lds) + rg * (64 * XO_PITCH) + lane_f * XO_PITCH;
  float* xm = reinterpret_cast<float*>(lds) + 4 * (64 * XO_PITCH) + rg * 128;  // [rg][m | lsum][lane]
  if (ks == 1) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
        *reinterpret_cast<f32x4_t*>(xo + mb * 16 + qd * 4) =
            f32x4_t{o[mb][qd * 4], o[mb][qd * 4 + 1], o[mb][qd * 4 + 2], o[mb][qd * 4 + 3]};
    xm[lane_f] = st.m;
    xm[64 + lane_f] = st.lsum;
  }
  __syncthreads();
  if (ks == 0) {
    const float m1 = xm[lane_f], l1 = xm[64 + lane_f];
    const float m0 = st.m, l0 = st.lsum;
    // a sink joins the row's softmax: in the maximum and, once, in the sum
    const float m = fmaxf(fmaxf(m0, m1), sink_l2);
    const float a0 = m0 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m0 - m);
    const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
    const float lrow_sum =
        pair_sum(l0 * a0 + l1 * a1) + (sink_l2 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sink_l2 - m));
    // (an fp8 cache's V scale multiplies the normalised output)
    const float inv = lrow_sum > 0.f ? vsc / lrow_sum : 0.f;
    if constexpr (SPLIT) {
      // this split's normalised partial O and LSE, every row of the tile
      const int64_t slot = (int64_t)(unit * mtiles + mt) * nsplit + split;
      uint16_t* po = a.ws_o + (slot * MF_ROWS + rg * 32 + lrow_f) * HD + 4 * lhalf_f;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          float v[4];
          const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(xo + mb * 16 + qd * 4);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int rr = qd * 4 + u;
            v[u] = (o[mb][rr] * a0 + x1[u] * a1) * inv;
          }
          const u32x2_t w = {Mma<DT>::pack2(v[0], v[1]), Mma<DT>::pack2(v[2], v[3])};
          *reinterpret_cast<u32x2_t*>(po + mb * 32 + qd * 8) = w;
        }
      }
      if (lhalf_f == 0)
        a.ws_lse[slot * MF_ROWS + rg * 32 + lrow_f] =
            lrow_sum > 0.f ? (m + __builtin_amdgcn_logf(lrow_sum)) * 0.6931471805599453f : -INFINITY;
    } else if (ok_f) {
      const int64_t tok = PREFILL ? (int64_t)(nb0 + qi_f) : (int64_t)(nb0 + b_f) * a.T + qi_f;
      // (head pairs: only the row's own half of the 128 dims, dim blocks 2 half, 2 half + 1)
      const int half_f = PAIR ? g_f / (G >> 1) : 0;
      S* dst = static_cast<S*>(a.out) + tok * a.out_tok_stride + (int64_t)(hk * G + g_f) * (PAIR ? HD / 2 : HD) +
               4 * lhalf_f - (PAIR ? half_f * (HD / 2) : 0);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (PAIR && (mb >> 1) != half_f) continue;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          float v[4];
          const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(xo + mb * 16 + qd * 4);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int rr = qd * 4 + u;
            v[u] = (o[mb][rr] * a0 + x1[u] * a1) * inv;
          }
          const u32x2_t w = {Mma<DT>::pack2(v[0], v[1]), Mma<DT>::pack2(v[2], v[3])};
          *reinterpret_cast<u32x2_t*>(dst + mb * 32 + qd * 8) = w;
        }
      }
      if (a.lse_out && lhalf_f == 0) {
        a.lse_out[tok * a.Hq + hk * G + g_f] =
            lrow_sum > 0.f ? (m + __builtin_amdgcn_logf(lrow_sum)) * 0.6931471805599453f : -INFINITY;
      }
    }
  }
}

// Merge of the split decode's partials: one thread per (row, 8 dims), 16 rows
// of one row tile per workgroup.  LSE* = log sum_s exp(LSE_s), O = sum_s
// exp(LSE_s - LSE*) O_s (the merge_attn_states rule), written as the final
// output and LSE.
constexpr int MG_ROWS = 16;
template <int DT>
__global__ __launch_bounds__(256) void split_merge(DecodeArgs a, int mtiles) {
  kernarg_lines<kernarg_line_count<DecodeArgs>(4)>();
  using S = uint16_t;
  constexpr int PER_TILE = MF_ROWS / MG_ROWS;
  const int tile = blockIdx.x / PER_TILE;
  const int row = (blockIdx.x % PER_TILE) * MG_ROWS + threadIdx.x / (HD / 8);
  const int d8 = (threadIdx.x % (HD / 8)) * 8;  // 8 dims: one 16-byte vector per partial
  const int unit = tile / mtiles, mt = tile % mtiles;
  const int r = unit / a.Hkv, hk = unit % a.Hkv;
  const int nb0 = a.beam_start[r], W = a.beam_start[r + 1] - nb0;
  if (nb0 < 0 || W < 0 || nb0 + W > a.num_beams) return;  // flagged by the decode kernel
  const int G = a.Hq / a.Hkv, TG = a.T * G, rows_r = W * TG;
  const int rho = mt * MF_ROWS + row;
  if (rho >= rows_r) return;
  const int nsplit = a.nsplit;
  const float* lse = a.ws_lse + (int64_t)tile * nsplit * MF_ROWS + row;
  const uint16_t* po = a.ws_o + ((int64_t)tile * nsplit * MF_ROWS + row) * HD + d8;
  const float sk = a.sinks ? a.sinks[hk * G + rho % G] : -INFINITY;  // joins the merged softmax once
  float mx = sk;
#pragma unroll 4
  for (int s2 = 0; s2 < nsplit; ++s2) mx = fmaxf(mx, lse[s2 * MF_ROWS]);
  float acc[8] = {}, sum = sk == -INFINITY ? 0.f : __expf(sk - mx);
  if (mx != -INFINITY) {
#pragma unroll 4
    for (int s2 = 0; s2 < nsplit; ++s2) {
      const float w = __expf(lse[s2 * MF_ROWS] - mx);
      const u32x4_t pv = *reinterpret_cast<const u32x4_t*>(po + (int64_t)s2 * MF_ROWS * HD);
      sum += w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += w * Mma<DT>::lo(pv[e]);
        acc[2 * e + 1] += w * Mma<DT>::hi(pv[e]);
      }
    }
  }
  const float inv = sum > 0.f ? 1.f / sum : 0.f;
  const int b = rho / TG, qi = (rho / G) % a.T, g = rho % G;
  const int64_t tok = (int64_t)(nb0 + b) * a.T + qi;
  u32x4_t wv;
#pragma unroll
  for (int e = 0; e < 4; ++e) wv[e] = Mma<DT>::pack2(acc[2 * e] * inv, acc[2 * e + 1] * inv);
  *reinterpret_cast<u32x4_t*>(static_cast<S*>(a.out) + tok * a.out_tok_stride + (int64_t)(hk * G + g) * HD + d8) = wv;
  if (a.lse_out && d8 == 0) a.lse_out[tok * a.Hq + hk * G + g] = mx == -INFINITY ? -INFINITY : mx + __logf(sum);
}

}  // namespace

bool mfma_decode_supported(const DecodeArgs& a) {
  if (a.D != HD || (a.dtype != GR_DTYPE_BF16 && a.dtype != GR_DTYPE_F16)) return false;
  // options here: sinks, fp8 caches, and a decode's left window and ALiBi;
  // right windows and non-causal batches take the generic kernel
  if (!a.causal || a.win_right >= 0) return false;
  if (a.bs_shift < 2) return false;  // power-of-two block size >= 4
  if (a.num_blocks < 1) return false;  // an empty pool: the generic kernel reads nothing
  // the suffix tiles tag each key with its 16-bit index within the beam's suffix
  if ((int64_t)a.suffix_bt_stride * a.bs > 0xFFFF) return false;
  // 16-byte vector access: base pointers and element strides multiples of 8 elements
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!al(a.q) || !al(a.out) || !al(a.k_cache) || !al(a.v_cache)) return false;
  // (an fp8 cache's rows move in 16-byte chunks of 16 elements)
  const int kv_al = a.kv8 ? 16 : 8;
  if (a.q_tok_stride % 8 || a.out_tok_stride % 8 || a.kv_block_stride % kv_al || a.kv_tok_stride % kv_al ||
      a.kv_head_stride % kv_al)
    return false;
  // tile loads multiply block ids by the block stride in 32 bits
  if (a.kv_block_stride <= 0 || a.kv_block_stride > 0xFFFFFFFFll) return false;
  return true;
}

bool mfma_prefill_supported(const DecodeArgs& a) { return mfma_decode_supported(a) && a.win_left < 0 && !a.alibi; }

// head_dim 64: KV heads 2j and 2j + 1 sit side by side in a cache row (head
// stride 64), so they read as one 128-dim head j serving both heads' query
// heads (2 G of them).  A query row's Q fills its own head's half of the 128
// dims and zeros the other, so its scores are its own head's; the PV product
// gives both halves and only the row's own half is written.  Twice the
// matrix-core work of the 64-dim problem, at the 128-dim kernel's speed.
bool mfma_pair_args(const DecodeArgs& a, DecodeArgs& p) {
  if (a.D != HD / 2 || a.Hkv % 2 != 0 || a.kv_head_stride != HD / 2) return false;
  p = a;
  p.D = HD;
  p.Hkv = a.Hkv / 2;
  p.kv_head_stride = HD;
  p.pair = 1;
  return mfma_decode_supported(p);
}

template <bool PREFILL, bool SPLIT, bool OPT, bool KV8, bool PAIR>
static void launch_mfma_kernel_p(const DecodeArgs& a, dim3 grid, int units, int mtiles, hipStream_t stream) {
  const bool cap = a.softcap > 0.f;
  const dim3 blk(MF_THREADS);
  if (a.dtype == GR_DTYPE_BF16) {
    if (cap) hipLaunchKernelGGL((decode_mfma<GR_DTYPE_BF16, true, PREFILL, SPLIT, OPT, KV8, PAIR>), grid, blk, 0, stream, a, units, mtiles);
    else hipLaunchKernelGGL((decode_mfma<GR_DTYPE_BF16, false, PREFILL, SPLIT, OPT, KV8, PAIR>), grid, blk, 0, stream, a, units, mtiles);
  } else {
    if (cap) hipLaunchKernelGGL((decode_mfma<GR_DTYPE_F16, true, PREFILL, SPLIT, OPT, KV8, PAIR>), grid, blk, 0, stream, a, units, mtiles);
    else hipLaunchKernelGGL((decode_mfma<GR_DTYPE_F16, false, PREFILL, SPLIT, OPT, KV8, PAIR>), grid, blk, 0, stream, a, units, mtiles);
  }
}

// head pairs have their own instantiations (never split), so the 128-dim
// kernels carry none of their arithmetic
template <bool PREFILL, bool SPLIT, bool OPT, bool KV8>
static void launch_mfma_kernel(const DecodeArgs& a, dim3 grid, int units, int mtiles, hipStream_t stream) {
  if constexpr (!SPLIT) {
    if (a.pair) {
      launch_mfma_kernel_p<PREFILL, SPLIT, OPT, KV8, true>(a, grid, units, mtiles, stream);
      return;
    }
  }
  launch_mfma_kernel_p<PREFILL, SPLIT, OPT, KV8, false>(a, grid, units, mtiles, stream);
}

// the option variant (a decode's window or ALiBi) and the fp8-cache variant
template <bool PREFILL, bool SPLIT, bool KV8>
static void launch_mfma_opt(const DecodeArgs& a, dim3 grid, int units, int mtiles, hipStream_t stream) {
  if (!PREFILL && (a.win_left >= 0 || a.alibi))
    launch_mfma_kernel<PREFILL, SPLIT, !PREFILL, KV8>(a, grid, units, mtiles, stream);
  else launch_mfma_kernel<PREFILL, SPLIT, false, KV8>(a, grid, units, mtiles, stream);
}

template <bool PREFILL, bool SPLIT>
static gr_status_t launch_mfma(const DecodeArgs& a, hipStream_t stream) {
  const int G = a.Hq / a.Hkv;
  const int64_t rows = (int64_t)(PREFILL ? 1 : a.max_beams) * a.T * G;
  const int64_t mt64 = (rows + MF_ROWS - 1) / MF_ROWS;
  const int units = a.num_reqs * a.Hkv;
  if (mt64 == 0 || units == 0) return GR_OK;
  const int64_t nwg = (int64_t)((units + 7) / 8) * 8 * mt64 * (SPLIT ? a.nsplit : 1);
  if (nwg > 0x7fffffff) return GR_ERR_INVALID_ARG;
  const int mtiles = (int)mt64;
  dim3 grid((unsigned)nwg);
  if (a.kv8) launch_mfma_opt<PREFILL, SPLIT, true>(a, grid, units, mtiles, stream);
  else launch_mfma_opt<PREFILL, SPLIT, false>(a, grid, units, mtiles, stream);
  return launch_status();
}

gr_status_t launch_mfma_decode(const DecodeArgs& a, hipStream_t stream) { return launch_mfma<false, false>(a, stream); }
gr_status_t launch_mfma_prefill(const DecodeArgs& a, hipStream_t stream) { return launch_mfma<true, false>(a, stream); }
gr_status_t launch_mfma_decode_split(const DecodeArgs& a, hipStream_t stream) {
  const gr_status_t st = launch_mfma<false, true>(a, stream);
  if (st != GR_OK) return st;
  const int G = a.Hq / a.Hkv;
  const int mtiles = (int)(((int64_t)a.max_beams * a.T * G + MF_ROWS - 1) / MF_ROWS);
  const int64_t nwg = (int64_t)a.num_reqs * a.Hkv * mtiles * (MF_ROWS / MG_ROWS);
  if (nwg == 0) return GR_OK;
  if (nwg > 0x7fffffff) return GR_ERR_INVALID_ARG;
  if (a.dtype == GR_DTYPE_BF16)
    hipLaunchKernelGGL(split_merge<GR_DTYPE_BF16>, dim3((unsigned)nwg), dim3(256), 0, stream, a, mtiles);
  else
    hipLaunchKernelGGL(split_merge<GR_DTYPE_F16>, dim3((unsigned)nwg), dim3(256), 0, stream, a, mtiles);
  return launch_status();
}

// Enough splits to give the grid ~256 workgroups (one per CU at this kernel's
// LDS use), at most 16, and no fewer than 4 prefix tiles per split when the
// longest prefix is known.
void mfma_decode_plan(int num_reqs, int max_beams, int q_per_beam, int Hq, int Hkv, int max_prefix_len,
                      int* tiles, int* nsplit) {
  const int G = Hq / Hkv;
  const int64_t mtiles = ((int64_t)max_beams * q_per_beam * G + MF_ROWS - 1) / MF_ROWS;
  const int64_t units = (int64_t)num_reqs * Hkv;
  const int64_t wg = (units + 7) / 8 * 8 * mtiles;
  *tiles = (int)(units * mtiles);
  int ns = wg <= 0 || wg >= 256 ? 1 : (int)((256 + wg - 1) / wg);
  if (max_prefix_len > 0) ns = std::min(ns, std::max(1, max_prefix_len / (4 * ST_KEYS)));
  *nsplit = std::min(ns, 16);
}

}  // namespace gr
