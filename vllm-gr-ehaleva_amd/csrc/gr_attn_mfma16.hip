// BeamAttention decode on gfx950 matrix cores with 64 query rows per wave
// (bf16/fp16, head_dim 128).
//
// Work decomposition.  For request r and KV head h the query rows of all its
// beams form one dense M x 128 matrix (M = beams * q_per_beam * GQA group).
// A 256-thread workgroup owns 128 of those rows: 4 waves, one per SIMD, wave
// (rg, ks) holding rows 64 rg .. 64 rg + 63 against key half ks of every
// 64-key tile.  The request's prefix K/V streams through LDS in 64-key tiles,
// each loaded once for all 128 rows, straight from global memory into LDS
// (global_load_lds_dwordx4, four buffers, three tiles in flight ahead of the
// one being computed); the beams' own suffix tokens follow as masked tiles
// gathered from their paged blocks.  The two key halves keep separate
// online-softmax states, merged in LDS at the end.  Workgroups of one
// (request, KV head) sit on one XCD (blockIdx % 8 is the XCD under
// round-robin dispatch), so their prefix re-reads hit that XCD's L2.
//
// Why 64 rows per wave: with v_mfma_f32_16x16x32 every K or V fragment read
// from LDS (16 keys x 32 dims, or 16 dims x 32 keys: 1 KB) feeds four MFMAs,
// one per 16-row block, so the LDS traffic per tile is half that of 32-row
// waves and stays under the matrix-core time of the step.  The registers this
// takes (Q 64 and O 128 in accumulation registers; S 64, fragments 64, P 16)
// need the whole 512-entry register file of a SIMD: one wave per SIMD, whose
// latencies are covered inside the wave -- every step issues all its LDS
// fragment reads and its tile loads first, and the loads land in LDS without
// passing through registers.
//
// MFMA formulation (v_mfma_f32_16x16x32_{bf16,f16}, wave64; lane = n + 16 g):
//   S^T[key][row] = K[key][:] . Q[row][:]   A = K (16 keys x 32 dims), B = Q^T
//   O^T[d][row]  += V^T[d][key] . P^T[key][row]   A = V^T (16 dims x 32 keys)
// A lane holds A[m = n][8g .. 8g+7], B[8g .. 8g+7][n] and D[4g .. 4g+3][n].
// The two 16-key S^T tiles of a key half read K rows in the order
// key(t, m) = 8 (m >> 2) + 4 t + (m & 3), so lane (n, g) ends up with keys
// 8g .. 8g+7 of its half -- exactly the eight keys the PV B operand of lane
// (n, g) needs: P^T is packed from S^T in registers, with no data exchange.
// V^T is assembled with gfx950's transposing LDS read (ds_read_b64_tr_b16:
// in each 16-lane group, source lane s addresses V[k0 + s/4][d0 + 4(s%4) ..
// +3] and lane i receives V[k0 .. k0+3][d0 + i]).
//
// Softmax: exp2 against a per-row reference maximum that the first tile sets
// and that never moves in the loop (O is never rescaled there); a weight that
// could exceed 2^Rescale16::THRESH, or a row whose first visible key comes
// after the first tile, flags the workgroup, which then recomputes its rows
// in two exact passes (the maxima, then the weights).
#include <algorithm>
#include <type_traits>

#include "gr_attn_decode.h"

namespace gr {
namespace {

constexpr int T16 = 256;          // threads: 4 waves
constexpr int R16 = 128;          // query rows per workgroup
constexpr int K16 = 64;           // keys per tile
constexpr int HD = 128;           // head dim
constexpr int ROWB = HD * 2;      // bytes per K or V row in LDS (no padding: swizzled)
constexpr int KTB = K16 * ROWB;   // bytes of a tile's K (then its V)
constexpr int BUFB = 2 * KTB;     // bytes per buffer
constexpr int NB = 4;             // tile buffers: the tile computed, its successor, two in flight
constexpr int MAXB = R16 + 1;     // beams the rows of a workgroup can touch
constexpr int SBT = 2048;         // suffix block-table entries staged in LDS (all of the workgroup's beams)
constexpr int SKT = 1024;         // suffix keys of a workgroup with a precomputed gather entry
constexpr float LOG2E = 1.4426950408889634f;

template <int DT> struct Rescale16;
template <> struct Rescale16<GR_DTYPE_BF16> {
  static constexpr float THRESH = 60.0f;
  static constexpr float SUM = 1.152921504606846976e18f;  // 2^60
};
template <> struct Rescale16<GR_DTYPE_F16> {
  static constexpr float THRESH = 15.0f;  // the packed fp16 P operand ends at 65504
  static constexpr float SUM = 32768.0f;
};

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));
typedef uint32_t u32x4_t __attribute__((__vector_size__(4 * sizeof(uint32_t))));
typedef uint32_t u32x2_t __attribute__((__vector_size__(2 * sizeof(uint32_t))));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

__device__ __attribute__((aligned(16))) uint32_t g_zero16b[4];

template <int DT> struct M16;
template <> struct M16<GR_DTYPE_BF16> {
  __device__ static inline f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});
  }
};
template <> struct M16<GR_DTYPE_F16> {
  __device__ static inline f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, f16x2_t{(_Float16)lo, (_Float16)hi});
  }
};

// LDS layouts (256-byte rows).  K row r: logical 16-byte chunk c at
// physical chunk c ^ kswz(r) -- the eight rows one 8-lane group of the
// A-operand read touches, {0..3, 8..11} (+4, +16, +32), land on eight chunk
// columns.  V row r: logical 32-byte pair q (dims 16q .. 16q+15) at physical
// pair q ^ (r & 3) -- the four rows one 16-lane group of a transposing read
// touches land on four pair columns.
__device__ inline int kswz(int r) { return (r & 3) | (((r >> 3) & 1) << 2); }
__device__ inline int vchunk(int r, int c) { return (((c >> 1) ^ (r & 3)) << 1) | (c & 1); }

__device__ inline u32x4_t lds16(uint32_t a) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(a);
}
__device__ inline uint2 lds_tr(uint32_t a) {
  auto v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)(uintptr_t)a);
  return __builtin_bit_cast(uint2, v);
}

// workgroup barrier after this wave's LDS writes and all but its newest
// `inflight` (0 or 8) tile loads have landed
template <int INFLIGHT>
__device__ inline void tile_barrier() {
  if constexpr (INFLIGHT == 8) __asm__ volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <bool SOFTCAP>
__device__ inline float score_l2(float v, float c, float cap) {
  return SOFTCAP ? cap * tanhf(v * c) * LOG2E : v * c;
}
template <bool SOFTCAP>
__device__ inline float weight(float v, float c, float cap, float mref) {
  return SOFTCAP ? __builtin_amdgcn_exp2f(score_l2<true>(v, c, cap) - mref)
                 : __builtin_amdgcn_exp2f(fmaf(v, c, -mref));
}

// max over the four lanes (n, g = 0..3) that hold one row
__device__ inline float row_max4(float x) {
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  return fmaxf(x, __shfl_xor(x, 32, 64));
}
__device__ inline float row_sum4(float x) {
  x += __shfl_xor(x, 16, 64);
  return x + __shfl_xor(x, 32, 64);
}

struct St16 {
  float m[4];     // per row block: the row's reference maximum (log2 units), -inf before any key
  float l[4];     // this lane's partial weight sum of the row
};

// The K fragments of the wave's key half of a tile (K at LDS byte address
// kb): kf[c4][t] = keys key(t, n) x dims 32 c4 + 8 g .. +7.  koff: this
// lane's byte offsets of chunk c4 in row key(0, n) of the half.
__device__ inline void read_k(uint32_t kb, const uint32_t (&koff)[4], u32x4_t (&kf)[4][2]) {
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
    for (int t = 0; t < 2; ++t) kf[c4][t] = lds16(kb + koff[c4] + t * 4 * ROWB);
}
// The V^T fragments of the wave's key half (V at byte address vb):
// vf[db] = dims 16 db .. +15 x keys 8 g .. 8g+7, two transposing reads each.
// voff[d]: this lane's byte offset for pair columns d and d + 4.
__device__ inline void read_v(uint32_t vb, const uint32_t (&voff)[4], u32x4_t (&vf)[8]) {
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    const uint32_t a = vb + voff[db & 3] + (db >> 2) * 128;
    const uint2 lo = lds_tr(a);
    const uint2 hi = lds_tr(a + 4 * ROWB);
    vf[db] = u32x4_t{lo.x, lo.y, hi.x, hi.y};
  }
}

// S^T of row block rb: the two 16-key tiles of the wave's key half, over
// the four 32-dim chunks (two accumulation chains).
template <int DT>
__device__ inline void qk_rb(int rb, const u32x4_t (&kf)[4][2], const u32x4_t (&qf)[4][4], f32x4_t (&s)[2][4]) {
  using M = M16<DT>;
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
    for (int t = 0; t < 2; ++t)
      s[t][rb] = M::mma(kf[c4][t], qf[rb][c4], c4 == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : s[t][rb]);
}

template <int DT>
__device__ inline void pv_mma(const u32x4_t (&vf)[8], const u32x4_t (&p)[4], f32x4_t (&o)[8][4]) {
  using M = M16<DT>;
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) o[db][rb] = M::mma(vf[db], p[rb], o[db][rb]);
}

template <int DT>
__device__ inline void pv_rb(const u32x4_t (&vf)[8], const u32x4_t& p, f32x4_t (&o)[8][4], int rb) {
#pragma unroll
  for (int db = 0; db < 8; ++db) o[db][rb] = M16<DT>::mma(vf[db], p, o[db][rb]);
}

// Weights of row block rb of a tile against the row's reference, which never
// moves here (so O is never rescaled in the loop); MASKED: bit 4t+i of vis =
// key visible.  Returns true when some weight could exceed 2^THRESH or a
// row with a visible key has no reference yet -- the workgroup then
// recomputes its rows in two exact passes.
template <int DT, bool SOFTCAP, bool MASKED>
__device__ inline bool weights_rb(const f32x4_t (&s)[2][4], int rb, uint32_t vis, St16& st, float c, float cap,
                                  u32x4_t& p) {
  using M = M16<DT>;
  float e[2][4];
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float w = weight<SOFTCAP>(s[t][rb][i], c, cap, st.m[rb]);
      e[t][i] = !MASKED || ((vis >> (4 * t + i)) & 1) ? w : 0.f;
      acc += e[t][i];
    }
  p = u32x4_t{M::pack2(e[0][0], e[0][1]), M::pack2(e[0][2], e[0][3]), M::pack2(e[1][0], e[1][1]),
              M::pack2(e[1][2], e[1][3])};
  st.l[rb] += acc;
  return !(acc <= Rescale16<DT>::SUM);
}

// One phase of a decode step: two groups of eight MFMAs (KA, KB: 0 = the QK
// of row block RA / RB into s, 1 = the PV of that row block, 2 = none),
// issued one at a time, each followed by a slice of the weights of row
// block WRB (score, exp2, sum, pack), the order fixed against the scheduler:
// with one wave per SIMD, VALU work hides under the matrix core only when it
// sits between the MFMAs.  The weights read S^T of WRB in slots 0-7, before
// group B (slots 8-15) may overwrite it.  Returns the hot flag of
// weights_rb.
template <int DT, bool SOFTCAP, bool MASKED, int KA, int RA, int KB, int RB, int WRB>
__device__ inline bool phase16(f32x4_t (&s)[2][4], f32x4_t (&o)[8][4], u32x4_t (&p)[4], const u32x4_t (&kf)[4][2],
                               const u32x4_t (&vf)[8], const u32x4_t (&qf)[4][4], uint32_t vis, St16& st, float c,
                               float cap) {
  using M = M16<DT>;
  float x[8], e[8], acc = 0.f;
  uint32_t pw[4];
  bool hot = false;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int kind = k < 8 ? KA : KB, rb = k < 8 ? RA : RB, i = k & 7;
    if (kind == 0) {
      const int c4 = i >> 1, tt = i & 1;
      s[tt][rb] = M::mma(kf[c4][tt], qf[rb][c4], c4 == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : s[tt][rb]);
    } else if (kind == 1) {
      o[i][rb] = M::mma(vf[i], p[rb], o[i][rb]);
    }
    if (WRB >= 0) {
      if (k < 8) x[k] = SOFTCAP ? score_l2<true>(s[k >> 2][WRB][k & 3], c, cap) - st.m[WRB]
                                : fmaf(s[k >> 2][WRB][k & 3], c, -st.m[WRB]);
      if (k >= 1 && k <= 8) {
        const float w = __builtin_amdgcn_exp2f(x[k - 1]);
        e[k - 1] = !MASKED || ((vis >> (k - 1)) & 1) ? w : 0.f;
      }
      if (k >= 2 && k <= 9) acc += e[k - 2];
      if (k >= 3 && k <= 9 && (k & 1)) pw[(k - 3) >> 1] = M::pack2(e[k - 3], e[k - 2]);
      if (k == 10) {
        p[WRB] = u32x4_t{pw[0], pw[1], pw[2], pw[3]};
        st.l[WRB] += acc;
        hot = !(acc <= Rescale16<DT>::SUM);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  return hot;
}

// The rows' maxima over the visible keys of the tile (log2 units), reduced
// over the four lanes that hold a row; -inf for a row without one.
template <bool SOFTCAP>
__device__ inline void tile_max(const f32x4_t (&s)[2][4], const uint32_t (&vis)[4], float c, float cap,
                                float (&mx)[4]) {
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        m = (vis[rb] >> (4 * t + i)) & 1 ? fmaxf(m, score_l2<SOFTCAP>(s[t][rb][i], c, cap)) : m;
    mx[rb] = row_max4(m);
  }
}

template <int DT, bool SOFTCAP>
__global__ __launch_bounds__(T16, 1) void decode_d16(DecodeArgs a, int units, int mtiles) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NB * BUFB];
  __shared__ int suf_cum[MAXB + 1];
  __shared__ int suf_s0[MAXB];
  __shared__ int suf_bt[SBT];
  __shared__ int2 suf_key[SKT];
  __shared__ __attribute__((aligned(16))) int info_s[NB][K16];
  __shared__ int scan_tmp[T16 / 64];
  __shared__ int hot_flag;

  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  const int unit = (local / mtiles) * 8 + xcd;
  const int mt = local % mtiles;
  if (unit >= units) return;
  const int r = unit / a.Hkv, hk = unit % a.Hkv;
  const int G = a.Hq / a.Hkv;
  const int nb0 = a.beam_start[r];
  const int W = a.beam_start[r + 1] - nb0;
  const int TG = a.T * G;
  const int rows_r = W * TG;
  if (nb0 < 0 || W < 0 || nb0 + W > a.num_beams) {  // beam_start is device data
    if (threadIdx.x == 0 && mt == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
    return;
  }
  const int row_base = mt * R16;
  if (row_base >= rows_r) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int rg = wave >> 1, ks = wave & 1;
  const int n16 = lane & 15, g4 = lane >> 4;
  using S = uint16_t;
  const S* qp = static_cast<const S*>(a.q);
  const S* kc = static_cast<const S*>(a.k_cache);
  const S* vc = static_cast<const S*>(a.v_cache);
  const int64_t head_off = (int64_t)hk * a.kv_head_stride;
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(lds);

  // ---- this lane's four rows (one per 16-row block) and their Q fragments
  const int b_lo = row_base / TG;
  int my_bi[4], my_qi[4], my_g[4];
  bool my_ok[4];
  u32x4_t qf[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int rho = row_base + rg * 64 + rb * 16 + n16;
    my_ok[rb] = rho < rows_r;
    const int b = rho / TG;
    my_bi[rb] = my_ok[rb] ? b - b_lo : -1;
    my_qi[rb] = (rho / G) % a.T;
    my_g[rb] = rho % G;
    const S* src = qp + (int64_t)((nb0 + b) * a.T + my_qi[rb]) * a.q_tok_stride + (int64_t)(hk * G + my_g[rb]) * HD +
                   8 * g4;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      qf[rb][c4] = my_ok[rb] ? *reinterpret_cast<const u32x4_t*>(src + 32 * c4) : u32x4_t{0, 0, 0, 0};
      // Q is only ever an MFMA operand: keep it in the accumulation registers
      __asm__ volatile("" : "+a"(qf[rb][c4]));
    }
  }
  const float c = SOFTCAP ? a.scale / a.softcap : a.scale * LOG2E;
  const float cap = a.softcap;

  // ---- the prefix: its length, and the block of a wave's rows of a tile
  // (a wave's 16 rows of a tile lie in one block: block size >= 16), read
  // with scalar loads
  const int pre_cap = a.prefix_bt_stride * a.bs;
  const int32_t* pbt = a.prefix_bt + (int64_t)r * a.prefix_bt_stride;
  const auto* pbt_c = (const __attribute__((address_space(4))) int32_t*)pbt;
  int P = a.prefix_len[r];
  if (P < 0 || P > pre_cap) {
    if (tid == 0) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
    P = P < 0 ? 0 : pre_cap;
  }
  const int bsh = a.bs_shift;
  const int n_pre = (P + K16 - 1) / K16;
  const int n_full = P / K16;
  auto pre_blk = [&](int t) __attribute__((always_inline)) -> int {
    const int key0 = t * K16 + 16 * wave_u;
    return key0 < P ? pbt_c[key0 >> bsh] : 0;
  };
  // an invalid block id reads block 0; it is reported after the loop
  bool bad_blk = false;
  auto checked = [&](int blk) __attribute__((always_inline)) -> int {
    const bool bad = (uint32_t)blk >= (uint32_t)a.num_blocks;
    bad_blk |= bad;
    return bad ? 0 : blk;
  };

  // ---- tile loads: wave w moves K and V rows 16 w .. 16 w + 15 of a tile,
  // four rows (1 KB of LDS) per instruction: lane i -> row 16 w + 4 j + (i >> 4),
  // physical chunk i & 15 (the swizzles pick which logical chunk it fetches).
  // Every wave issues exactly 8 loads per tile, tiles in order: the waits
  // count on it.
  const int q4 = lane >> 4, pch = lane & 15;
  const int ck0 = pch ^ q4, ck1 = pch ^ (q4 | 4);       // K: rows 4j + q4 for j < 2 and j >= 2
  const int cv = (((pch >> 1) ^ q4) << 1) | (pch & 1);  // V
  const int64_t tokb = a.kv_tok_stride;
  const uint32_t vo_k0 = (uint32_t)((q4 * tokb + ck0 * 8) * 2);
  const uint32_t vo_k1 = (uint32_t)((q4 * tokb + ck1 * 8) * 2);
  const uint32_t vo_v = (uint32_t)((q4 * tokb + cv * 8) * 2);
  const uint32_t blk_stride = (uint32_t)a.kv_block_stride;
  const void* zero = g_zero16b;
  // prefix tile t, the wave's rows in block blk (checked)
  auto issue_pre = [&](int t, int blk) __attribute__((always_inline)) {
    const uint32_t dst = lds0 + (t % NB) * BUFB + 16 * wave_u * ROWB;
    const int key0 = t * K16 + 16 * wave_u;
    const int64_t el =
        (int64_t)((uint64_t)(uint32_t)blk * blk_stride) + (int64_t)(key0 & (a.bs - 1)) * tokb + head_off;
    if (key0 + 16 <= P) {  // one uniform base address per instruction
#pragma unroll
      for (int j = 0; j < 4; ++j) dma_s(dst + j * 1024, kc + el + j * 4 * tokb, j < 2 ? vo_k0 : vo_k1);
#pragma unroll
      for (int j = 0; j < 4; ++j) dma_s(dst + KTB + j * 1024, vc + el + j * 4 * tokb, vo_v);
    } else {  // the end of the prefix: zero rows past it
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = key0 + 4 * j + q4 < P;
        const int64_t e = el + (4 * j + q4) * tokb;
        dma_v(dst + j * 1024, ok ? static_cast<const void*>(kc + e + (j < 2 ? ck0 : ck1) * 8) : zero);
        dma_v(dst + KTB + j * 1024, ok ? static_cast<const void*>(vc + e + cv * 8) : zero);
      }
    }
  };
  // suffix tile t: rows gathered through the per-key table built below, tags
  // (beam index << 16 | position in the beam's suffix; -1: a zero row) to info_s
  int tot = 0;
  int nbw = 0;
  auto suf_src = [&](int gs, int64_t& off) __attribute__((always_inline)) -> int {
    int tag = -1, bp = 0;
    if (gs < SKT) {
      const int2 e = suf_key[gs];
      tag = e.x;
      bp = e.y;
    } else {  // past the table: find the beam (skipping empty ones) and its block
      int lo = 0, hi = nbw - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (suf_cum[mid] <= gs) lo = mid; else hi = mid - 1;
      }
      const int j = gs - suf_cum[lo];
      const int pos = suf_s0[lo] + j;
      const int blk = suf_bt[lo * a.suffix_bt_stride + (pos >> bsh)];
      if (blk >= 0 && blk < a.num_blocks) {
        tag = (lo << 16) | j;
        bp = (blk << 8) | (pos & (a.bs - 1));
      }
    }
    off = (int64_t)((uint64_t)(uint32_t)(bp >> 8) * blk_stride) + (int64_t)(bp & 255) * tokb + head_off;
    return tag;
  };
  auto issue_suf = [&](int t) __attribute__((always_inline)) {
    const uint32_t dst = lds0 + (t % NB) * BUFB + 16 * wave_u * ROWB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 16 * wave_u + 4 * j + q4;
      const int gs = (t - n_pre) * K16 + row;
      int64_t off = 0;
      const int tag = gs < tot ? suf_src(gs, off) : -1;
      const bool ok = tag >= 0;
      dma_v(dst + j * 1024, ok ? static_cast<const void*>(kc + off + (j < 2 ? ck0 : ck1) * 8) : zero);
      dma_v(dst + KTB + j * 1024, ok ? static_cast<const void*>(vc + off + cv * 8) : zero);
      if (pch == 0) info_s[t % NB][row] = tag;
    }
  };
  int blk_pf = 0;  // the raw pre_blk of the next prefix tile to issue
  // issue tile t (blk: its checked block when a prefix tile)
  auto issue_any = [&](int t, int blk) __attribute__((always_inline)) {
    if (t < n_pre) issue_pre(t, blk);
    else issue_suf(t);
  };

  // ---- the first prefix tiles go out before the suffix metadata is read
  const int n_early = min(n_pre, 3);
  for (int t = 0; t < n_early; ++t) issue_pre(t, checked(pre_blk(t)));

  // ---- the workgroup's beams' suffix metadata and per-key gather table
  const int suf_cap = a.suffix_bt_stride * a.bs;
  nbw = min(W - 1, (min(row_base + R16, rows_r) - 1) / TG) - b_lo + 1;  // 1 .. MAXB
  int slen = 0;
  if (tid < nbw) {
    const int n = nb0 + b_lo + tid;
    const int L = a.suffix_len[n];
    const int s0 = a.suffix_start ? a.suffix_start[n] : 0;
    slen = (L < 0 || s0 < 0 || s0 + L > suf_cap) ? 0 : L;
    if (slen != L) flag_status(a.dev_status, GR_DEV_BAD_LENGTH);
    suf_s0[tid] = s0;
  }
  // the beams' suffix block tables (the launcher checks they fit)
  for (int i = tid; i < nbw * a.suffix_bt_stride; i += T16)
    suf_bt[i] = a.suffix_bt[(int64_t)(nb0 + b_lo) * a.suffix_bt_stride + i];
  {  // exclusive scan of the suffix lengths over the workgroup's beams
    int incl = slen;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    if (lane == 63) scan_tmp[wave] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += scan_tmp[w];
    if (tid < nbw) suf_cum[tid + 1] = base + incl;
    if (tid == 0) {
      suf_cum[0] = 0;
      hot_flag = 0;
    }
  }
  __syncthreads();
  tot = suf_cum[nbw];
  // suffix key gs (< SKT): {tag, block << 8 | position in the block}
  for (int gs = tid; gs < min(tot, SKT); gs += T16) {
    int lo = 0, hi = nbw - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (suf_cum[mid] <= gs) lo = mid; else hi = mid - 1;
    }
    const int j = gs - suf_cum[lo];
    const int pos = suf_s0[lo] + j;
    const int blk = suf_bt[lo * a.suffix_bt_stride + (pos >> bsh)];
    const bool ok = blk >= 0 && blk < a.num_blocks;
    if (!ok) flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
    suf_key[gs] = ok ? make_int2((lo << 16) | j, (blk << 8) | (pos & (a.bs - 1))) : make_int2(-1, 0);
  }
  __syncthreads();
  const int n_all = n_pre + (tot + K16 - 1) / K16;
  // this lane's rows: beam length limit (bottom-right causal over the suffix)
  int my_lim[4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
    my_lim[rb] = my_ok[rb] ? suf_cum[my_bi[rb] + 1] - suf_cum[my_bi[rb]] - a.T + my_qi[rb] : -1;
  for (int t = n_early; t < min(n_all, 3); ++t) issue_suf(t);
  if (3 < n_pre) blk_pf = pre_blk(3);

  // ---- this lane's fragment offsets
  uint32_t koff[4], voff[4];
  {
    const int row = 32 * ks + 8 * (n16 >> 2) + (n16 & 3);  // key(0, n16) of this half
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) koff[c4] = row * ROWB + ((4 * c4 + g4) ^ kswz(row)) * 16;
    const int q = n16 >> 2;
    const int vrow = 32 * ks + 8 * g4 + q;
#pragma unroll
    for (int d = 0; d < 4; ++d) voff[d] = KTB + vrow * ROWB + (d ^ q) * 32 + (n16 & 3) * 8;
  }
  // visibility of the lane's keys in tile t: bit 4t2 + i = key 8 g4 + 4 t2 + i of the half
  auto vis_bits = [&](int t, uint32_t (&vis)[4]) __attribute__((always_inline)) {
    if (t < n_pre) {
      const int k0 = t * K16 + 32 * ks + 8 * g4;
      uint32_t v = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) v |= (k0 + j < P ? 1u : 0u) << j;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) vis[rb] = v;
      return;
    }
    const int4 i0 = *reinterpret_cast<const int4*>(&info_s[t % NB][32 * ks + 8 * g4]);
    const int4 i1 = *reinterpret_cast<const int4*>(&info_s[t % NB][32 * ks + 8 * g4 + 4]);
    const int tags[8] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      uint32_t v = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v |= (tags[j] >= 0 && (tags[j] >> 16) == my_bi[rb] && (tags[j] & 0xFFFF) <= my_lim[rb] ? 1u : 0u) << j;
      vis[rb] = v;
    }
  };

  f32x4_t o[8][4];
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) o[db][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  St16 st;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    st.m[rb] = -INFINITY;
    st.l[rb] = 0.f;
  }

  // ---- tiles 0 and 1 in LDS (tile 2 may be in flight), S^T of tile 0
  if (n_all > 2) tile_barrier<8>();
  else tile_barrier<0>();
  f32x4_t s[2][4];  // S^T: row block rb holds tile t until weighted, then tile t+1
  bool hot_lane = false;
  u32x4_t p[4];
  if (n_all > 0) {  // S^T of tile 0, the rows' references, the weights of row block 0
    u32x4_t kf[4][2];
    read_k(lds0, koff, kf);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) qk_rb<DT>(rb, kf, qf, s);
    uint32_t vis[4];
    vis_bits(0, vis);
    tile_max<SOFTCAP>(s, vis, c, cap, st.m);  // (O is still zero)
    hot_lane |= weights_rb<DT, SOFTCAP, true>(s, 0, vis[0], st, c, cap, p[0]);
  }
  // step t (row block 0 of tile t already weighted): tile t+3's loads first,
  // then every fragment read of the step (K of tile t+1, V of tile t); then
  // four phases of 16 MFMAs, each beside the weights of one row block:
  //   QK(t+1) rb 0, 1   | weights(t) rb 1
  //   QK(t+1) rb 2, PV(t) rb 0 | weights(t) rb 2
  //   QK(t+1) rb 3, PV(t) rb 1 | weights(t) rb 3
  //   PV(t) rb 2, 3     | weights(t+1) rb 0
  // (a row block's weights read its S^T before its QK overwrites it), then
  // the barrier that sees tile t+2 landed.  FAST: tiles t+1 .. t+3 are whole
  // prefix tiles, every key of tiles t and t+1 visible.
  auto step = [&](int t, auto fast_c, auto nxt_c) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast_c)::value;
    constexpr bool NXT = decltype(nxt_c)::value;
    constexpr bool MSK = !FAST;
    const bool more = FAST || t + 3 < n_all;
    if (FAST) issue_pre(t + 3, checked(blk_pf));
    else if (more) issue_any(t + 3, checked(blk_pf));
    if (t + 4 < n_pre) blk_pf = pre_blk(t + 4);
    u32x4_t kf[4][2], vf[8];
    if (NXT) read_k(lds0 + ((t + 1) % NB) * BUFB, koff, kf);
    read_v(lds0 + (t % NB) * BUFB, voff, vf);
    uint32_t vis[4] = {0xFFu, 0xFFu, 0xFFu, 0xFFu}, vis1[4] = {0xFFu, 0xFFu, 0xFFu, 0xFFu};
    if (!FAST) {
      vis_bits(t, vis);
      if (NXT) vis_bits(t + 1, vis1);
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr int QK = NXT ? 0 : 2;
    hot_lane |= phase16<DT, SOFTCAP, MSK, QK, 0, QK, 1, 1>(s, o, p, kf, vf, qf, vis[1], st, c, cap);
    hot_lane |= phase16<DT, SOFTCAP, MSK, 1, 0, QK, 2, 2>(s, o, p, kf, vf, qf, vis[2], st, c, cap);
    hot_lane |= phase16<DT, SOFTCAP, MSK, 1, 1, QK, 3, 3>(s, o, p, kf, vf, qf, vis[3], st, c, cap);
    hot_lane |= phase16<DT, SOFTCAP, MSK, 1, 2, 1, 3, NXT ? 0 : -1>(s, o, p, kf, vf, qf, vis1[0], st, c, cap);
    if (more) tile_barrier<8>();
    else tile_barrier<0>();
  };
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  int t = 0;
  if (n_all > 1) step(0, F_{}, T_{});
  for (t = 1; t + 3 < n_full; ++t) step(t, T_{}, T_{});
  for (t = max(t, 1); t + 1 < n_all; ++t) step(t, F_{}, T_{});
  if (n_all > 0) step(n_all - 1, F_{}, F_{});
  if (bad_blk && lane == 0) flag_status(a.dev_status, GR_DEV_BAD_BLOCK);
  if (__ballot(hot_lane) != 0 && lane == 0) hot_flag = 1;
  __syncthreads();
  if (hot_flag) {
    // exact recomputation in two passes, one tile at a time: the rows' maxima
    // over every visible key, then the weights against them (none above 1,
    // so O is never rescaled)
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (int u = 0; u < n_all; ++u) {
      issue_any(u, u < n_pre ? checked(pre_blk(u)) : 0);
      tile_barrier<0>();
      u32x4_t kf[4][2];
      read_k(lds0 + (u % NB) * BUFB, koff, kf);
      f32x4_t s1[2][4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) qk_rb<DT>(rb, kf, qf, s1);
      uint32_t vis[4];
      vis_bits(u, vis);
      float tm[4];
      tile_max<SOFTCAP>(s1, vis, c, cap, tm);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) mx[rb] = fmaxf(mx[rb], tm[rb]);
      tile_barrier<0>();
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      st.m[rb] = mx[rb];
      st.l[rb] = 0.f;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) o[db][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int u = 0; u < n_all; ++u) {
      issue_any(u, u < n_pre ? checked(pre_blk(u)) : 0);
      tile_barrier<0>();
      u32x4_t kf[4][2], vf[8];
      read_k(lds0 + (u % NB) * BUFB, koff, kf);
      read_v(lds0 + (u % NB) * BUFB, voff, vf);
      f32x4_t s1[2][4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) qk_rb<DT>(rb, kf, qf, s1);
      uint32_t vis[4];
      vis_bits(u, vis);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) weights_rb<DT, SOFTCAP, true>(s1, rb, vis[rb], st, c, cap, p[rb]);
      pv_mma<DT>(vf, p, o);
      tile_barrier<0>();
    }
  }

  // ---- merge the two key halves and write O, LSE
  f32x4_t* xo = reinterpret_cast<f32x4_t*>(lds) + rg * (8 * 4 * 64);                   // [rg][db][rb][lane]
  float2* xm = reinterpret_cast<float2*>(reinterpret_cast<f32x4_t*>(lds) + 2 * (8 * 4 * 64)) + rg * (4 * 64);  // [rg][rb][lane]
  if (ks == 1) {
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) xo[(db * 4 + rb) * 64 + lane] = o[db][rb];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) xm[rb * 64 + lane] = make_float2(st.m[rb], st.l[rb]);
  }
  __syncthreads();
  if (ks == 0) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const float2 ml = xm[rb * 64 + lane];
      const float m1 = ml.x, l1 = ml.y;
      const float m0 = st.m[rb], l0 = st.l[rb];
      const float m = fmaxf(m0, m1);
      const float a0 = m0 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m0 - m);
      const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
      const float lrow = row_sum4(l0 * a0 + l1 * a1);
      const float inv = lrow > 0.f ? 1.f / lrow : 0.f;
      if (!my_ok[rb]) continue;
      const int b = my_bi[rb] + b_lo;
      const int64_t tok = (int64_t)(nb0 + b) * a.T + my_qi[rb];
      S* dst = static_cast<S*>(a.out) + tok * a.out_tok_stride + (int64_t)(hk * G + my_g[rb]) * HD + 4 * g4;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const f32x4_t x1 = xo[(db * 4 + rb) * 64 + lane];
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (o[db][rb][i] * a0 + x1[i] * a1) * inv;
        const u32x2_t w = {M16<DT>::pack2(v[0], v[1]), M16<DT>::pack2(v[2], v[3])};
        *reinterpret_cast<u32x2_t*>(dst + 16 * db) = w;
      }
      if (a.lse_out && g4 == 0)
        a.lse_out[tok * a.Hq + hk * G + my_g[rb]] =
            lrow > 0.f ? (m + __builtin_amdgcn_logf(lrow)) * 0.6931471805599453f : -INFINITY;
    }
  }
}

}  // namespace

bool d16_decode_supported(const DecodeArgs& a) {
  if (!mfma_decode_supported(a)) return false;
  // a wave's 16 rows of a prefix tile lie in one block; the suffix gather
  // table packs block << 8 | position in the block into 31 bits
  if (a.bs_shift < 4 || a.bs_shift > 8 || a.num_blocks > (1 << 23)) return false;
  // suffix keys are tagged with their 16-bit index within the beam's suffix
  if ((int64_t)a.suffix_bt_stride * a.bs > 0xFFFF) return false;
  // the block tables of the beams one workgroup's rows touch fit in LDS
  const int TG = a.T * (a.Hq / a.Hkv);
  return (int64_t)(127 / TG + 2) * a.suffix_bt_stride <= SBT;
}

gr_status_t launch_d16_decode(const DecodeArgs& a, hipStream_t stream) {
  const int G = a.Hq / a.Hkv;
  const int64_t rows = (int64_t)a.max_beams * a.T * G;
  const int64_t mt64 = (rows + R16 - 1) / R16;
  const int units = a.num_reqs * a.Hkv;
  if (mt64 == 0 || units == 0) return GR_OK;
  const int64_t nwg = (int64_t)((units + 7) / 8) * 8 * mt64;
  if (nwg > 0x7fffffff) return GR_ERR_INVALID_ARG;
  const int mtiles = (int)mt64;
  const bool cap = a.softcap > 0.f;
  const dim3 grid((unsigned)nwg);
  if (a.dtype == GR_DTYPE_BF16) {
    if (cap) hipLaunchKernelGGL((decode_d16<GR_DTYPE_BF16, true>), grid, dim3(T16), 0, stream, a, units, mtiles);
    else hipLaunchKernelGGL((decode_d16<GR_DTYPE_BF16, false>), grid, dim3(T16), 0, stream, a, units, mtiles);
  } else {
    if (cap) hipLaunchKernelGGL((decode_d16<GR_DTYPE_F16, true>), grid, dim3(T16), 0, stream, a, units, mtiles);
    else hipLaunchKernelGGL((decode_d16<GR_DTYPE_F16, false>), grid, dim3(T16), 0, stream, a, units, mtiles);
  }
  return launch_status();
}

}  // namespace gr
