// MFMA tile helpers of the BeamAttention matrix-core kernel (gr_attn_mfma.hip).
//
// MFMA formulation (v_mfma_f32_32x32x16_{bf16,f16}, wave64):
//   S^T[key][row]  = K[key][:] . Q[row][:]    A = K tile, B = Q^T (registers)
//   O^T[d][row]   += V^T[d][key] . P^T[key][row]
// so every lane owns one query row (lane % 32) in both accumulators and the
// online softmax needs no cross-lane traffic except the lane-pair (l, l^32)
// max/sum.  K rows are fed to the A operand through the permutation PI that
// swaps bits 2 and 3 of the row index; with it the S^T accumulator registers
// of each lane hold keys in exactly the order the PV B operand needs.  V stays
// in its natural [key][d] layout in LDS (64-byte segments XOR-swizzled per
// row, see vchunk) and the V^T operand is assembled with
// gfx950's transposing LDS read (ds_read_b64_tr_b16): in each 16-lane group,
// source lane s addresses V[k0 + s/4][d0 + 4*(s%4) .. +3] and lane i receives
// V[k0 .. k0+3][d0 + i].
#pragma once

#include "gr_attn_decode.h"

namespace gr {
namespace {

constexpr int ST_KEYS = 64;    // keys per super-tile (two 32-key halves)
constexpr int HD = 128;        // head dim
constexpr int KS_PITCH = 128;  // K tile row pitch in elements (256 B); 16-byte chunks XOR-swizzled
constexpr int VS_PITCH = 128;  // V tile row pitch in elements (256 B); 64-byte segments XOR-swizzled
constexpr int K_TILE = ST_KEYS * KS_PITCH;
constexpr int V_TILE = ST_KEYS * VS_PITCH;
constexpr int BUF = K_TILE + V_TILE;  // elements per buffer (32 KB)
constexpr float LOG2E = 1.4426950408889634f;
// Lazy softmax reference: a key may exceed the row's reference by up to
// Rescale::THRESH log2 units before the exact path moves the reference; a lane
// weight sum above 2^Rescale::THRESH forces it.  The packed P operand bounds
// the margin: 60 for bf16 (range to 2^127), 15 for fp16 (largest finite value
// 65504 < 2^16).
template <int DT> struct Rescale;
template <> struct Rescale<GR_DTYPE_BF16> {
  static constexpr float THRESH = 60.0f;
  static constexpr float SUM = 1.152921504606846976e18f;  // 2^60
};
template <> struct Rescale<GR_DTYPE_F16> {
  static constexpr float THRESH = 15.0f;
  static constexpr float SUM = 32768.0f;  // 2^15
};
static_assert(Rescale<GR_DTYPE_BF16>::SUM == (float)(1ull << 60) && Rescale<GR_DTYPE_F16>::SUM == (float)(1 << 15),
              "Rescale::SUM is 2^THRESH");

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));
typedef uint32_t u32x4_t __attribute__((__vector_size__(4 * sizeof(uint32_t))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));
typedef uint32_t u32x2_t __attribute__((__vector_size__(2 * sizeof(uint32_t))));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Zero source for loads of keys outside the prefix or in an invalid block.
__device__ __attribute__((aligned(16))) uint32_t g_zero16[4];

template <int DT> struct Mma;
template <> struct Mma<GR_DTYPE_BF16> {
  using vec = bf16x8_t;
  __device__ static inline f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(vec, a),
                                                   __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});  // one v_cvt_pk_bf16_f32
  }
  __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};
template <> struct Mma<GR_DTYPE_F16> {
  using vec = f16x8_t;
  __device__ static inline f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(vec, a),
                                                  __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, f16x2_t{(_Float16)lo, (_Float16)hi});
  }
  __device__ static inline float lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[0]; }
  __device__ static inline float hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[1]; }
};

// Eight OCP e4m3 bytes (two dwords, element 0 in the low byte) as eight
// bf16 / fp16 values (exact: e4m3 fits both).
template <int DT> struct Fp8Cvt;
template <> struct Fp8Cvt<GR_DTYPE_BF16> {
  __device__ static inline u32x4_t x8(uint32_t w0, uint32_t w1) {
    return u32x4_t{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true))};
  }
};
template <> struct Fp8Cvt<GR_DTYPE_F16> {
  __device__ static inline u32x4_t x8(uint32_t w0, uint32_t w1) {
    return u32x4_t{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true))};
  }
};

// S^T row slot i holds tile key PI(i): bits 2 and 3 swapped.
__device__ inline int key_perm(int i) { return (i & 0x13) | ((i & 4) << 1) | ((i & 8) >> 1); }

// Physical 16-byte chunk of logical chunk c in K tile row `row`.  The A
// operand reads rows PI(0..7) = {0..3, 8..11} (and +4, +16) in one 8-lane
// group; the XOR spreads those rows over 8 distinct 16-byte bank groups.
__device__ inline int kchunk(int row, int c) { return c ^ ((row & 3) | (((row >> 3) & 1) << 2)); }
// Physical 16-byte chunk of logical chunk c in V tile row `row`: the 64-byte
// segment c >> 2 (32 dims) sits at segment (c >> 2) ^ (row & 3), so the four
// rows that one half-wave of a transposing read touches (keys k0 .. k0 + 3,
// 64 bytes each) cover all 64 banks.
__device__ inline int vchunk(int row, int c) { return (((c >> 2) ^ (row & 3)) << 2) | (c & 3); }

typedef short s16x4_t __attribute__((ext_vector_type(4)));
// 4 keys x 1 dim per lane via the transposing LDS read (see the header comment)
__device__ inline uint2 lds_read_tr(const uint16_t* p) {
  auto v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(reinterpret_cast<uintptr_t>(p)));
  return __builtin_bit_cast(uint2, v);
}

// Value of x held by lane l ^ 32 (the other lane of the same query row).
// v_permlane32_swap exchanges the upper 32 lanes of its first operand with the
// lower 32 lanes of its second: with both operands = x, lanes 0..31 find the
// partner in the second result and lanes 32..63 in the first.  The half is
// selected explicitly: the compiler folds fmaxf(v[0], v[1]) to v[0] when both
// operands are the same value, which drops the partner on lanes 0..31.
__device__ inline float lane_partner(float x) {
  auto v = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                            __builtin_bit_cast(uint32_t, x), false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? v[0] : v[1]);
}
// max / sum over the lane pair (l, l ^ 32); both lanes get the same result
__device__ inline float pair_max(float x) { return fmaxf(x, lane_partner(x)); }
__device__ inline float pair_sum(float x) { return x + lane_partner(x); }

__device__ inline u32x4_t lds_read16(const uint16_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// Per-lane online-softmax state of the lane's query row.
struct RowState {
  float m;     // running max in scaled log2 units (-inf before any visible key)
  float lsum;  // this lane's partial sum of exp2(x - m)
};

// Softmax of one 32-key x 32-row S^T tile held by this lane (16 keys of its
// row).  vis: bit r set when register r is a visible key.  Returns the
// rescale factor for O (1 when unchanged) and writes the packed P operand.
// log2-domain score of one S^T entry (c = scale * log2(e), or scale / softcap
// with the soft cap applied first)
// The cap's tanh is 1 - 2 / (2^(2x log2 e) + 1): one exp2 and one reciprocal
// (the hardware's, each within about an ulp) instead of the library tanhf's
// long branchy sequence, 16 times per step: 19 % off a soft-capped decode,
// 21 % off a prefill.  Exact at both ends (an exp2 that overflows to inf
// gives 1, one that underflows to 0 gives -1); near 0 its absolute error is
// about an ulp of 1, which the cap turns into ~1e-5 log2 units of a score,
// far inside the bf16 rounding of the weights.
template <bool SOFTCAP>
__device__ inline float score_l2(float v, float c, float cap) {
  if constexpr (SOFTCAP) {
    const float e = __builtin_amdgcn_exp2f(v * (c * (2.f * LOG2E)));
    const float t = fmaf(-2.f, __builtin_amdgcn_rcpf(e + 1.f), 1.f);
    return (cap * LOG2E) * t;
  } else {
    return v * c;
  }
}

// The additive term of a weight's exponent (log2 units) for register r of a
// lane's 16: the negated reference mref plus the key's own bias.  NoBias: none.
// LinBias: ALiBi's alpha * (key - qpos) over a tile's keys, b0 = the bias of
// the lane's first key (register r holds the key 16 (r >> 3) + (r & 7) past
// it).  ArrBias: one bias per register (gathered suffix keys).  The reference
// itself follows the scores without bias: an ALiBi bias is never positive for
// a key at or before the query, so it cannot push a weight past the bound the
// fast path checks.
struct NoBias {
  __device__ float operator()(int, float mref) const { return -mref; }
};
struct LinBias {
  float alpha, b0;
  __device__ float operator()(int r, float mref) const {
    return fmaf(alpha, (float)(16 * (r >> 3) + (r & 7)), b0 - mref);
  }
};
struct ArrBias {
  const float* b;
  __device__ float operator()(int r, float mref) const { return b[r] - mref; }
};

// A lane's 16 weights of one half-tile against the row's reference maximum
// mref (log2 domain), with no tile maximum: the branch-free common case.
// Weights are packed pairwise as they are produced (p0: registers 0..7, p1:
// 8..15).  Returns the lane's weight sum.  The caller sends the tile to
// softmax_exact when any lane's sum exceeds 2^Rescale::THRESH (some key is
// more than Rescale::THRESH above the reference) or is not finite (the row
// has no reference yet: mref = -inf makes every visible weight +inf).
template <int DT, bool SOFTCAP, bool MASKED, typename B = NoBias>
__device__ inline float softmax_fast(const f32x16_t& s, uint32_t vis, float mref, float c, float cap,
                                     u32x4_t& p0, u32x4_t& p1, const B& bias = B{}) {
  using M = Mma<DT>;
  float acc0 = 0.f, acc1 = 0.f;
  uint32_t pk[8];
#pragma unroll
  for (int r = 0; r < 16; r += 2) {
    float e0 = SOFTCAP ? __builtin_amdgcn_exp2f(score_l2<true>(s[r], c, cap) + bias(r, mref))
                       : __builtin_amdgcn_exp2f(fmaf(s[r], c, bias(r, mref)));
    float e1 = SOFTCAP ? __builtin_amdgcn_exp2f(score_l2<true>(s[r + 1], c, cap) + bias(r + 1, mref))
                       : __builtin_amdgcn_exp2f(fmaf(s[r + 1], c, bias(r + 1, mref)));
    if (MASKED) {
      e0 = (vis >> r) & 1 ? e0 : 0.f;
      e1 = (vis >> (r + 1)) & 1 ? e1 : 0.f;
    }
    acc0 += e0;
    acc1 += e1;
    pk[r >> 1] = M::pack2(e0, e1);
  }
  p0 = u32x4_t{pk[0], pk[1], pk[2], pk[3]};
  p1 = u32x4_t{pk[4], pk[5], pk[6], pk[7]};
  return acc0 + acc1;
}

// S^T of the wave's 32 rows against the 32-key half-tile at row kbase.
template <int DT>
__device__ inline f32x16_t qk_half(const uint16_t* buf, int kbase, int lane, const u32x4_t (&qf)[8]) {
  using M = Mma<DT>;
  const int krow_i = kbase + key_perm(lane & 31);
  const uint16_t* krow = buf + krow_i * KS_PITCH;
  const int lhalf = lane >> 5;
  f32x16_t s = {};
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    s = M::mma(lds_read16(krow + kchunk(krow_i, 2 * (kk & 3) + lhalf) * 8 + (kk >> 2) * 64), qf[kk], s);
  return s;
}

// Weight of one score given its exponent term negoff (the negated reference
// plus the key's bias, log2 domain).
template <bool SOFTCAP>
__device__ inline float weight1(float v, float c, float cap, float negoff) {
  return SOFTCAP ? __builtin_amdgcn_exp2f(score_l2<true>(v, c, cap) + negoff)
                 : __builtin_amdgcn_exp2f(fmaf(v, c, negoff));
}

// O += V^T . P^T over NH 32-key halves starting at row kbase.  The V^T
// operand: lane group g = lane/16 covers dims 16*(g&1) .. +15 of the 32-dim
// block and keys 8*(g>>1) .. +7 of the 16-key step (two 4-key transposing
// reads).  The four dim blocks are independent accumulators, issued in turn.
template <int DT, int NH>
__device__ inline void pv(const uint16_t* buf, int kbase, int lane, const u32x4_t (&p)[NH][2], f32x16_t (&o)[4]) {
  using M = Mma<DT>;
  const int g = lane >> 4, sl = lane & 15;
  // every row this lane reads has row & 3 == sl >> 2: dim block mb sits in segment mb ^ (sl >> 2)
  const uint16_t* vsrc = buf + K_TILE + (kbase + 8 * (g >> 1) + (sl >> 2)) * VS_PITCH + 16 * (g & 1) + 4 * (sl & 3);
#pragma unroll
  for (int h = 0; h < NH; ++h) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const uint16_t* vp = vsrc + (32 * h + 16 * kk) * VS_PITCH + 32 * (mb ^ (sl >> 2));
        const uint2 lo = lds_read_tr(vp);
        const uint2 hi = lds_read_tr(vp + 4 * VS_PITCH);
        o[mb] = M::mma(u32x4_t{lo.x, lo.y, hi.x, hi.y}, p[h][kk], o[mb]);
      }
    }
  }
}

// Weights of NH half-tiles of the wave's rows (one row per lane pair): the
// branch-free fast path against the row's reference, or -- when some weight
// could exceed 2^Rescale::THRESH or the row has no reference yet -- the exact
// path that moves the reference to the maximum over all NH halves and scales
// O (skipped while the row has accumulated nothing).
template <int DT, bool SOFTCAP, bool MASKED, int NH, typename B = NoBias>
__device__ inline void weights(const f32x16_t (&s)[NH], const uint32_t (&vis)[NH], RowState& st, float c, float cap,
                               u32x4_t (&p)[NH][2], f32x16_t (&o)[4], const B& bias = B{}) {
  static_assert(NH == 1 || sizeof(B) == sizeof(NoBias), "a bias covers one half-tile");
  float acc = 0.f;
  bool hot = false;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const float a_h = softmax_fast<DT, SOFTCAP, MASKED>(s[h], vis[h], st.m, c, cap, p[h][0], p[h][1], bias);
    hot |= !(a_h <= Rescale<DT>::SUM);
    acc += a_h;
  }
  if (__ballot(hot) == 0) {
    st.lsum += acc;
    return;
  }
  // exact path (wave-uniform; after a row's first tile it needs a score more
  // than Rescale::THRESH log2 units above everything before it).  The empty
  // volatile asm keeps the compiler from speculating this rare work into the
  // common path.
  __asm__ volatile("" ::: "memory");
  float mx = -INFINITY;
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float v = score_l2<SOFTCAP>(s[h][r], c, cap);
      mx = (!MASKED || ((vis[h] >> r) & 1)) ? fmaxf(mx, v) : mx;
    }
  mx = pair_max(mx);
  const float new_m = fmaxf(st.m, mx);
  const float alpha = st.m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m - new_m);
  const float mref = new_m == -INFINITY ? 0.f : new_m;
  const bool had_mass = st.lsum > 0.f;
  st.m = new_m;
  float acc2 = 0.f;
#pragma unroll
  for (int h = 0; h < NH; ++h)
    acc2 += softmax_fast<DT, SOFTCAP, MASKED>(s[h], vis[h], mref, c, cap, p[h][0], p[h][1], bias);
  st.lsum = st.lsum * alpha + acc2;
  if (__ballot(had_mass && alpha != 1.f) != 0) {
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) o[mb] *= alpha;
  }
}

// Phase A of a pipelined step of a wave over its 32-key half of a fully
// visible tile: in 8 fixed segments, one MFMA of the next tile's QK^T (with
// the LDS read of the fragment two MFMAs ahead) beside the weights of two
// scores of the current tile against the row's reference.  s_in holds S^T of
// the current tile, s_out receives that of the next tile (the caller
// alternates two register sets: no copies).  Returns true when some weight
// could exceed 2^Rescale::THRESH or the row has no reference yet (the tile then
// needs the exact path); otherwise adds the weight sum to the row's state.
// DEFER: no wave vote -- the lane's sum is always added and the lane's own
// flag returned (the caller votes once, after its loop, and recomputes).
template <int DT, bool SOFTCAP, bool DEFER = false, typename B = NoBias>
__device__ inline bool phase_a1(const uint16_t* next_buf, int kbase, int lane, const u32x4_t (&qf)[8],
                                const f32x16_t& s_in, f32x16_t& s_out, RowState& st, float c, float cap,
                                u32x4_t (&p)[1][2], const B& bias = B{}) {
  using M = Mma<DT>;
  const int lhalf = lane >> 5;
  const int krow_i = kbase + key_perm(lane & 31);
  const uint16_t* krow = next_buf + krow_i * KS_PITCH;
  // the swizzle leaves chunk bit 3 alone: fragments kk and kk + 4 sit 64
  // elements apart, so four lane addresses serve all eight reads
  auto kfrag = [&](int kk) { return lds_read16(krow + kchunk(krow_i, 2 * (kk & 3) + lhalf) * 8 + (kk >> 2) * 64); };
  const float mref = st.m;
  u32x4_t kf[8];
  kf[0] = kfrag(0);
  kf[1] = kfrag(1);
  s_out = f32x16_t{};
  uint32_t pk[8];
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i + 2 < 8) kf[i + 2] = kfrag(i + 2);
    s_out = M::mma(kf[i], qf[i], s_out);
    const float e0 = weight1<SOFTCAP>(s_in[2 * i], c, cap, bias(2 * i, mref));
    const float e1 = weight1<SOFTCAP>(s_in[2 * i + 1], c, cap, bias(2 * i + 1, mref));
    acc0 += e0;
    acc1 += e1;
    pk[i] = M::pack2(e0, e1);
    // keeps this segment's weights, sums and packing beside its MFMA (without
    // it the instruction selector may gather them after the last MFMAs)
    __asm__ volatile("" : "+v"(acc0), "+v"(acc1), "+v"(pk[i]));
    __builtin_amdgcn_sched_barrier(0);
  }
  p[0][0] = u32x4_t{pk[0], pk[1], pk[2], pk[3]};
  p[0][1] = u32x4_t{pk[4], pk[5], pk[6], pk[7]};
  const float acc = acc0 + acc1;
  if constexpr (DEFER) {
    st.lsum += acc;
    return !(acc <= Rescale<DT>::SUM);
  }
  if (__ballot(!(acc <= Rescale<DT>::SUM)) != 0) return true;
  st.lsum += acc;
  return false;
}

// Phase C: the current tile's PV with its transposing reads two MFMAs ahead
// (MFMA j: step kk = j/4, dim block mb = j%4).
template <int DT>
__device__ inline void phase_c1(const uint16_t* cur_buf, int kbase, int lane, const u32x4_t (&p)[1][2],
                                f32x16_t (&o)[4]) {
  using M = Mma<DT>;
  const int g = lane >> 4, sl = lane & 15;
  const uint16_t* vsrc = cur_buf + K_TILE + (kbase + 8 * (g >> 1) + (sl >> 2)) * VS_PITCH + 16 * (g & 1) + 4 * (sl & 3);
  auto vfrag = [&](int j) {
    const uint16_t* vp = vsrc + (16 * (j >> 2)) * VS_PITCH + 32 * ((j & 3) ^ (sl >> 2));
    const uint2 lo = lds_read_tr(vp);
    const uint2 hi = lds_read_tr(vp + 4 * VS_PITCH);
    return u32x4_t{lo.x, lo.y, hi.x, hi.y};
  };
  u32x4_t vf[8];
  vf[0] = vfrag(0);
  vf[1] = vfrag(1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j + 2 < 8) vf[j + 2] = vfrag(j + 2);
    o[j & 3] = M::mma(vf[j], p[0][j >> 2], o[j & 3]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Phases A and C of a lean step in one body: the first two K fragment reads go
// out before `mid` (the step's tile loads: scalar work that covers their
// latency), and the first two V^T fragment reads of phase C during the last
// two QK MFMAs, so neither phase starts on an LDS round trip.  Same
// arithmetic, in the same order, as phase_a1<DEFER> followed by phase_c1.
template <int DT, bool SOFTCAP, typename Mid, typename B = NoBias>
__device__ inline bool phase_ac(const uint16_t* next_buf, const uint16_t* cur_buf, int kbase, int lane,
                                const u32x4_t (&qf)[8], const f32x16_t& s_in, f32x16_t& s_out, RowState& st, float c,
                                float cap, f32x16_t (&o)[4], Mid&& mid, const B& bias = B{}) {
  using M = Mma<DT>;
  const int lhalf = lane >> 5;
  const int krow_i = kbase + key_perm(lane & 31);
  const uint16_t* krow = next_buf + krow_i * KS_PITCH;
  auto kfrag = [&](int kk) { return lds_read16(krow + kchunk(krow_i, 2 * (kk & 3) + lhalf) * 8 + (kk >> 2) * 64); };
  const int g = lane >> 4, sl = lane & 15;
  const uint16_t* vsrc = cur_buf + K_TILE + (kbase + 8 * (g >> 1) + (sl >> 2)) * VS_PITCH + 16 * (g & 1) + 4 * (sl & 3);
  auto vfrag = [&](int j) {
    const uint16_t* vp = vsrc + (16 * (j >> 2)) * VS_PITCH + 32 * ((j & 3) ^ (sl >> 2));
    const uint2 lo = lds_read_tr(vp);
    const uint2 hi = lds_read_tr(vp + 4 * VS_PITCH);
    return u32x4_t{lo.x, lo.y, hi.x, hi.y};
  };
  const float mref = st.m;
  u32x4_t kf[8];
  kf[0] = kfrag(0);
  kf[1] = kfrag(1);
  __builtin_amdgcn_sched_barrier(0);
  mid();
  __builtin_amdgcn_sched_barrier(0);
  s_out = f32x16_t{};
  uint32_t pk[8];
  u32x4_t vf[8];
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i + 2 < 8) kf[i + 2] = kfrag(i + 2);
    else vf[i - 6] = vfrag(i - 6);
    s_out = M::mma(kf[i], qf[i], s_out);
    const float e0 = weight1<SOFTCAP>(s_in[2 * i], c, cap, bias(2 * i, mref));
    const float e1 = weight1<SOFTCAP>(s_in[2 * i + 1], c, cap, bias(2 * i + 1, mref));
    acc0 += e0;
    acc1 += e1;
    pk[i] = M::pack2(e0, e1);
    __asm__ volatile("" : "+v"(acc0), "+v"(acc1), "+v"(pk[i]));
    __builtin_amdgcn_sched_barrier(0);
  }
  const u32x4_t p0 = u32x4_t{pk[0], pk[1], pk[2], pk[3]};
  const u32x4_t p1 = u32x4_t{pk[4], pk[5], pk[6], pk[7]};
  const float acc = acc0 + acc1;
  st.lsum += acc;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j + 2 < 8) vf[j + 2] = vfrag(j + 2);
    o[j & 3] = M::mma(vf[j], j < 4 ? p0 : p1, o[j & 3]);
    __builtin_amdgcn_sched_barrier(0);
  }
  return !(acc <= Rescale<DT>::SUM);
}

// One pipelined step with the exact path in line (phase A; the exact weights
// when phase A reports it; phase C).
template <int DT, bool SOFTCAP, typename B = NoBias>
__device__ inline void pipe_step(const uint16_t* cur_buf, const uint16_t* next_buf, int kbase, int lane,
                                 const u32x4_t (&qf)[8], const f32x16_t& s_in, f32x16_t& s_out,
                                 f32x16_t (&o)[4], RowState& st, float c, float cap, const B& bias = B{}) {
  u32x4_t p[1][2];
  if (phase_a1<DT, SOFTCAP, false, B>(next_buf, kbase, lane, qf, s_in, s_out, st, c, cap, p, bias)) {
    __asm__ volatile("" ::: "memory");
    const uint32_t vis[1] = {0xFFFFu};
    const f32x16_t s1[1] = {s_in};
    weights<DT, SOFTCAP, false, 1>(s1, vis, st, c, cap, p, o, bias);
  }
  phase_c1<DT>(cur_buf, kbase, lane, p, o);
}


}  // namespace
}  // namespace gr
