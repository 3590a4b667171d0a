// Shared device/host helpers for the gfx950 beam path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gr_beam.h"

#define GR_VERSION_CODE 100  // 0.1.0

namespace gr {

// ---- kernel arguments ------------------------------------------------------
// A kernel reads its arguments through the scalar cache where the code first
// uses them, and the compiler waits for each read before work that needs it,
// so arguments that span several 64-byte lines can cost one cache miss per
// line, in turn, on the kernel's critical path.  kernarg_lines<N>() reads one
// dword of each of the first N lines (N * 64 <= the explicit arguments'
// size, rounded up) in one statement that then waits once, so the misses
// overlap; call it first in the kernel.  Loads only: nothing is written.
template <int N>
__device__ __forceinline__ void kernarg_lines() {
  static_assert(N >= 1 && N <= 12, "one to twelve lines");
  int d0, d1, d2, d3, d4, d5, d6, d7, d8, d9, d10, d11;
  __asm__ volatile(
      "s_load_dword %0, %12, 0x0\n\t"
      ".if %13 > 1\n\ts_load_dword %1, %12, 0x40\n\t.endif\n\t"
      ".if %13 > 2\n\ts_load_dword %2, %12, 0x80\n\t.endif\n\t"
      ".if %13 > 3\n\ts_load_dword %3, %12, 0xc0\n\t.endif\n\t"
      ".if %13 > 4\n\ts_load_dword %4, %12, 0x100\n\t.endif\n\t"
      ".if %13 > 5\n\ts_load_dword %5, %12, 0x140\n\t.endif\n\t"
      ".if %13 > 6\n\ts_load_dword %6, %12, 0x180\n\t.endif\n\t"
      ".if %13 > 7\n\ts_load_dword %7, %12, 0x1c0\n\t.endif\n\t"
      ".if %13 > 8\n\ts_load_dword %8, %12, 0x200\n\t.endif\n\t"
      ".if %13 > 9\n\ts_load_dword %9, %12, 0x240\n\t.endif\n\t"
      ".if %13 > 10\n\ts_load_dword %10, %12, 0x280\n\t.endif\n\t"
      ".if %13 > 11\n\ts_load_dword %11, %12, 0x2c0\n\t.endif\n\t"
      "s_waitcnt lgkmcnt(0)"
      // early-clobber outputs: a destination must never share a register
      // with the base address, which later loads of the statement still read
      // while earlier ones are pending (a load may return between the two)
      : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7), "=&s"(d8),
        "=&s"(d9), "=&s"(d10), "=&s"(d11)
      : "s"(__builtin_amdgcn_kernarg_segment_ptr()), "n"(N));
  __builtin_amdgcn_sched_barrier(0);  // no argument read moves above it
}
template <typename T> constexpr int kernarg_line_count(int extra_bytes = 0) {
  return (int)((sizeof(T) + extra_bytes + 63) / 64);
}

// ---- wave prefix sums --------------------------------------------------------
// Inclusive prefix sum of one int per lane over the wave's 64 lanes (L = 64)
// or over each 32-lane half (L = 32), by DPP moves: within each row of 16
// lanes, shifts by 1, 2 and 3 of the inputs, then by 4 (banks 1-3) and 8
// (banks 2-3) of the partial sums; across rows, row 0's and row 2's last
// lanes broadcast into rows 1 and 3 (row_bcast:15), then lane 31 into rows 2
// and 3 (row_bcast:31).  A lane whose source lies outside its row, or whose
// row or bank is masked off, adds 0.  No LDS round trip and no lane-address
// arithmetic, against six of each for a shuffle-based scan.
template <int L = 64>
__device__ __forceinline__ int wave_incl_scan(int v) {
  static_assert(L == 32 || L == 64, "a wave or each half");
  int s = v;
  s += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  s += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  s += __builtin_amdgcn_update_dpp(0, v, 0x113, 0xf, 0xf, true);  // row_shr:3
  s += __builtin_amdgcn_update_dpp(0, s, 0x114, 0xf, 0xe, true);  // row_shr:4, banks 1-3
  s += __builtin_amdgcn_update_dpp(0, s, 0x118, 0xf, 0xc, true);  // row_shr:8, banks 2-3
  s += __builtin_amdgcn_update_dpp(0, s, 0x142, 0xa, 0xf, true);  // row_bcast:15 into rows 1, 3
  if constexpr (L == 64) s += __builtin_amdgcn_update_dpp(0, s, 0x143, 0xc, 0xf, true);  // row_bcast:31 into rows 2, 3
  return s;
}

// ---- element conversion ---------------------------------------------------
// bf16 and fp16 are handled as raw 16-bit patterns; conversion to float is
// exact, conversion from float rounds to nearest even.
template <int DT> struct Elem;
template <> struct Elem<GR_DTYPE_F32> {
  using storage = float;
  __device__ static inline float to_float(float v) { return v; }
  __device__ static inline float from_float(float v) { return v; }
};
template <> struct Elem<GR_DTYPE_BF16> {
  using storage = uint16_t;
  __device__ static inline float to_float(uint16_t v) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(v) << 16);
  }
  __device__ static inline uint16_t from_float(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  }
};
template <> struct Elem<GR_DTYPE_F16> {
  using storage = uint16_t;
  __device__ static inline float to_float(uint16_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  }
  __device__ static inline uint16_t from_float(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  }
};

inline int dtype_size(int dtype) { return dtype == GR_DTYPE_F32 ? 4 : dtype == GR_DTYPE_FP8_E4M3 ? 1 : 2; }
inline bool dtype_valid(int dtype) {
  return dtype == GR_DTYPE_F32 || dtype == GR_DTYPE_F16 || dtype == GR_DTYPE_BF16;
}
// element types a KV cache may hold (the byte-moving kernels: fork, append)
inline bool cache_dtype_valid(int dtype) { return dtype_valid(dtype) || dtype == GR_DTYPE_FP8_E4M3; }

// ---- OCP fp8 e4m3 (float8_e4m3fn) -------------------------------------------
// Value of a byte: sign, 4 exponent bits e (bias 7), 3 mantissa bits m:
// 2^(e-7) (1 + m/8); e = 0: 2^-6 m/8; e = 15, m = 7: NaN (no infinities).
__device__ inline float fp8e4m3_to_float(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float v = e == 0 ? (float)m * 0x1p-9f : __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  v = (e == 15 && m == 7) ? __builtin_bit_cast(float, 0x7FC00000u) : v;  // quiet NaN
  return (b & 0x80u) ? -v : v;
}
// The e4m3 byte nearest to clamp(x, -448, 448), ties to even; NaN -> 0x7F.
// With e' = max(floor(log2 |x|), -6) the quantum is 2^(e' - 3), q = rint(|x| /
// quantum) (exact scaling) and the code is ((e' + 7) << 3) + q - 8: a q of 16
// carries into the next exponent, and e' = -6 covers the subnormals.
__device__ inline uint32_t float_to_fp8e4m3(float x) {
  if (x != x) return 0x7Fu;
  const uint32_t sign = (__builtin_bit_cast(uint32_t, x) >> 24) & 0x80u;
  const float a = fminf(fabsf(x), 448.0f);
  const int fe = (int)((__builtin_bit_cast(uint32_t, a) >> 23) & 0xFFu) - 127;
  const int e = fe < -6 ? -6 : fe;
  const int q = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(a, 3 - e));
  return a == 0.0f ? sign : sign | (uint32_t)(((e + 7) << 3) + q - 8);
}

// One 16-byte chunk per lane from global memory straight into LDS: lane i's
// chunk lands at lds + 16 i (lds wave-uniform).  The compiler does not see
// these writes: the code waits for them explicitly (vmcnt) before a barrier
// that precedes their readers, and M0 is restored after each instruction.
// On gfx9 an LDS load that reads M0 needs one wait state after the SALU
// write of M0: the s_nop.
__device__ inline void dma_s(uint32_t lds, const void* sbase, uint32_t voff) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  const uint64_t b = reinterpret_cast<uint64_t>(sbase);
  const uint64_t sb = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  uint32_t save;
  __asm__ volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
                   : "=&s"(save) : "s"(m), "v"(voff), "s"(sb) : "memory");
}
// Four dma_s loads in one statement: M0 saved and restored once.  Load i
// moves 64 x 16 bytes from sbase[i] + voff[i] to LDS byte address lds[i].
__device__ inline void dma_s4(const uint32_t (&lds)[4], const void* const (&sbase)[4], const uint32_t (&voff)[4]) {
  uint32_t m[4];
  uint64_t sb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = __builtin_amdgcn_readfirstlane(lds[i]);
    const uint64_t b = reinterpret_cast<uint64_t>(sbase[i]);
    sb[i] = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
            (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  }
  uint32_t save;
  __asm__ volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %5, %9\n\t"
      "s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %6, %10\n\t"
      "s_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %7, %11\n\t"
      "s_mov_b32 m0, %4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %8, %12\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "s"(m[0]), "s"(m[1]), "s"(m[2]), "s"(m[3]), "v"(voff[0]), "v"(voff[1]), "v"(voff[2]), "v"(voff[3]),
        "s"(sb[0]), "s"(sb[1]), "s"(sb[2]), "s"(sb[3])
      : "memory");
}
__device__ inline void dma_v(uint32_t lds, const void* addr) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
  uint32_t save;
  __asm__ volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                   : "=&s"(save) : "s"(m), "v"(addr) : "memory");
}
__device__ inline void flag_status(int32_t* dev_status, int bit) {
  if (dev_status) atomicOr(dev_status, bit);
}

inline gr_status_t launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? GR_OK : GR_ERR_LAUNCH;
}

}  // namespace gr
