// Shared device/host helpers for the gfx950 beam path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gr_beam.h"

#define GR_VERSION_CODE 100  // 0.1.0

namespace gr {

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

inline int dtype_size(int dtype) { return dtype == GR_DTYPE_F32 ? 4 : 2; }
inline bool dtype_valid(int dtype) {
  return dtype == GR_DTYPE_F32 || dtype == GR_DTYPE_F16 || dtype == GR_DTYPE_BF16;
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
