// Shared device helpers for the gfx950 kernels: element conversion with the
// round-to-nearest-even of c10::BFloat16, wave64 reductions, error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/coda_mi355x.h"

namespace coda {

// ----------------------------------------------------------------- errors
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

#define CODA_REQUIRE(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::coda::fail(CODA_EINVAL, __VA_ARGS__);   \
  } while (0)

// ----------------------------------------------------------------- types
typedef uint16_t bf16_t;  // raw bfloat16 bits

__host__ __device__ __forceinline__ float bf2f(bf16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}

// float -> bfloat16 bits, round to nearest even, NaN -> 0x7FC0 (c10 rule).
// On the GPU this is the hardware conversion (v_cvt_pk_bf16_f32, round to
// nearest even; a NaN keeps its sign and the top of its payload, quietened).
__host__ __device__ __forceinline__ bf16_t f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(bf16_t, (__bf16)f);
#else
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)0x7FC0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
#endif
}

// Element type traits.  `rnd` rounds an fp32 value to the precision of the
// element type: this is where the reference's eager ops materialise a
// tensor (one rounding per torch op in bf16; nothing in fp32).
template <typename T> struct Elt;
template <> struct Elt<float> {
  static __host__ __device__ __forceinline__ float ld(float x) { return x; }
  static __host__ __device__ __forceinline__ float st(float x) { return x; }
  static __host__ __device__ __forceinline__ float rnd(float x) { return x; }
};
template <> struct Elt<bf16_t> {
  static __host__ __device__ __forceinline__ float ld(bf16_t x) { return bf2f(x); }
  static __host__ __device__ __forceinline__ bf16_t st(float x) { return f2bf(x); }
  static __host__ __device__ __forceinline__ float rnd(float x) { return bf2f(f2bf(x)); }
};

// ----------------------------------------------------------------- wave64
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace coda
