// Shared device helpers for the gfx950 kernels: element conversion with the
// round-to-nearest-even of c10::BFloat16, wave64 reductions, error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
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

// Dynamic LDS above 64 KiB needs the kernel's limit raised: raised once per
// kernel and device to all that the kernel's static LDS leaves of the CU's
// 160 KiB (a limit, not a reservation: each launch still takes only the
// LDS it asks for).  KERN is the kernel.
static constexpr size_t kLdsMax = 160 * 1024;
template <auto KERN>
inline int lds_limit(size_t lds, const char* who) {
  if (lds <= 64 * 1024) return CODA_OK;
  static std::atomic<uint64_t> done{0};
  static std::atomic<int64_t> room{-1};
  int64_t r = room.load(std::memory_order_acquire);
  if (r < 0) {
    hipFuncAttributes fa;
    const hipError_t e = hipFuncGetAttributes(&fa, (const void*)KERN);
    if (e != hipSuccess) return fail(CODA_EHIP, "%s: kernel attributes: %s", who, hipGetErrorString(e));
    r = (int64_t)kLdsMax - (int64_t)fa.sharedSizeBytes;
    room.store(r, std::memory_order_release);
  }
  if ((int64_t)lds > r)
    return fail(CODA_EUNSUP, "%s: %zu bytes of LDS needed (%lld available)", who, lds, (long long)r);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const uint64_t bit = dev < 64 ? (uint64_t(1) << dev) : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return CODA_OK;
  const hipError_t e = hipFuncSetAttribute((const void*)KERN, hipFuncAttributeMaxDynamicSharedMemorySize, (int)r);
  if (e != hipSuccess) return fail(CODA_EHIP, "%s: LDS attribute: %s", who, hipGetErrorString(e));
  done.fetch_or(bit, std::memory_order_acq_rel);
  return CODA_OK;
}

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

// RoPE of one pair with (c, s), one rounding to T per multiply and add, as
// the reference's element-wise torch ops (primitives.py:83-113):
//   interleaved (e, o) = (x[2i], x[2i+1]):      (e c - o s, e s + o c)
//   half-split  (e, o) = (x[i], x[i + Dh/2]):   (e c + (-o) s, o c + e s)
template <typename T>
__device__ __forceinline__ void rope_pair_t(float e, float o, float c, float s, bool inter, float& r0, float& r1) {
  using E = Elt<T>;
  if (inter) {
    r0 = E::rnd(E::rnd(e * c) - E::rnd(o * s));
    r1 = E::rnd(E::rnd(e * s) + E::rnd(o * c));
  } else {
    r0 = E::rnd(E::rnd(e * c) + E::rnd(-o * s));
    r1 = E::rnd(E::rnd(o * c) + E::rnd(e * s));
  }
}

// The new token's K handed to a decode-step kernel before RoPE: the kernel
// ropes it with the token's own tables (cs / sn: Dh/2 entries of the
// element type) as it writes and reads it.  mode 0: K already roped,
// 1: interleaved pairs, 2: half-split pairs.
struct RopeK {
  const void* cs;
  const void* sn;
  int mode;
};
// Element d of the roped row from the raw row: partner element and table
// entry, then the pair's formula (one value of the pair)
template <typename T>
__device__ __forceinline__ float rope_k_elem(float x, float partner, float c, float s, int d, int DH, int mode) {
  float r0, r1;
  if (mode == 1) {
    const bool ev = (d & 1) == 0;
    rope_pair_t<T>(ev ? x : partner, ev ? partner : x, c, s, true, r0, r1);
    return ev ? r0 : r1;
  }
  const bool lo = d < DH / 2;
  rope_pair_t<T>(lo ? x : partner, lo ? partner : x, c, s, false, r0, r1);
  return lo ? r0 : r1;
}
// (partner index, table index) of element d
__device__ __forceinline__ int rope_k_partner(int d, int DH, int mode) {
  return mode == 1 ? (d ^ 1) : (d < DH / 2 ? d + DH / 2 : d - DH / 2);
}
__device__ __forceinline__ int rope_k_table(int d, int DH, int mode) { return mode == 1 ? (d >> 1) : (d % (DH / 2)); }

// ----------------------------------------------------------------- wave64
// Cross-lane moves without LDS traffic: DPP within 16-lane rows, the gfx950
// permlane swaps across rows (each hands both lanes of a pair the same two
// values in the same order).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
struct Pair2 {
  int a, b;
};
__device__ __forceinline__ Pair2 swap16(int v) {
  const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  return Pair2{(int)r[0], (int)r[1]};
}
__device__ __forceinline__ Pair2 swap32(int v) {
  const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return Pair2{(int)r[0], (int)r[1]};
}

// Sum over the wave, the same value in every lane: pairs at distance 1 and
// 2 (quad permutes), then quad pairs (half-row mirror), 8-lane halves (row
// mirror), rows (swap16), half waves (swap32).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  Pair2 p = swap16(__builtin_bit_cast(int, v));
  v = __builtin_bit_cast(float, p.a) + __builtin_bit_cast(float, p.b);
  p = swap32(__builtin_bit_cast(int, v));
  return __builtin_bit_cast(float, p.a) + __builtin_bit_cast(float, p.b);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  Pair2 p = swap16(__builtin_bit_cast(int, v));
  v = fmaxf(__builtin_bit_cast(float, p.a), __builtin_bit_cast(float, p.b));
  p = swap32(__builtin_bit_cast(int, v));
  return fmaxf(__builtin_bit_cast(float, p.a), __builtin_bit_cast(float, p.b));
}

}  // namespace coda
