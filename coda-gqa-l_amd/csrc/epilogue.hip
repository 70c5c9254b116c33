// Standalone differential epilogue: rows of Dh, one wave per row.
//   full : out = RMSNorm(sig - lam * noise) * w
//   sub  : out = sig - lam * noise
// Rounding follows the reference's eager fallback op by op
// (kernels/coda_diff_epilogue/torch-ext/coda_kernels/__init__.py:62-65,
// :95-96): one rounding to the element type after every torch op.
#include "common.h"

#include <hip/hip_fp16.h>

namespace coda {

// half storage: a distinct type so the traits do not collide with bf16_t
struct f16_t {
  uint16_t v;
};

template <typename T> struct EpiElt;
template <> struct EpiElt<float> : Elt<float> {};
template <> struct EpiElt<bf16_t> : Elt<bf16_t> {};
template <> struct EpiElt<f16_t> {
  static __device__ __forceinline__ float ld(f16_t x) { return __half2float(__ushort_as_half(x.v)); }
  static __device__ __forceinline__ f16_t st(float x) { return f16_t{__half_as_ushort(__float2half_rn(x))}; }
  static __device__ __forceinline__ float rnd(float x) { return ld(st(x)); }
};

template <typename T, bool NORM>
__global__ __launch_bounds__(256) void diff_epilogue_kernel(T* __restrict__ out, const T* __restrict__ sig,
                                                            const T* __restrict__ noise,
                                                            const T* __restrict__ lam,
                                                            const T* __restrict__ w, int rows, int dh,
                                                            float eps) {
  using E = EpiElt<T>;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = (int64_t)row * dh;
  const float lv = E::ld(lam[row]);
  float sq = 0.f;
  for (int d = lane; d < dh; d += 64) {
    const float y = E::rnd(E::ld(sig[base + d]) - E::rnd(lv * E::ld(noise[base + d])));
    if (NORM) sq += E::rnd(y * y);
    else out[base + d] = E::st(y);
  }
  if (!NORM) return;
  sq = wave_sum(sq);
  const float ms = E::rnd(sq / (float)dh);
  const float r = E::rnd(1.0f / sqrtf(E::rnd(ms + E::rnd(eps))));
  for (int d = lane; d < dh; d += 64) {
    const float y = E::rnd(E::ld(sig[base + d]) - E::rnd(lv * E::ld(noise[base + d])));
    out[base + d] = E::st(E::rnd(E::rnd(y * r) * E::ld(w[d])));
  }
}

template <bool NORM>
static int launch(int dtype, void* out, const void* sig, const void* noise, const void* lam,
                  const void* w, int rows, int dh, float eps, hipStream_t st) {
  const dim3 grid((rows + 3) / 4), block(256);
  switch (dtype) {
    case CODA_F32:
      hipLaunchKernelGGL((diff_epilogue_kernel<float, NORM>), grid, block, 0, st, (float*)out,
                         (const float*)sig, (const float*)noise, (const float*)lam, (const float*)w, rows,
                         dh, eps);
      break;
    case CODA_BF16:
      hipLaunchKernelGGL((diff_epilogue_kernel<bf16_t, NORM>), grid, block, 0, st, (bf16_t*)out,
                         (const bf16_t*)sig, (const bf16_t*)noise, (const bf16_t*)lam, (const bf16_t*)w,
                         rows, dh, eps);
      break;
    default:
      hipLaunchKernelGGL((diff_epilogue_kernel<f16_t, NORM>), grid, block, 0, st, (f16_t*)out,
                         (const f16_t*)sig, (const f16_t*)noise, (const f16_t*)lam, (const f16_t*)w, rows,
                         dh, eps);
  }
  return check_launch(NORM ? "diff_epilogue" : "diff_sub_only");
}

}  // namespace coda

using namespace coda;

extern "C" int coda_diff_epilogue_fwd(int dtype, void* out, const void* sig, const void* noise,
                                      const void* lam, const void* w, int num_rows, int head_dim,
                                      float eps, void* stream) {
  CODA_REQUIRE(dtype == CODA_F32 || dtype == CODA_BF16 || dtype == CODA_F16,
               "coda_diff_epilogue_fwd: unsupported dtype %d", dtype);
  CODA_REQUIRE(num_rows >= 0 && head_dim > 0, "coda_diff_epilogue_fwd: bad sizes rows=%d head_dim=%d",
               num_rows, head_dim);
  CODA_REQUIRE(out && sig && noise && lam && w, "coda_diff_epilogue_fwd: null pointer");
  if (num_rows == 0) return CODA_OK;
  return launch<true>(dtype, out, sig, noise, lam, w, num_rows, head_dim, eps, (hipStream_t)stream);
}

extern "C" int coda_diff_sub_only_fwd(int dtype, void* out, const void* sig, const void* noise,
                                      const void* lam, int num_rows, int head_dim, void* stream) {
  CODA_REQUIRE(dtype == CODA_F32 || dtype == CODA_BF16 || dtype == CODA_F16,
               "coda_diff_sub_only_fwd: unsupported dtype %d", dtype);
  CODA_REQUIRE(num_rows >= 0 && head_dim > 0, "coda_diff_sub_only_fwd: bad sizes rows=%d head_dim=%d",
               num_rows, head_dim);
  CODA_REQUIRE(out && sig && noise && lam, "coda_diff_sub_only_fwd: null pointer");
  if (num_rows == 0) return CODA_OK;
  return launch<false>(dtype, out, sig, noise, lam, nullptr, num_rows, head_dim, 0.f, (hipStream_t)stream);
}

// Typed entry points with the argument lists of the reference's extern "C"
// functions (kernels/coda_diff_epilogue/kernel_src/diff_epilogue.cu:465-568),
// so its torch binding (torch-ext/torch_binding.cpp:203-213) links against
// this library unchanged.  They return void like the reference's; an
// argument error or a failed launch leaves its message in coda_last_error().
#define CODA_TYPED_EPILOGUE(SUFFIX, CODE, TYPE)                                                                \
  extern "C" void diff_epilogue_forward_##SUFFIX(TYPE* output, const TYPE* out_sig, const TYPE* out_noise,     \
                                                 const TYPE* lam, const TYPE* weight, int num_rows,            \
                                                 int head_dim, float eps, void* stream) {                      \
    (void)coda_diff_epilogue_fwd(CODE, output, out_sig, out_noise, lam, weight, num_rows, head_dim, eps,       \
                                 stream);                                                               \
  }                                                                                                            \
  extern "C" void diff_sub_only_forward_##SUFFIX(TYPE* output, const TYPE* out_sig, const TYPE* out_noise,     \
                                                 const TYPE* lam, int num_rows, int head_dim,                  \
                                                 void* stream) {                                               \
    (void)coda_diff_sub_only_fwd(CODE, output, out_sig, out_noise, lam, num_rows, head_dim, stream);            \
  }

CODA_TYPED_EPILOGUE(bf16, CODA_BF16, uint16_t)
CODA_TYPED_EPILOGUE(fp16, CODA_F16, uint16_t)
CODA_TYPED_EPILOGUE(fp32, CODA_F32, float)
#undef CODA_TYPED_EPILOGUE
