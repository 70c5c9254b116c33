// RoPE of a (B, Hx, L, Dh) tensor with (L, Dh/2) tables, rounding after
// every multiply / add in the element type (primitives.py:83-113):
//   interleaved pairs (2i, 2i+1): (e c - o s, e s + o c)
//   half-split  (i, i + Dh/2)   : x * cos_full + rotate_half(x) * sin_full
// One thread per output pair; the (b, h, l) row index runs over the grid.
#include "common.h"

namespace coda {

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(T* __restrict__ out, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                                                   const T* __restrict__ x, int64_t x_sb, int64_t x_sh,
                                                   int64_t x_sl, const T* __restrict__ cs,
                                                   const T* __restrict__ sn, int Hx, int L, int Dh,
                                                   int interleaved, int64_t total_pairs) {
  using E = Elt<T>;
  const int half = Dh >> 1;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total_pairs) return;
  const int p = (int)(i % half);
  int64_t r = i / half;
  const int l = (int)(r % L);
  r /= L;
  const int h = (int)(r % Hx);
  const int b = (int)(r / Hx);
  const T* xr = x + b * x_sb + h * x_sh + (int64_t)l * x_sl;
  T* orow = out + b * o_sb + h * o_sh + (int64_t)l * o_sl;
  const float c = E::ld(cs[(int64_t)l * half + p]), s = E::ld(sn[(int64_t)l * half + p]);
  if (interleaved) {
    const float e = E::ld(xr[2 * p]), o = E::ld(xr[2 * p + 1]);
    orow[2 * p] = E::st(E::rnd(e * c) - E::rnd(o * s));
    orow[2 * p + 1] = E::st(E::rnd(e * s) + E::rnd(o * c));
  } else {
    const float a = E::ld(xr[p]), bb = E::ld(xr[p + half]);
    orow[p] = E::st(E::rnd(a * c) + E::rnd(-bb * s));
    orow[p + half] = E::st(E::rnd(bb * c) + E::rnd(a * s));
  }
}

}  // namespace coda

using namespace coda;

extern "C" int coda_rope_fwd(int dtype, void* out, int64_t o_sb, int64_t o_sh, int64_t o_sl, const void* x,
                             int64_t x_sb, int64_t x_sh, int64_t x_sl, const void* cos_t, const void* sin_t,
                             int B, int Hx, int L, int Dh, int interleaved, void* stream) {
  CODA_REQUIRE(dtype == CODA_F32 || dtype == CODA_BF16, "coda_rope_fwd: unsupported dtype %d", dtype);
  CODA_REQUIRE(B >= 0 && Hx >= 0 && L >= 0 && Dh > 0 && Dh % 2 == 0,
               "coda_rope_fwd: bad sizes B=%d Hx=%d L=%d Dh=%d", B, Hx, L, Dh);
  CODA_REQUIRE(out && x && cos_t && sin_t, "coda_rope_fwd: null pointer");
  const int64_t total = (int64_t)B * Hx * L * (Dh / 2);
  if (total == 0) return CODA_OK;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == CODA_F32)
    hipLaunchKernelGGL(rope_kernel<float>, grid, block, 0, st, (float*)out, o_sb, o_sh, o_sl, (const float*)x,
                       x_sb, x_sh, x_sl, (const float*)cos_t, (const float*)sin_t, Hx, L, Dh, interleaved, total);
  else
    hipLaunchKernelGGL(rope_kernel<bf16_t>, grid, block, 0, st, (bf16_t*)out, o_sb, o_sh, o_sl,
                       (const bf16_t*)x, x_sb, x_sh, x_sl, (const bf16_t*)cos_t, (const bf16_t*)sin_t, Hx, L,
                       Dh, interleaved, total);
  return check_launch("rope");
}
