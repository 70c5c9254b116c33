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

// bf16 rows whose bases are 16-byte aligned (Dh a multiple of 16): one
// thread per 16-byte piece of pairs, every load and store 16 (interleaved:
// x, out) or 8 bytes wide.  Interleaved: piece c holds pairs 4c .. 4c + 3
// (elements 8c .. 8c + 7); half-split: pairs 8c .. 8c + 7, elements
// 8c .. and 8c + Dh/2 .. .  Same rounding as rope_kernel.
__global__ __launch_bounds__(256) void rope_bf16_vec(bf16_t* __restrict__ out, int64_t o_sb, int64_t o_sh,
                                                     int64_t o_sl, const bf16_t* __restrict__ x, int64_t x_sb,
                                                     int64_t x_sh, int64_t x_sl, const bf16_t* __restrict__ cs,
                                                     const bf16_t* __restrict__ sn, int Hx, int L, int Dh,
                                                     int interleaved, int rows) {
  using E = Elt<bf16_t>;
  const int half = Dh >> 1;
  const int cpr = interleaved ? Dh / 8 : Dh / 16;  // pieces per row
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= rows * cpr) return;
  const int c = i % cpr, r = i / cpr;
  const int l = r % L, bh = r / L;
  const int h = bh % Hx, b = bh / Hx;
  const bf16_t* xr = x + b * x_sb + h * x_sh + (int64_t)l * x_sl;
  bf16_t* orow = out + b * o_sb + h * o_sh + (int64_t)l * o_sl;
  auto f = [](uint32_t w, int hi) { return bf2f((bf16_t)(hi ? w >> 16 : w & 0xffffu)); };
  auto pk = [](float a, float bb) { return (uint32_t)E::st(a) | ((uint32_t)E::st(bb) << 16); };
  if (interleaved) {
    const uint4 xv = *reinterpret_cast<const uint4*>(xr + 8 * c);
    const uint2 cv = *reinterpret_cast<const uint2*>(cs + (int64_t)l * half + 4 * c);
    const uint2 sv = *reinterpret_cast<const uint2*>(sn + (int64_t)l * half + 4 * c);
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, cw[2] = {cv.x, cv.y}, sw[2] = {sv.x, sv.y};
    uint32_t ow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e = f(xw[j], 0), o = f(xw[j], 1), cc = f(cw[j >> 1], j & 1), ss = f(sw[j >> 1], j & 1);
      ow[j] = pk(E::rnd(e * cc) - E::rnd(o * ss), E::rnd(e * ss) + E::rnd(o * cc));
    }
    *reinterpret_cast<uint4*>(orow + 8 * c) = uint4{ow[0], ow[1], ow[2], ow[3]};
  } else {
    const uint4 av = *reinterpret_cast<const uint4*>(xr + 8 * c);
    const uint4 bv = *reinterpret_cast<const uint4*>(xr + half + 8 * c);
    const uint4 cv = *reinterpret_cast<const uint4*>(cs + (int64_t)l * half + 8 * c);
    const uint4 sv = *reinterpret_cast<const uint4*>(sn + (int64_t)l * half + 8 * c);
    const uint32_t aw[4] = {av.x, av.y, av.z, av.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
    const uint32_t cw[4] = {cv.x, cv.y, cv.z, cv.w}, sw[4] = {sv.x, sv.y, sv.z, sv.w};
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float r0[2], r1[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float a = f(aw[j], u), bb = f(bw[j], u), cc = f(cw[j], u), ss = f(sw[j], u);
        r0[u] = E::rnd(a * cc) + E::rnd(-bb * ss);
        r1[u] = E::rnd(bb * cc) + E::rnd(a * ss);
      }
      lo[j] = pk(r0[0], r0[1]);
      hi[j] = pk(r1[0], r1[1]);
    }
    *reinterpret_cast<uint4*>(orow + 8 * c) = uint4{lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<uint4*>(orow + half + 8 * c) = uint4{hi[0], hi[1], hi[2], hi[3]};
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
  else if (Dh % 16 == 0 && (int64_t)B * Hx * L * (Dh / 8) < ((int64_t)1 << 31) &&
           ((uintptr_t)out % 16) == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)cos_t % 16) == 0 &&
           ((uintptr_t)sin_t % 16) == 0 && o_sb % 8 == 0 && o_sh % 8 == 0 && o_sl % 8 == 0 && x_sb % 8 == 0 &&
           x_sh % 8 == 0 && x_sl % 8 == 0) {
    const int rows = B * Hx * L, cpr = interleaved ? Dh / 8 : Dh / 16;
    const int64_t n = (int64_t)rows * cpr;
    hipLaunchKernelGGL(rope_bf16_vec, dim3((unsigned)((n + 255) / 256)), block, 0, st, (bf16_t*)out, o_sb, o_sh,
                       o_sl, (const bf16_t*)x, x_sb, x_sh, x_sl, (const bf16_t*)cos_t, (const bf16_t*)sin_t, Hx, L,
                       Dh, interleaved, rows);
  } else
    hipLaunchKernelGGL(rope_kernel<bf16_t>, grid, block, 0, st, (bf16_t*)out, o_sb, o_sh, o_sl,
                       (const bf16_t*)x, x_sb, x_sh, x_sl, (const bf16_t*)cos_t, (const bf16_t*)sin_t, Hx, L,
                       Dh, interleaved, total);
  return check_launch("rope");
}
