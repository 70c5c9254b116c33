// Fused two-stream differential attention for gfx950.
//
//   out = Norm( softmax(q K^T) V  -  lam * softmax(q_noise K^T) V )
//
// One launch covers the whole seam of the reference: RoPE of q, the
// per-head pairwise rotation that makes q_noise, GQA sharing of K/V (every
// K/V byte is read once for the G query heads of its KV head and for both
// streams), the prefix mask of the bounded cache (ring | exact | summary
// slots gated by `allowed`), the lower-right causal block, the lambda
// difference and HeadwiseRMSNorm.  Reference seam:
// src/coda_gqa_l/attention.py:416-465 (+ mask policy :635-693, :476-514).
//
// Kernels
//   attn_rows_bf16   decode shape (2*G*Lq <= 16 query rows per KV head):
//                    all rows of a KV head packed in one 16-row MFMA tile,
//                    the 4 waves of a workgroup split the keys; optional
//                    split over workgroups with a merge kernel.  HBM-bound:
//                    K/V stream straight from HBM into MFMA fragments (K)
//                    and a per-wave LDS transpose (V).
//   attn_tile_bf16   prefill / unbounded shape: a workgroup owns one KV
//                    head and 16*NQ queries of its G heads; each wave owns
//                    a (head, 16 queries) pair as two 16-row tiles (signal,
//                    noise) sharing every K/V fragment; K/V tiles of 64
//                    keys are staged through LDS once per workgroup.
//                    MFMA-bound.
//   attn_generic     fp32 (VALU): config-C1-sized problems and tests.
//
// MFMA fragment layouts (wave64, l = lane, n = l % 16, g4 = l / 16):
//   v_mfma_f32_16x16x32_bf16 A[m=n][k=8*g4+j], B[k=8*g4+j][col=n], j<8
//   v_mfma_f32_16x16x16_bf16 A[m=n][k=4*g4+j], B[k=4*g4+j][col=n], j<4
//   both:                    D[m=4*g4+j][col=n], j<4
// S^T = K Q^T puts keys on m and query rows on n, so the D fragment of S^T
// is directly the B fragment (P^T, keys on k) of O^T = V^T P^T.

#include "bank_ops.h"
#include "common.h"

#include <atomic>
#include <cstring>

#include <math.h>
#include <type_traits>
#include <utility>
#include <stdlib.h>

namespace coda {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
// dword 3 of a raw buffer resource on gfx9 (32-bit data format, no swizzle)
static constexpr int kBufWord3 = 0x00020000;
typedef float f32x4 __attribute__((ext_vector_type(4)));

static constexpr float kLog2e = 1.4426950408889634f;
static constexpr int kMaxRowsPrefix = 2048;  // prefix slots whose `allowed` bytes fit the LDS copy

// ------------------------------------------------------------ query prep
// Eight consecutive channels [d0, d0+8) of the (roped) signal query or of
// the noise query of (b, h, qi), with the rounding of the reference's eager
// ops (primitives.py:58-80 rotation, :83-113 RoPE: one rounding per op).
template <typename T>
__device__ __forceinline__ void load8(const T* p, float x[8]) {
  if constexpr (sizeof(T) == 2) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf2f((bf16_t)(w[i] & 0xffffu));
      x[2 * i + 1] = bf2f((bf16_t)(w[i] >> 16));
    }
  } else {
    float4 a = *reinterpret_cast<const float4*>(p);
    float4 b = *reinterpret_cast<const float4*>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
}

template <typename T>
__device__ __forceinline__ void rotate_pairs8(float x[8], const T* c, const T* s) {
  using E = Elt<T>;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float cc = E::ld(c[p]), ss = E::ld(s[p]);
    const float e = x[2 * p], o = x[2 * p + 1];
    x[2 * p] = E::rnd(E::rnd(e * cc) - E::rnd(o * ss));
    x[2 * p + 1] = E::rnd(E::rnd(e * ss) + E::rnd(o * cc));
  }
}

template <typename T>
__device__ __forceinline__ void prep_q8(const coda_attn_desc& a, int b, int h, int qi, int d0,
                                        int stream, float x[8]) {
  using E = Elt<T>;
  const int half = a.Dh >> 1;
  if (stream == 1 && a.q_noise) {
    load8<T>((const T*)a.q_noise + b * a.qn_sb + h * a.qn_sh + qi * a.qn_sl + d0, x);
    return;
  }
  const T* qrow = (const T*)a.q + b * a.q_sb + h * a.q_sh + qi * a.q_sl;
  load8<T>(qrow + d0, x);
  if (a.rope_cos) {
    const T* c = (const T*)a.rope_cos + (int64_t)qi * half;
    const T* s = (const T*)a.rope_sin + (int64_t)qi * half;
    if (a.rope_interleaved) {
      rotate_pairs8<T>(x, c + (d0 >> 1), s + (d0 >> 1));
    } else {
      float y[8];
      const bool lo = d0 < half;
      load8<T>(qrow + (lo ? d0 + half : d0 - half), y);
      const int f0 = lo ? d0 : d0 - half;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float rot = lo ? -y[j] : y[j];
        const float cc = E::ld(c[f0 + j]), ss = E::ld(s[f0 + j]);
        x[j] = E::rnd(E::rnd(x[j] * cc) + E::rnd(rot * ss));
      }
    }
  }
  if (stream == 1) {
    rotate_pairs8<T>(x, (const T*)a.theta_cos + (int64_t)h * half + (d0 >> 1),
                     (const T*)a.theta_sin + (int64_t)h * half + (d0 >> 1));
  }
}

// Cooperative query staging into LDS (bf16 rows of Dh): row r of the
// workgroup maps to (stream s, head h, query qi) through `map(r, s, h, qi)`.
// One thread prepares 4 channels {2i, 2i+1, half+2i, half+2i+1}, which
// closes both pairings (interleaved RoPE / noise rotation pairs and
// half-split RoPE pairs) inside one thread; all of its loads are issued
// before any arithmetic.  Rounding as prep_q8.
template <typename MapF>
__device__ __forceinline__ void stage_queries(const coda_attn_desc& a, int b, int rows, bf16_t* qs, int qs_stride,
                                              MapF map) {
  using E = Elt<bf16_t>;
  const int Dh = a.Dh, half = Dh >> 1, quarter = Dh >> 2;
  for (int it = threadIdx.x; it < rows * quarter; it += blockDim.x) {
    const int r = it / quarter, i = it % quarter;
    int st, h, qi;
    const bool live = map(r, st, h, qi);
    const int d0 = 2 * i, d1 = 2 * i + 1, d2 = half + 2 * i, d3 = half + 2 * i + 1;
    float x[4] = {0.f, 0.f, 0.f, 0.f};
    if (live) {
      const bool given_noise = st == 1 && a.q_noise;
      const bf16_t* src = given_noise ? (const bf16_t*)a.q_noise + b * a.qn_sb + h * a.qn_sh + qi * a.qn_sl
                                      : (const bf16_t*)a.q + b * a.q_sb + h * a.q_sh + qi * a.q_sl;
      const uint32_t w01 = *reinterpret_cast<const uint32_t*>(src + d0);
      const uint32_t w23 = *reinterpret_cast<const uint32_t*>(src + d2);
      x[0] = bf2f((bf16_t)(w01 & 0xffffu)); x[1] = bf2f((bf16_t)(w01 >> 16));
      x[2] = bf2f((bf16_t)(w23 & 0xffffu)); x[3] = bf2f((bf16_t)(w23 >> 16));
      if (!given_noise) {
        if (a.rope_cos) {
          const bf16_t* c = (const bf16_t*)a.rope_cos + (int64_t)qi * half;
          const bf16_t* sn = (const bf16_t*)a.rope_sin + (int64_t)qi * half;
          if (a.rope_interleaved) {
            // pairs (d0, d1) with angle i, (d2, d3) with angle quarter + i
            const float c0 = E::ld(c[i]), s0 = E::ld(sn[i]), c1 = E::ld(c[quarter + i]), s1 = E::ld(sn[quarter + i]);
            const float e0 = x[0], o0 = x[1], e1 = x[2], o1 = x[3];
            x[0] = E::rnd(E::rnd(e0 * c0) - E::rnd(o0 * s0));
            x[1] = E::rnd(E::rnd(e0 * s0) + E::rnd(o0 * c0));
            x[2] = E::rnd(E::rnd(e1 * c1) - E::rnd(o1 * s1));
            x[3] = E::rnd(E::rnd(e1 * s1) + E::rnd(o1 * c1));
          } else {
            // half-split pairs (d0, d2) and (d1, d3) with angles 2i, 2i+1
            const float c0 = E::ld(c[d0]), s0 = E::ld(sn[d0]), c1 = E::ld(c[d1]), s1 = E::ld(sn[d1]);
            const float lo0 = x[0], lo1 = x[1], hi0 = x[2], hi1 = x[3];
            x[0] = E::rnd(E::rnd(lo0 * c0) + E::rnd(-hi0 * s0));
            x[1] = E::rnd(E::rnd(lo1 * c1) + E::rnd(-hi1 * s1));
            x[2] = E::rnd(E::rnd(hi0 * c0) + E::rnd(lo0 * s0));
            x[3] = E::rnd(E::rnd(hi1 * c1) + E::rnd(lo1 * s1));
          }
        }
        if (st == 1) {
          const bf16_t* tc = (const bf16_t*)a.theta_cos + (int64_t)h * half;
          const bf16_t* ts = (const bf16_t*)a.theta_sin + (int64_t)h * half;
          const float c0 = E::ld(tc[i]), s0 = E::ld(ts[i]), c1 = E::ld(tc[quarter + i]), s1 = E::ld(ts[quarter + i]);
          const float e0 = x[0], o0 = x[1], e1 = x[2], o1 = x[3];
          x[0] = E::rnd(E::rnd(e0 * c0) - E::rnd(o0 * s0));
          x[1] = E::rnd(E::rnd(e0 * s0) + E::rnd(o0 * c0));
          x[2] = E::rnd(E::rnd(e1 * c1) - E::rnd(o1 * s1));
          x[3] = E::rnd(E::rnd(e1 * s1) + E::rnd(o1 * c1));
        }
      }
    }
    bf16_t* dst = qs + r * qs_stride;
    *reinterpret_cast<uint32_t*>(dst + d0) = (uint32_t)f2bf(x[0]) | ((uint32_t)f2bf(x[1]) << 16);
    *reinterpret_cast<uint32_t*>(dst + d2) = (uint32_t)f2bf(x[2]) | ((uint32_t)f2bf(x[3]) << 16);
  }
}

// Key visibility for query qi at key index kidx in [0, Lp + Lb).
__device__ __forceinline__ bool key_visible(const coda_attn_desc& a, int b, int qi, int kidx) {
  if (kidx < a.Lp) return a.allowed ? (a.allowed[(int64_t)b * a.al_sb + kidx] != 0) : true;
  const int j = kidx - a.Lp;
  if (j >= a.Lb) return false;
  return !a.causal || j <= qi + (a.causal == 2 ? 0 : a.Lb - a.Lq);
}

template <typename T>
__device__ __forceinline__ const T* key_ptr(const coda_attn_desc& a, int b, int hk, int kidx,
                                            bool value) {
  if (kidx < a.Lp)
    return (const T*)(value ? a.vp : a.kp) + b * a.p_sb + hk * a.p_sh + (int64_t)kidx * a.p_sl;
  return (const T*)(value ? a.vb : a.kb) + b * a.b_sb + hk * a.b_sh +
         (int64_t)(kidx - a.Lp) * a.b_sl;
}

// ------------------------------------------------------------ epilogue
// One output row (values os[], on[] of the two streams at this lane's
// channels) -> Norm(os - lam * on).  bf16 follows the eager op sequence of
// attention.py:463-464 + primitives.py:23-27 (round after every op; the eps
// add rounds eps to bf16 like torch's tensor+scalar add); fp32 is plain.
template <typename T, int NV>
__device__ __forceinline__ void diff_norm(float (&y)[NV], const float (&os)[NV],
                                          const float (&on)[NV], const bool (&act)[NV], float lam,
                                          const T* w, const int (&dd)[NV], float eps, int Dh,
                                          bool wave_reduce_all, int xor_lo, int xor_hi) {
  using E = Elt<T>;
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const float s = E::rnd(os[i]), n = E::rnd(on[i]);
    y[i] = E::rnd(s - E::rnd(lam * n));
    if (act[i]) sq += E::rnd(y[i] * y[i]);
  }
  if (!w) return;
  if (wave_reduce_all) {
    sq = wave_sum(sq);
  } else {
    for (int o = xor_lo; o <= xor_hi; o <<= 1) sq += __shfl_xor(sq, o, 64);
  }
  const float ms = E::rnd(sq / (float)Dh);
  const float r = E::rnd(1.0f / sqrtf(E::rnd(ms + E::rnd(eps))));
#pragma unroll
  for (int i = 0; i < NV; ++i) y[i] = act[i] ? E::rnd(E::rnd(y[i] * r) * E::ld(w[dd[i]])) : 0.f;
}

// diff_norm for bf16 with the weight values of this lane's channels
// already in registers (w[i] for channel lane + 64 i; null: identity norm).
template <int NV>
__device__ __forceinline__ void diff_norm_w(float (&y)[NV], const float (&os)[NV], const float (&on)[NV],
                                            const bool (&act)[NV], float lam, const float* w, float eps, int Dh) {
  using E = Elt<bf16_t>;
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const float s = E::rnd(os[i]), n = E::rnd(on[i]);
    y[i] = E::rnd(s - E::rnd(lam * n));
    if (act[i]) sq += E::rnd(y[i] * y[i]);
  }
  if (!w) return;
  sq = wave_sum(sq);
  const float ms = E::rnd(sq / (float)Dh);
  const float r = E::rnd(1.0f / sqrtf(E::rnd(ms + E::rnd(eps))));
#pragma unroll
  for (int i = 0; i < NV; ++i) y[i] = act[i] ? E::rnd(E::rnd(y[i] * r) * w[i]) : 0.f;
}

// ------------------------------------------------------------ fp32 / VALU
// Workgroup = (query qi, KV head, batch); rows = 2 streams x G heads.
template <typename T, int DH>
__global__ __launch_bounds__(256) void attn_generic(const coda_attn_desc a) {
  using E = Elt<T>;
  constexpr int KT = 256, RMAX = 16;
  __shared__ float qs[RMAX][DH];
  __shared__ float sc[RMAX][KT];
  __shared__ float red_alpha[RMAX];
  __shared__ float m_run[RMAX], l_run[RMAX];
  const int qi = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int G = a.H / a.Hkv, R = 2 * G;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float scale = (a.sm_scale > 0.f ? a.sm_scale : rsqrtf((float)DH));

  for (int i = t; i < R * (DH / 8); i += 256) {
    const int r = i / (DH / 8), c = i % (DH / 8);
    const int s = r / G, g = r % G;
    float x[8];
    prep_q8<T>(a, b, hk * G + g, qi, c * 8, s, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) qs[r][c * 8 + j] = x[j];
  }
  if (t < RMAX) { m_run[t] = -INFINITY; l_run[t] = 0.f; }
  constexpr int TPR = 256 / DH;                 // threads per row group
  constexpr int RPT = (RMAX + TPR - 1) / TPR;   // rows per thread
  const int dcol = t % DH, rg = t / DH;
  float o[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) o[i] = 0.f;
  __syncthreads();

  const int Lk = a.Lp + a.Lb;
  for (int k0 = 0; k0 < Lk; k0 += KT) {
    const int kidx = k0 + t;
    if (kidx < Lk) {
      const T* kr = key_ptr<T>(a, b, hk, kidx, false);
      float acc[RMAX];
#pragma unroll
      for (int r = 0; r < RMAX; ++r) acc[r] = 0.f;
      for (int d = 0; d < DH; d += 8) {
        float kx[8];
        load8<T>(kr + d, kx);
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
          if (r < R) {
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[r] = fmaf(qs[r][d + j], kx[j], acc[r]);
          }
        }
      }
      const bool vis = key_visible(a, b, qi, kidx);
      for (int r = 0; r < R; ++r) sc[r][t] = vis ? acc[r] * scale : -INFINITY;
    } else {
      for (int r = 0; r < R; ++r) sc[r][t] = -INFINITY;
    }
    __syncthreads();
    for (int r = wv; r < R; r += 4) {
      float mx = -INFINITY;
      for (int i = lane; i < KT; i += 64) mx = fmaxf(mx, sc[r][i]);
      mx = wave_max(mx);
      const float mold = m_run[r];
      const float mnew = fmaxf(mold, mx);
      const float muse = (mnew == -INFINITY) ? 0.f : mnew;
      float ps = 0.f;
      for (int i = lane; i < KT; i += 64) {
        const float p = expf(sc[r][i] - muse);
        sc[r][i] = p;
        ps += p;
      }
      ps = wave_sum(ps);
      if (lane == 0) {
        const float al = expf(mold - muse);
        red_alpha[r] = al;
        l_run[r] = l_run[r] * al + ps;
        m_run[r] = mnew;
      }
    }
    __syncthreads();
    const int kn = min(KT, Lk - k0);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = rg + i * TPR;
      if (r < R) o[i] *= red_alpha[r];
    }
    for (int kk = 0; kk < kn; ++kk) {
      const float v = E::ld(key_ptr<T>(a, b, hk, k0 + kk, true)[dcol]);
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int r = rg + i * TPR;
        if (r < R) o[i] = fmaf(sc[r][kk], v, o[i]);
      }
    }
    __syncthreads();
  }
  // normalise into qs (reused as the output staging buffer)
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = rg + i * TPR;
    if (r < R) qs[r][dcol] = l_run[r] > 0.f ? o[i] / l_run[r] : 0.f;
  }
  __syncthreads();
  // epilogue: wave per head of the group
  constexpr int NV = (DH + 63) / 64;
  for (int g = wv; g < G; g += 4) {
    const int h = hk * G + g;
    float os[NV], on[NV], y[NV];
    bool act[NV];
    int dd[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = d < DH;
      dd[i] = act[i] ? d : 0;
      os[i] = act[i] ? qs[g][dd[i]] : 0.f;
      on[i] = act[i] ? qs[G + g][dd[i]] : 0.f;
    }
    const float lam = E::ld(((const T*)a.lam)[b * a.lam_sb + h * a.lam_sh + qi * a.lam_sl]);
    diff_norm<T, NV>(y, os, on, act, lam, (const T*)a.rms_w, dd, a.eps, DH, true, 0, 0);
    T* orow = (T*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_sl;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) orow[dd[i]] = E::st(y[i]);
  }
}

// ------------------------------------------------------------ MFMA helpers
__device__ __forceinline__ f32x4 mfma_k32(const bf16x8_t& a, const bf16x8_t& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_k16(const short4_t& a, const short4_t& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8_t pack8(const float x[8]) {
  uint4 u;
  u.x = (uint32_t)f2bf(x[0]) | ((uint32_t)f2bf(x[1]) << 16);
  u.y = (uint32_t)f2bf(x[2]) | ((uint32_t)f2bf(x[3]) << 16);
  u.z = (uint32_t)f2bf(x[4]) | ((uint32_t)f2bf(x[5]) << 16);
  u.w = (uint32_t)f2bf(x[6]) | ((uint32_t)f2bf(x[7]) << 16);
  return __builtin_bit_cast(bf16x8_t, u);
}
__device__ __forceinline__ short4_t pack4(float a, float b, float c, float d) {
  uint2 u;
  u.x = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
  u.y = (uint32_t)f2bf(c) | ((uint32_t)f2bf(d) << 16);
  return __builtin_bit_cast(short4_t, u);
}

// V^T staging for one 16-key sub-tile: [key group kg (4 keys)][channel d]
// [4 keys] as 8-byte cells.  The row swizzle d ^ (((d >> 5) & 3) << 1) and
// the 128-byte pad per key group keep both the transposing writes (8 d of
// one lane) and the MFMA reads (16 consecutive d per lane group) at the
// minimum of two LDS cycles per wave instruction.
template <int DH>
struct VtLayout {
  static constexpr int kGroupBytes = DH * 8 + 128;
  static constexpr int kTileBytes = 4 * kGroupBytes;
  static __device__ __forceinline__ int off(int kg, int d) {
    return kg * kGroupBytes + ((d ^ (((d >> 5) & 3) << 1)) << 3);
  }
};

// Transpose 4 keys x 8 channels (four 16-byte rows) into 8 cells of
// 4 keys and store them.
template <int DH>
__device__ __forceinline__ void store_vt(char* base, int kg, int d0, const uint4 (&v)[4]) {
  const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&v[0]);
  const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&v[1]);
  const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&v[2]);
  const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&v[3]);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int sh = (e & 1) * 16;
    const int wi = e >> 1;
    uint2 cell;
    cell.x = ((w0[wi] >> sh) & 0xffffu) | (((w1[wi] >> sh) & 0xffffu) << 16);
    cell.y = ((w2[wi] >> sh) & 0xffffu) | (((w3[wi] >> sh) & 0xffffu) << 16);
    *reinterpret_cast<uint2*>(base + VtLayout<DH>::off(kg, d0 + e)) = cell;
  }
}

// ------------------------------------------------------------ decode rows
// Workgroup = (split, KV head, batch); 4 waves take 16-key tiles in turn.
// Partial (m, l, O) of the 4 waves merge in LDS; with nsplit > 1 each
// workgroup leaves its merged partial in `ws` for attn_rows_merge.
// Workgroup = (split, KV head, batch); 4 attention waves take 16-key tiles
// in turn and merge their partial (m, l, O) in LDS; with nsplit > 1 each
// workgroup leaves its merged partial in `ws` for attn_rows_merge.
template <int DH>
__global__ __launch_bounds__(256) void attn_rows_bf16(const coda_attn_desc a, int keys_per_split, float* ws) {
  constexpr int NC = DH / 32, NM = DH / 16, NW = 4;
  __shared__ __attribute__((aligned(16))) char vt_smem[NW][VtLayout<DH>::kTileBytes];
  __shared__ float red_m[NW][16], red_l[NW][16];
  __shared__ float red_o[NW][16][DH + 4];
  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int nsplit = gridDim.x;
  const int G = a.H / a.Hkv, GL = G * a.Lq, R = 2 * GL;
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g4 = lane >> 4;
  const float scale = (a.sm_scale > 0.f ? a.sm_scale : rsqrtf((float)DH)) * kLog2e;

  __shared__ __attribute__((aligned(16))) bf16_t q_lds[16][DH + 8];
  __shared__ uint8_t al_lds[kMaxRowsPrefix];
  constexpr int DCH = DH / 8;
  // V load roles: lane -> (key group kgl, 8-channel chunk dcl)
  const int kgl = lane / DCH, dcl = lane % DCH;
  const bool vload = kgl < 4;
  char* vt = vt_smem[wv];

  // Keys come from two sources, the prefix (state cache, visibility from
  // `allowed`) and the block (causal), each through a raw buffer resource of
  // its (sequence, KV head) plane: one 32-bit offset per load, rows past the
  // plane read as zero (hardware range check), so every load is
  // unconditional; keys outside a tile's range are removed by its mask.
  struct Src {
    const bf16_t* k;
    const bf16_t* v;
    int nbytes;      // bytes of the (sequence, KV head) plane
    int row0;        // global key index of the source's row 0
    int rb;          // row stride in bytes
  };
  auto make_src = [&](const void* kbase, const void* vbase, int64_t sb, int64_t sh, int64_t sl, int rows, int row0) {
    Src sr;
    const int64_t off = (int64_t)b * sb + (int64_t)hk * sh;
    sr.k = rows > 0 ? (const bf16_t*)kbase + off : (const bf16_t*)nullptr;
    sr.v = rows > 0 ? (const bf16_t*)vbase + off : (const bf16_t*)nullptr;
    sr.nbytes = rows > 0 ? (int)(((int64_t)(rows - 1) * sl + DH) * 2) : 0;
    sr.row0 = row0;
    sr.rb = (int)(sl * 2);
    return sr;
  };
  // buffer resources from wave-uniform values (readfirstlane makes the
  // uniformity explicit, so the resource stays in SGPRs and each load is a
  // single instruction)
  auto rsrc = [](const bf16_t* p, int nbytes) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0,
                                             __builtin_amdgcn_readfirstlane(nbytes), kBufWord3);
  };
  const int coff = a.causal == 2 ? 0 : a.Lb - a.Lq;
  // this split's keys [kbeg, kend): prefix tiles over [kbeg, pe), then
  // block tiles over [bs0, kend), 16 keys each
  const int kbeg = split * keys_per_split;
  const int kend = min(a.Lp + a.Lb, kbeg + keys_per_split);
  const int pe = min(kend, a.Lp);
  const int n1 = (a.Lp > 0 && kbeg < a.Lp) ? (pe - kbeg + 15) / 16 : 0;
  const int bs0 = max(kbeg, a.Lp);
  const int n2 = (a.Lb > 0 && kend > a.Lp) ? (kend - bs0 + 15) / 16 : 0;
  const int n_tiles = n1 + n2;
  const Src sp = make_src(a.kp, a.vp, a.p_sb, a.p_sh, a.p_sl, a.Lp, 0);
  const Src sb = make_src(a.kb, a.vb, a.b_sb, a.b_sh, a.b_sl, a.Lb, a.Lp);
  auto tile_kt = [&](int i) { return i < n1 ? kbeg + 16 * i : bs0 + 16 * (i - n1); };
  // K fragments straight from memory, V rows for the LDS transpose, of
  // this wave's i-th tile (tile wv + i * NW; past the end: the last tile
  // again, masked out by tile_mask)
  auto issue = [&](int i, bf16x8_t (&kf)[NC], uint4 (&vv)[4]) {
    int t = wv + i * NW;
    t = t < n_tiles ? t : n_tiles - 1;
    const bool pre = t < n1;
    const int kt = tile_kt(t);
    const __amdgpu_buffer_rsrc_t rk = rsrc(pre ? sp.k : sb.k, pre ? sp.nbytes : sb.nbytes);
    const __amdgpu_buffer_rsrc_t rv = rsrc(pre ? sp.v : sb.v, pre ? sp.nbytes : sb.nbytes);
    const int row0 = pre ? sp.row0 : sb.row0, rb = pre ? sp.rb : sb.rb;
    const int koff = (kt + n - row0) * rb + 16 * g4;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      kf[c] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + 64 * c, 0, 0));
    // every lane loads (lanes past the 4 key groups re-read group kgl & 3)
    // so the loads stay unconditional; only their LDS store is predicated
    const int voff = (kt + 4 * (kgl & 3) - row0) * rb + 16 * dcl;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      vv[jj] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff + jj * rb, 0, 0));
  };
  int row_qi = 0;
  // visibility of this lane's 4 keys (kt + 4 g4 + j) for query row n in
  // this wave's i-th tile; branch-free (a branch would make the compiler
  // wait for loads in flight)
  auto tile_mask = [&](int i) {
    const int t = wv + i * NW;
    const bool live = t < n_tiles;
    const bool pre = t < n1;
    const int kt = tile_kt(live ? t : 0);
    const int lo = live ? (pre ? kbeg : bs0) : 0, hi = live ? (pre ? pe : kend) : 0;
    const int pre_i = pre ? 1 : 0;
    int m4 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = kt + 4 * g4 + j;
      const int in = (kk >= lo) & (kk < hi);
      const int kc = in ? kk : lo;
      const int al_ok = al_lds[pre_i ? kc : 0] != 0;
      const int blk_ok = (a.causal == 0) | ((kc - a.Lp) <= row_qi + coff);
      m4 |= (in & (pre_i ? al_ok : blk_ok)) << j;
    }
    return m4;
  };
  const int nt_w = (n_tiles + NW - 1) / NW;
  bf16x8_t kf0[NC], kf1[NC];
  uint4 vv0[4], vv1[4];
  int vm0 = 0, vm1 = 0;
  // the first tile loads while the queries are staged
  if (n_tiles > 0) issue(0, kf0, vv0);
  // epilogue operands of this wave's output rows (single split), early
  constexpr int NV = (DH + 63) / 64;
  float lam_pf[2] = {0.f, 0.f}, w_pf[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) w_pf[i] = 1.f;
  if (nsplit == 1) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int orow = wv + r * NW;
      if (orow < GL) {
        const int g = orow / a.Lq, qi = orow % a.Lq, h = hk * G + g;
        lam_pf[r] = bf2f(((const bf16_t*)a.lam)[b * a.lam_sb + h * a.lam_sh + qi * a.lam_sl]);
      }
    }
    if (a.rms_w) {
#pragma unroll
      for (int i = 0; i < NV; ++i) w_pf[i] = bf2f(((const bf16_t*)a.rms_w)[min(lane + 64 * i, DH - 1)]);
    }
  }
  // queries (roped, rotated) and the visibility bytes of the prefix (1
  // where unmasked) go to LDS once; the host guarantees Lp <=
  // kMaxRowsPrefix, so the tile masks read them from LDS without a branch
  stage_queries(a, b, R, &q_lds[0][0], DH + 8, [&](int r, int& st, int& h, int& qi) {
    st = r / GL;
    const int rem = r % GL;
    h = hk * G + rem / a.Lq;
    qi = rem % a.Lq;
    return true;
  });
  for (int i = threadIdx.x; i < a.Lp; i += blockDim.x)
    al_lds[i] = a.allowed ? a.allowed[(int64_t)b * a.al_sb + i] : (uint8_t)1;
  __syncthreads();
  // query fragments (B operand of S^T): row n, channels 32c + 8 g4 + j
  bf16x8_t qf[NC];
  {
    const bool live = n < R;
    const int rem = live ? n % GL : 0;
    row_qi = rem % a.Lq;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint4 u = live ? *reinterpret_cast<const uint4*>(&q_lds[n][32 * c + 8 * g4]) : uint4{0, 0, 0, 0};
      qf[c] = __builtin_bit_cast(bf16x8_t, u);
    }
  }
  if (n_tiles > 0) vm0 = tile_mask(0);
  float m_i = -INFINITY, l_i = 0.f;
  f32x4 o[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One tile of MFMA + online-softmax work on already-loaded registers.
  auto consume = [&](const bf16x8_t (&kf)[NC], const uint4 (&vv)[4], int vmask) {
    f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) st = mfma_k32(kf[c], qf[c], st);
    // this lane: keys kt + 4 g4 + j, query row n
    float sv[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sv[j] = ((vmask >> j) & 1) ? st[j] * scale : -INFINITY;
      tmax = fmaxf(tmax, sv[j]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnew = fmaxf(m_i, tmax);
    const float muse = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = exp2f(m_i - muse);
    float p[4], ps = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[j] = bf2f(f2bf(exp2f(sv[j] - muse)));
      ps += p[j];
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l_i = l_i * alpha + ps;
    m_i = mnew;
    const short4_t pf = pack4(p[0], p[1], p[2], p[3]);
    if (vload) store_vt<DH>(vt, kgl, 8 * dcl, vv);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): LDS writes of this wave done
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) {
      const uint2 cell = *reinterpret_cast<const uint2*>(vt + VtLayout<DH>::off(g4, 16 * mt + n));
      o[mt] *= alpha;
      o[mt] = mfma_k16(__builtin_bit_cast(short4_t, cell), pf, o[mt]);
    }
    __builtin_amdgcn_wave_barrier();
  };
  // this wave's tiles i = 0 .. nt_w-1 (tile wv + i * NW) in ping-pong
  // register buffers: tile i+1 loads while tile i computes, with no
  // register copies between iterations (a copy would wait for the loads)
  for (int i = 0; i < nt_w; i += 2) {
    issue(i + 1, kf1, vv1);
    vm1 = tile_mask(i + 1);
    __builtin_amdgcn_sched_barrier(0);
    consume(kf0, vv0, vm0);
    if (i + 1 >= nt_w) break;
    issue(i + 2, kf0, vv0);
    vm0 = tile_mask(i + 2);
    __builtin_amdgcn_sched_barrier(0);
    consume(kf1, vv1, vm1);
  }
  // merge the 4 attention waves
  {
    if (g4 == 0) { red_m[wv][n] = m_i; red_l[wv][n] = l_i; }
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) red_o[wv][n][16 * mt + 4 * g4 + j] = o[mt][j];
  }
  __syncthreads();

  if (nsplit > 1) {
    // partial row r: [m, l, O(DH)] unnormalised w.r.t. the merged max
    float* base = ws + ((((int64_t)b * a.Hkv + hk) * nsplit + split) * 16) * (DH + 2);
    for (int i = threadIdx.x; i < R * (DH + 2); i += blockDim.x) {
      const int r = i / (DH + 2), c = i % (DH + 2);
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, red_m[w][r]);
      const float Mu = M == -INFINITY ? 0.f : M;
      float v = 0.f;
      if (c == 0) {
        v = M;
      } else if (c == 1) {
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red_l[w][r] * exp2f(red_m[w][r] - Mu);
      } else {
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red_o[w][r][c - 2] * exp2f(red_m[w][r] - Mu);
      }
      base[r * (DH + 2) + c] = v;
    }
    return;
  }
  // single split: merge + epilogue, one wave per (head, query) output row
  for (int orow = wv, r_pf = 0; orow < GL; orow += NW, ++r_pf) {
    const int g = orow / a.Lq, qi = orow % a.Lq, h = hk * G + g;
    float os[NV], on[NV], y[NV];
    bool act[NV];
    int dd[NV];
    float M[2] = {-INFINITY, -INFINITY}, L[2] = {0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int r = s * GL + orow;
#pragma unroll
      for (int w = 0; w < NW; ++w) M[s] = fmaxf(M[s], red_m[w][r]);
      const float Mu = M[s] == -INFINITY ? 0.f : M[s];
#pragma unroll
      for (int w = 0; w < NW; ++w) L[s] += red_l[w][r] * exp2f(red_m[w][r] - Mu);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = d < DH;
      dd[i] = act[i] ? d : 0;
      float acc[2] = {0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int r = s * GL + orow;
        const float Mu = M[s] == -INFINITY ? 0.f : M[s];
#pragma unroll
        for (int w = 0; w < NW; ++w) acc[s] += red_o[w][r][dd[i]] * exp2f(red_m[w][r] - Mu);
        acc[s] = L[s] > 0.f ? acc[s] / L[s] : 0.f;
      }
      os[i] = act[i] ? acc[0] : 0.f;
      on[i] = act[i] ? acc[1] : 0.f;
    }
    const float lam = r_pf == 0   ? lam_pf[0]
                      : r_pf == 1 ? lam_pf[1]
                                  : bf2f(((const bf16_t*)a.lam)[b * a.lam_sb + h * a.lam_sh + qi * a.lam_sl]);
    diff_norm_w<NV>(y, os, on, act, lam, a.rms_w ? w_pf : nullptr, a.eps, DH);
    bf16_t* orow_p = (bf16_t*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_sl;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) orow_p[dd[i]] = f2bf(y[i]);
  }
}

// Merge the per-split partials of attn_rows_bf16 and apply the epilogue.
template <int DH>
__global__ __launch_bounds__(256) void attn_rows_merge(const coda_attn_desc a, int nsplit,
                                                       const float* ws) {
  const int hk = blockIdx.x, b = blockIdx.y;
  const int G = a.H / a.Hkv, GL = G * a.Lq;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const float* base = ws + (((int64_t)b * a.Hkv + hk) * nsplit) * 16 * (DH + 2);
  constexpr int NV = (DH + 63) / 64;
  for (int orow = wv; orow < GL; orow += 4) {
    const int g = orow / a.Lq, qi = orow % a.Lq, h = hk * G + g;
    float os[NV], on[NV], y[NV];
    bool act[NV];
    int dd[NV];
    float M[2] = {-INFINITY, -INFINITY}, L[2] = {0.f, 0.f};
    for (int s = 0; s < 2; ++s) {
      const int r = s * GL + orow;
      for (int sp = 0; sp < nsplit; ++sp) M[s] = fmaxf(M[s], base[(sp * 16 + r) * (DH + 2)]);
      const float Mu = M[s] == -INFINITY ? 0.f : M[s];
      for (int sp = 0; sp < nsplit; ++sp) {
        const float* pr = base + (sp * 16 + r) * (DH + 2);
        L[s] += pr[1] * exp2f(pr[0] - Mu);
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = d < DH;
      dd[i] = act[i] ? d : 0;
      float acc[2] = {0.f, 0.f};
      for (int s = 0; s < 2; ++s) {
        const int r = s * GL + orow;
        const float Mu = M[s] == -INFINITY ? 0.f : M[s];
        for (int sp = 0; sp < nsplit; ++sp) {
          const float* pr = base + (sp * 16 + r) * (DH + 2);
          acc[s] += pr[2 + dd[i]] * exp2f(pr[0] - Mu);
        }
        acc[s] = L[s] > 0.f ? acc[s] / L[s] : 0.f;
      }
      os[i] = act[i] ? acc[0] : 0.f;
      on[i] = act[i] ? acc[1] : 0.f;
    }
    const float lam = bf2f(((const bf16_t*)a.lam)[b * a.lam_sb + h * a.lam_sh + qi * a.lam_sl]);
    diff_norm<bf16_t, NV>(y, os, on, act, lam, (const bf16_t*)a.rms_w, dd, a.eps, DH, true, 0, 0);
    bf16_t* orow_p = (bf16_t*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)qi * a.o_sl;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) orow_p[dd[i]] = f2bf(y[i]);
  }
}

// ------------------------------------------------------------ gfx950 helpers
// 16 bytes per lane global -> LDS (direct load): lane l's bytes land at
// lds + 16 l (lds wave-uniform); counted in vmcnt
__device__ __forceinline__ void lds_load16(const void* gsrc, void* lds) {
  __builtin_amdgcn_global_load_lds(gsrc, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element
// (j & 3) of the 8-byte segments addressed by lanes 4 y + (j & 15) / 4,
// y = 0..3 (a 4 x 16 -> 16 x 4 transpose of 16-bit elements)
typedef __bf16 bf16x4v_t __attribute__((ext_vector_type(4)));
// 32-bit LDS byte address of a pointer into LDS
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
// ds_read_b64_tr_b16 issued by hand, at an immediate byte offset.  The
// compiler treats the intrinsic as a read that may alias any direct
// global->LDS load in flight and waits for all of them first, which
// serialises the next tile's loads with this tile's PV product; here the
// caller orders the reads (barrier after the tile's loads landed) and waits
// for the results with lds_wait4_n.
template <int OFF>
__device__ __forceinline__ uint2 lds_read_tr16_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  uint2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// lgkmcnt(N) tied to four raw reads: they have landed once at most N LDS
// operations issued after them are still outstanding (LDS returns in order)
template <int N>
__device__ __forceinline__ void lds_wait4_n(uint2& a, uint2& b, uint2& c, uint2& d) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(N));
}
// f(std::integral_constant<int, 0>{}) .. f(..<N - 1>{}): loop indices that
// are constant expressions (immediate offsets, wait counts)
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
__device__ __forceinline__ uint2 lds_read_tr16(const void* lds) {
  const bf16x4v_t t =
      __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4v_t*)lds);
  return __builtin_bit_cast(uint2, t);
}

// max / sum of v over lanes l and l ^ 16 (or l ^ 32): the permlane swaps
// hand each lane the pair {v[l], v[l ^ d]} in the same order on both lanes
__device__ __forceinline__ float xmax16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float xmax32(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float xsum16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ float xsum32(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}


// chunk position of V row k is chunk ^ fa_vswz<DH>(k) (even, so the two
// chunks of a 32-byte channel group stay adjacent)
template <int DH>
__device__ __forceinline__ int fa_vswz(int k) {
  return DH == 128 ? 2 * (k & 7) : 2 * ((k >> 1) & 3);
}

// v_exp_f32 (2^x; -inf -> 0)
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// (e, o) -> (e c - o s, e s + o c) for a bf16 pair packed in one word, the
// angle's cos / sin taken from half `hf` of the words cw / sw: two bf16
// dot2 (exact products, fp32 sum) and one rounding of each output
__device__ __forceinline__ uint32_t rot_pair(uint32_t eo, uint32_t cw, uint32_t sw, int hf) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const uint32_t sel = hf ? 0x07060302u : 0x05040100u;
  const uint32_t cs = __builtin_amdgcn_perm(sw, cw, sel) ^ 0x80000000u;  // (c, -s)
  const uint32_t sc = __builtin_amdgcn_perm(cw, sw, sel);                // (s, c)
  const bf16x2_t x = __builtin_bit_cast(bf16x2_t, eo);
  const float r0 = __builtin_amdgcn_fdot2_f32_bf16(x, __builtin_bit_cast(bf16x2_t, cs), 0.f, false);
  const float r1 = __builtin_amdgcn_fdot2_f32_bf16(x, __builtin_bit_cast(bf16x2_t, sc), 0.f, false);
  return pk_bf16(r0, r1);
}

__device__ __forceinline__ void unpack8(const uint4& u, float x[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = bf2f((bf16_t)(w[j] & 0xffffu));
    x[2 * j + 1] = bf2f((bf16_t)(w[j] >> 16));
  }
}
__device__ __forceinline__ void unpack4(const uint2& u, float x[4]) {
  x[0] = bf2f((bf16_t)(u.x & 0xffffu));
  x[1] = bf2f((bf16_t)(u.x >> 16));
  x[2] = bf2f((bf16_t)(u.y & 0xffffu));
  x[3] = bf2f((bf16_t)(u.y >> 16));
}

// ------------------------------------------------------------ fused decode step
static constexpr int kFusedMaxBank = 256;  // exact + summary slots of the fused step
// decode_step_bf16: one workgroup per (KV head hk, sequence b) runs the
// whole decode step of that pair once the ring is full (the same work as
// decode_bank_kernel followed by attn_rows_bf16):
//   wave 3     the bank update of head hk for the token evicted from ring
//              slot j: decisions from the carried routing record, row
//              writes, metadata, the dots of the norm rows it rewrites;
//   waves 0-2  meanwhile attend to the ring slots other than j (the update
//              does not touch them) and to the new token (k_new, v_new: the
//              row the update writes into slot j), then take the next
//              step's routing record (dots of head hk's norm rows);
//   barrier    the decision and the rows rewritten by wave 3 are in LDS;
//   waves 0-3  attend to the exact and summary slots (tiles loaded before
//              the barrier, the rewritten rows taken from LDS in every
//              tile), merge; epilogue.
// Tiles of 16 keys: K straight into MFMA fragments, V through a row-major
// LDS copy read back transposed, online softmax per wave.
template <int DH>
__global__ __launch_bounds__(256) void decode_step_bf16(const coda_attn_desc a, const coda_bank_desc s,
                                                        const bf16_t* __restrict__ k_new,
                                                        const bf16_t* __restrict__ v_new, int64_t nb_sb,
                                                        int64_t nb_sh, const float* __restrict__ g_new, int j,
                                                        int64_t pos, const float* __restrict__ rec_in,
                                                        float* __restrict__ rec_out, RopeK rpk) {
  using T = bf16_t;
  constexpr int NC = DH / 32, NM = DH / 16, NW = 4, NVb = (DH + 63) / 64;
  __shared__ __attribute__((aligned(16))) char vt_smem[NW][VtLayout<DH>::kTileBytes];
  __shared__ uint8_t al_lds[kMaxRowsPrefix];
  __shared__ float red_m[NW][16], red_l[NW][16];
  __shared__ DecodeDecision dec;
  // the rows the bank update rewrites: K, V of the exact slot, K, V of the
  // summary slot (new values, for the bank tiles loaded before the update)
  __shared__ __attribute__((aligned(16))) T newrows[4][DH];
  // the next record's dots of head hk (exact slots, then summary slots),
  // and the dots of the two norm rows this update rewrites
  __shared__ float dots_lds[kFusedMaxBank];
  __shared__ float fix_lds[2];
  // bank stage during the update; the partial outputs of the 4 waves after
  extern __shared__ __attribute__((aligned(16))) char ds_u[];
  const int hk = blockIdx.x, b = blockIdx.y;
  const int G = a.H / a.Hkv, R = 2 * G;
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g4 = lane >> 4;
  const float scale = (a.sm_scale > 0.f ? a.sm_scale : rsqrtf((float)DH)) * kLog2e;
  const int Hkv = s.Hkv, W = s.W, Me = s.Me, Ms = s.Ms, Lbuf = W + Me + Ms;
  constexpr int DCH = DH / 8;
  const int kgl = lane / DCH, dcl = lane % DCH;
  const bool vload = kgl < 4;
  char* vt = vt_smem[wv];
  const T* kn_row = k_new + b * nb_sb + hk * nb_sh;
  const T* vn_row = v_new + b * nb_sb + hk * nb_sh;

  // K / V of the (sequence, head) plane and of the new token through raw
  // buffer resources (wave-uniform, in SGPRs); rows past the plane read 0
  auto rsrc = [](const T* p, int nbytes) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0,
                                             __builtin_amdgcn_readfirstlane(nbytes), kBufWord3);
  };
  const int64_t poff = (int64_t)b * a.p_sb + (int64_t)hk * a.p_sh;
  const __amdgpu_buffer_rsrc_t rk = rsrc((const T*)a.kp + poff, Lbuf * DH * 2);
  const __amdgpu_buffer_rsrc_t rv = rsrc((const T*)a.vp + poff, Lbuf * DH * 2);
  const __amdgpu_buffer_rsrc_t rkn = rsrc(kn_row, DH * 2);
  const __amdgpu_buffer_rsrc_t rvn = rsrc(vn_row, DH * 2);
  // a raw new K (rpk.mode != 0): the table entries of this lane's chunks load
  // with the new token's tile (interleaved: the 4 pairs of chunk c in
  // kcs[c]; half-split: the 8 entries chunks q and q + NC/2 share in
  // kcs[2q], kcs[2q + 1])
  uint2 kcs[NC], ksn[NC];
  // tile at key kt of the plane, or (nt) the new token in every row
  auto issue = [&](int kt, bool nt, bf16x8_t (&kf)[NC], uint4 (&vv)[4]) {
    if (nt && rpk.mode) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int e0 = rpk.mode == 1 ? 16 * c + 4 * g4 : 32 * (c >> 1) + 8 * g4 + 4 * (c & 1);
        kcs[c] = *reinterpret_cast<const uint2*>((const T*)rpk.cs + e0);
        ksn[c] = *reinterpret_cast<const uint2*>((const T*)rpk.sn + e0);
      }
    }
    const int koff = nt ? 16 * g4 : (kt + n) * (DH * 2) + 16 * g4;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      kf[c] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(nt ? rkn : rk, koff + 64 * c, 0, 0));
    const int voff = nt ? 16 * dcl : (kt + 4 * (kgl & 3)) * (DH * 2) + 16 * dcl;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      vv[jj] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(nt ? rvn : rv, voff + (nt ? 0 : jj * DH * 2), 0, 0));
  };
  // RoPE of the new token's K fragments (lane: channels 32 c + 8 g4 .. + 8
  // of chunk c), each value as the bank wave writes it into the ring
  auto rope_nt = [&](bf16x8_t (&kf)[NC]) {
    auto half16 = [](uint32_t w, int hi) { return bf2f((bf16_t)(hi ? (w >> 16) : (w & 0xffffu))); };
    auto word = [](const uint2& u, int i) { return i ? u.y : u.x; };
    if (rpk.mode == 1) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 u = __builtin_bit_cast(uint4, kf[c]);
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          float r0, r1;
          rope_pair_t<T>(half16(w[pp], 0), half16(w[pp], 1), half16(word(kcs[c], pp >> 1), pp & 1),
                         half16(word(ksn[c], pp >> 1), pp & 1), true, r0, r1);
          w[pp] = pk_bf16(r0, r1);
        }
        kf[c] = __builtin_bit_cast(bf16x8_t, uint4{w[0], w[1], w[2], w[3]});
      }
    } else {
#pragma unroll
      for (int q = 0; q < NC / 2; ++q) {
        const uint4 ul = __builtin_bit_cast(uint4, kf[q]), uh = __builtin_bit_cast(uint4, kf[q + NC / 2]);
        uint32_t wl[4] = {ul.x, ul.y, ul.z, ul.w}, wh[4] = {uh.x, uh.y, uh.z, uh.w};
        float rl[8], rh[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint2& cw = kcs[2 * q + (e >> 2)];
          const uint2& sw = ksn[2 * q + (e >> 2)];
          rope_pair_t<T>(half16(wl[e >> 1], e & 1), half16(wh[e >> 1], e & 1), half16(word(cw, (e >> 1) & 1), e & 1),
                         half16(word(sw, (e >> 1) & 1), e & 1), false, rl[e], rh[e]);
        }
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          wl[pp] = pk_bf16(rl[2 * pp], rl[2 * pp + 1]);
          wh[pp] = pk_bf16(rh[2 * pp], rh[2 * pp + 1]);
        }
        kf[q] = __builtin_bit_cast(bf16x8_t, uint4{wl[0], wl[1], wl[2], wl[3]});
        kf[q + NC / 2] = __builtin_bit_cast(bf16x8_t, uint4{wh[0], wh[1], wh[2], wh[3]});
      }
    }
  };
  // visibility of this lane's keys kt + 4 g4 + jj of a bank tile: inside
  // [W, Lbuf) and allowed (LDS copy with this step's update applied)
  auto tile_mask = [&](int kt) {
    int m4 = 0;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int kk = kt + 4 * g4 + jj;
      const int in = (kk >= W) & (kk < Lbuf);
      m4 |= (in & (al_lds[in ? kk : W] != 0)) << jj;
    }
    return m4;
  };
  // ring tile kt: inside [0, W), not slot j (the evicted token), allowed
  // (bytes loaded with the tile); the new-token tile keeps its key 0 only
  // (raw bytes, loaded unconditionally with the tile and combined at use:
  // a use right after the load would wait for every load in flight)
  const uint8_t* al_row = a.allowed + (int64_t)b * a.al_sb;
  struct Al4 {
    uint32_t v[4];  // 32-bit: byte values packed into one register would need the loads first
  };
  // (a buffer resource over the W ring bytes: bytes past the ring read 0
  // without a memory access)
  const __amdgpu_buffer_rsrc_t ral = [&]() {
    const uint64_t v = (uint64_t)al_row;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, W, kBufWord3);
  }();
  auto ring_al = [&](int kt) {
    Al4 r;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) r.v[jj] = __builtin_amdgcn_raw_buffer_load_b8(ral, kt + 4 * g4 + jj, 0, 0);
    return r;
  };
  auto ring_mask = [&](int kt, bool nt, const Al4& al) {
    const int ntm = -(int)nt;  // all ones for the new-token tile
    int m4 = 0;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int ok_r = (al.v[jj] != 0) & (kt + 4 * g4 + jj != j);
      const int ok_n = 4 * g4 + jj == 0;
      m4 |= ((ok_n & ntm) | (ok_r & ~ntm)) << jj;
    }
    return m4;
  };
  // phase 1 tiles of waves 0-2: u < nR ring tile u, u == nR the new token
  const int nR = (W + 15) / 16, nB = (Me + Ms + 15) / 16;
  // (u > nR: past the plane, so the buffer loads return 0 without touching
  // memory; issued anyway, which keeps every path's loads alike)
  auto p1_kt = [&](int u) { return u < nR ? 16 * u : u == nR ? 0 : Lbuf; };
  const int n1_w = wv < 3 ? (nR + 1 - wv + 2) / 3 : 0;   // tiles u = wv + 3 i
  // phase 2 tiles: bank tile u of wave u % 4
  const int n2_w = nB > wv ? (nB - wv + 3) / 4 : 0;  // tiles u = wv + 4 i
  // (i >= n2_w: past the plane, so the buffer loads return 0 without
  // touching memory; issued anyway, which keeps every path's loads alike)
  auto kt2 = [&](int i) { return i < n2_w ? W + 16 * (wv + 4 * i) : Lbuf; };

  bf16x8_t kf0[NC], kf1[NC];
  uint4 vv0[4], vv1[4];
  Al4 al0, al1;
  int vm0 = 0, vm1 = 0;
  // ---- prologue: every wave's first loads; no workgroup barrier until the
  // end of phase 1
  // bank wave: the record straight to LDS, evicted / next rows, the
  // visibility bytes of the bank slots
  const int LF = DH - s.lf, words = dstep_words(Hkv, Me, Ms);
  const int jn = j + 1 == W ? 0 : j + 1;
  float* rec = reinterpret_cast<float*>(ds_u);
  T* nnorm_e = reinterpret_cast<T*>(rec + words);  // norm rows the update rewrites
  T* nnorm_s = nnorm_e + DH;
  float* ke = reinterpret_cast<float*>(nnorm_s + DH);
  float* ve = ke + DH;
  float* vnrm = ve + DH;
  float* knrm = vnrm + DH;
  // raw values in 32-bit registers: packing 16- or 8-bit values would make
  // the compiler wait for the loads here
  uint32_t kev[NVb], vev[NVb], xv_r[NVb], xk_r[NVb];
  bool av[NVb], ak[NVb];
  constexpr int kAlBank = 4;  // (Me + Ms) <= 256 bank slots: bytes per lane
  uint32_t alb[kAlBank];
  if (wv == 3) {
    const float* src_r = rec_in + (int64_t)b * words;
    wave_copy_lds(rec, src_r, words * 4, lane);
    const int64_t plane = ((int64_t)b * Hkv + hk) * Lbuf;
    const T* kr = (const T*)s.k_buf + (plane + j) * DH;
    const T* vr = (const T*)s.v_buf + (plane + j) * DH;
    const T* kx = jn == j ? kn_row : (const T*)s.k_buf + (plane + jn) * DH;
    const T* vx = jn == j ? vn_row : (const T*)s.v_buf + (plane + jn) * DH;
#pragma unroll
    for (int i = 0; i < NVb; ++i) {
      const int d = lane + 64 * i;
      const int dc = d < DH ? d : 0;
      av[i] = d < DH;
      ak[i] = d < LF;
      kev[i] = kr[dc];
      vev[i] = vr[dc];
      xv_r[i] = vx[dc];
      xk_r[i] = kx[s.lf + (ak[i] ? d : 0)];
    }
#pragma unroll
    for (int k = 0; k < kAlBank; ++k) {
      const int m = lane + 64 * k;
      alb[k] = al_row[W + (m < Me + Ms ? m : 0)];
    }
  }
  // epilogue operands (raw: a conversion here would wait for every load in
  // flight)
  constexpr int NV = (DH + 63) / 64;
  uint32_t lam_r[2] = {0, 0}, w_r[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) w_r[i] = 0x3f80;  // 1.0
  // (unconditional, from clamped valid addresses: a branch would end in a
  // wait for the loads)
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int orow = min(wv + r * NW, G - 1);
    lam_r[r] = ((const T*)a.lam)[b * a.lam_sb + (hk * G + orow) * a.lam_sh];
  }
  const T* w_src = a.rms_w ? (const T*)a.rms_w : (const T*)a.lam;
#pragma unroll
  for (int i = 0; i < NV; ++i) w_r[i] = w_src[a.rms_w ? min(lane + 64 * i, DH - 1) : 0];
  // query fragments of every wave (B operand of S^T): row n = stream st,
  // head g; RoPE and the noise rotation as bf16 dot2 pairs, or given noise
  // queries; the half-split RoPE with the eager-op rounding
  bf16x8_t qf[NC];
  {
    using E = Elt<T>;
    constexpr int half = DH / 2;
    const bool live = n < R;
    const int st = live ? n / G : 0, h = hk * G + (live ? n % G : 0);
    const bool given = st == 1 && a.q_noise != nullptr;
    const bool rot = st == 1 && a.q_noise == nullptr;
    const T* qr = given ? (const T*)a.q_noise + b * a.qn_sb + h * a.qn_sh : (const T*)a.q + b * a.q_sb + h * a.q_sh;
    const bool rope = a.rope_cos != nullptr && !given, inter = a.rope_interleaved != 0;
    const T* csr = (const T*)a.rope_cos;
    const T* snr = (const T*)a.rope_sin;
    uint4 uq[NC], up[NC], rc[NC], rs[NC];
    uint2 rc2[NC], rs2[NC], tcs[NC], tsn[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d0 = 32 * c + 8 * g4;
      if (wv == 3) break;  // wave 3 takes its fragments from wave 0 after phase 1
      uq[c] = *reinterpret_cast<const uint4*>(qr + d0);
      if (rope && inter) {
        rc2[c] = *reinterpret_cast<const uint2*>(csr + d0 / 2);
        rs2[c] = *reinterpret_cast<const uint2*>(snr + d0 / 2);
      }
      if (rope && !inter) {
        const int f0 = d0 < half ? d0 : d0 - half;
        up[c] = *reinterpret_cast<const uint4*>(qr + (d0 < half ? d0 + half : d0 - half));
        rc[c] = *reinterpret_cast<const uint4*>(csr + f0);
        rs[c] = *reinterpret_cast<const uint4*>(snr + f0);
      }
      if (rot) {
        tcs[c] = *reinterpret_cast<const uint2*>((const T*)a.theta_cos + (int64_t)h * half + d0 / 2);
        tsn[c] = *reinterpret_cast<const uint2*>((const T*)a.theta_sin + (int64_t)h * half + d0 / 2);
      }
    }
    // the first two ring tiles load behind the queries
    if (wv < 3) {
      issue(p1_kt(wv), wv == nR, kf0, vv0);
      al0 = ring_al(p1_kt(wv));
      issue(p1_kt(wv + 3), wv + 3 == nR, kf1, vv1);
      al1 = ring_al(p1_kt(wv + 3));
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d0 = 32 * c + 8 * g4;
      if (wv == 3) break;
      uint32_t w[4] = {uq[c].x, uq[c].y, uq[c].z, uq[c].w};
      if (rope && inter) {
#pragma unroll
        for (int pp = 0; pp < 4; ++pp)
          w[pp] = rot_pair(w[pp], pp >> 1 ? rc2[c].y : rc2[c].x, pp >> 1 ? rs2[c].y : rs2[c].x, pp & 1);
      }
      if (rope && !inter) {
        float x[8], cc[8], ss[8], y[8];
        unpack8(uq[c], x);
        unpack8(rc[c], cc);
        unpack8(rs[c], ss);
        unpack8(up[c], y);
        const bool lo = d0 < half;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const float rt = lo ? -y[jj] : y[jj];
          x[jj] = E::rnd(E::rnd(x[jj] * cc[jj]) + E::rnd(rt * ss[jj]));
        }
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) w[pp] = pk_bf16(x[2 * pp], x[2 * pp + 1]);
      }
      if (rot) {
#pragma unroll
        for (int pp = 0; pp < 4; ++pp)
          w[pp] = rot_pair(w[pp], pp >> 1 ? tcs[c].y : tcs[c].x, pp >> 1 ? tsn[c].y : tsn[c].x, pp & 1);
      }
      qf[c] = __builtin_bit_cast(bf16x8_t, live ? uint4{w[0], w[1], w[2], w[3]} : uint4{0, 0, 0, 0});
    }
    // wave 0 leaves the fragments for wave 3 in wave 3's (idle) V buffer
    if (wv == 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
        reinterpret_cast<uint4*>(vt_smem[3])[c * 64 + lane] = __builtin_bit_cast(uint4, qf[c]);
    }
  }
  float m_i = -INFINITY, l_i = 0.f;
  f32x4 o[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  // V of a tile goes row-major into the wave's LDS buffer (rows padded to
  // 2 DH + 32 bytes, which spreads the 4 rows of a transposed read over
  // distinct banks) and comes back through transposed reads: lane (n, g4)
  // gets channel 16 mt + n of keys 4 g4 .. 4 g4 + 3, the A operand of the
  // PV product
  constexpr int VRB = 2 * DH + 32;
  static_assert(16 * VRB <= VtLayout<DH>::kTileBytes, "V tile fits the wave's LDS buffer");
  const int v_rd = (4 * g4 + (n >> 2)) * VRB + 8 * (n & 3);
  const int v_wr = 4 * (kgl & 3) * VRB + 16 * dcl;
  auto consume = [&](const bf16x8_t (&kf)[NC], const uint4 (&vv)[4], int vmask) {
    f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) st = mfma_k32(kf[c], qf[c], st);
    float sv[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      sv[jj] = ((vmask >> jj) & 1) ? st[jj] * scale : -INFINITY;
      tmax = fmaxf(tmax, sv[jj]);
    }
    // max and sum over the 4 lane groups through permlane swaps (no LDS)
    tmax = xmax32(xmax16(tmax));
    const float mnew = fmaxf(m_i, tmax);
    const float muse = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = fast_exp2(m_i - muse);
    // the accumulators need rescaling only where a running max moved
    const bool grow = __builtin_amdgcn_ballot_w64(mnew != m_i) != 0;
    float p[4], ps = 0.f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      p[jj] = bf2f(f2bf(fast_exp2(sv[jj] - muse)));
      ps += p[jj];
    }
    // (l_i is this lane's share of the row sum, rescaled with the row's
    // alpha, which every lane group of the row shares; the four shares add
    // up once, before the merge)
    l_i = l_i * alpha + ps;
    m_i = mnew;
    const short4_t pf = pack4(p[0], p[1], p[2], p[3]);
    if (vload) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) *reinterpret_cast<uint4*>(vt + v_wr + jj * VRB) = vv[jj];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): LDS writes of this wave done
    __builtin_amdgcn_wave_barrier();
    if (grow) {
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) o[mt] *= alpha;
    }
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) {
      const uint2 cell = lds_read_tr16(vt + v_rd + 32 * mt);
      o[mt] = mfma_k16(__builtin_bit_cast(short4_t, cell), pf, o[mt]);
    }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- phase 1
  if (wv < 3) {
    // ring tiles and the new token, ping-pong register buffers, two in
    // flight: a buffer is refilled as soon as it has been consumed
    for (int i = 0; i < n1_w; i += 2) {
      const int u0 = wv + 3 * i;
      vm0 = ring_mask(p1_kt(u0), u0 == nR, al0);
      if (rpk.mode && u0 == nR) rope_nt(kf0);
      __builtin_amdgcn_sched_barrier(0);
      consume(kf0, vv0, vm0);
      issue(p1_kt(u0 + 6), u0 + 6 == nR, kf0, vv0);
      al0 = ring_al(p1_kt(u0 + 6));
      if (i + 1 >= n1_w) break;
      const int u1 = u0 + 3;
      vm1 = ring_mask(p1_kt(u1), u1 == nR, al1);
      if (rpk.mode && u1 == nR) rope_nt(kf1);
      __builtin_amdgcn_sched_barrier(0);
      consume(kf1, vv1, vm1);
      issue(p1_kt(u1 + 6), u1 + 6 == nR, kf1, vv1);
      al1 = ring_al(p1_kt(u1 + 6));
    }
    // the next step's record: head hk's dots against its norm rows (the
    // rows this step's update rewrites are redone by wave 3).  One lane per
    // norm row, each dot a sequential chain in the CPU matmul order
    // (lane_dot_cpu_order): exact rows on lanes 0 .. Me-1 of the waves in
    // order, then summary rows.  Loads first: slot j+1's rows (this wave's
    // own unit rows), then this wave's first two bank tiles (a row the
    // update rewrites is replaced from LDS after the barrier)
    {
      const T* en = (const T*)s.exact_v_norm + ((int64_t)b * Hkv + hk) * Me * DH;
      const T* sn = (const T*)s.sum_lf_k_norm + ((int64_t)b * Hkv + hk) * Ms * LF;
      const int64_t plane = ((int64_t)b * Hkv + hk) * Lbuf;
      const T* kx = jn == j ? kn_row : (const T*)s.k_buf + (plane + jn) * DH;
      const T* vx = jn == j ? vn_row : (const T*)s.v_buf + (plane + jn) * DH;
      uint32_t nv_r[NVb], nk_r[NVb];
#pragma unroll
      for (int i = 0; i < NVb; ++i) {
        nv_r[i] = vx[min(lane + 64 * i, DH - 1)];
        nk_r[i] = kx[s.lf + min(lane + 64 * i, LF - 1)];
      }
      issue(kt2(0), false, kf0, vv0);
      issue(kt2(1), false, kf1, vv1);
      // unit rows of slot j+1 through the wave's (idle) V buffer
      float* un = reinterpret_cast<float*>(vt);
      {
        float xv[NVb], xk[NVb];
        bool av2[NVb], ak2[NVb];
#pragma unroll
        for (int i = 0; i < NVb; ++i) {
          av2[i] = lane + 64 * i < DH;
          ak2[i] = lane + 64 * i < LF;
          xv[i] = av2[i] ? bf2f((bf16_t)nv_r[i]) : 0.f;
          xk[i] = ak2[i] ? bf2f((bf16_t)nk_r[i]) : 0.f;
        }
        wave_unit<T, NVb>(xv, av2);
        wave_unit<T, NVb>(xk, ak2);
#pragma unroll
        for (int i = 0; i < NVb; ++i) {
          if (av2[i]) un[lane + 64 * i] = xv[i];
          if (ak2[i]) un[DH + lane + 64 * i] = xk[i];
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_wave_barrier();
      for (int r = 64 * wv + lane; r < Me + Ms; r += 192) {
        const bool ex = r < Me;
        // (every 16-byte piece of the row in flight at once: one memory
        // round trip before the chain instead of one per few pieces)
        const float acc = ex ? lane_dot_cpu_order<T, DH / 16>(en + (int64_t)r * DH, un, DH)
                             : lane_dot_cpu_order<T, DH / 16>(sn + (int64_t)(r - Me) * LF, un + DH, LF);
        dots_lds[r] = Elt<T>::rnd(acc);
      }
    }
  } else {
    // the bank update of head hk (one wave)
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): record, norm rows, evicted / next rows
    float xv[NVb], xk[NVb];
#pragma unroll
    for (int i = 0; i < NVb; ++i) {
      if (av[i]) {
        ke[lane + 64 * i] = bf2f((bf16_t)kev[i]);
        ve[lane + 64 * i] = bf2f((bf16_t)vev[i]);
      }
      xv[i] = av[i] ? bf2f((bf16_t)xv_r[i]) : 0.f;
      xk[i] = ak[i] ? bf2f((bf16_t)xk_r[i]) : 0.f;
    }
    // unit rows of the token evicted next (for the next record's dots,
    // taken by every wave after the barrier)
    if (Me > 0) {
      wave_unit<T, NVb>(xv, av);
#pragma unroll
      for (int i = 0; i < NVb; ++i)
        if (av[i]) vnrm[lane + 64 * i] = xv[i];
    }
    if (Ms > 0) {
      wave_unit<T, NVb>(xk, ak);
#pragma unroll
      for (int i = 0; i < NVb; ++i)
        if (ak[i]) knrm[lane + 64 * i] = xk[i];
    }
    const DStepWs L = dstep_ws(rec, 0, Hkv, Me, Ms);
    const float g_e = *L.g_e;
    if (Me > 0) decide_exact<T>(s, L.dots, L.used, L.last, g_e, dec, hk == 0, lane);
    if (Ms > 0) decide_summary<T>(s, L.dots + Hkv * Me, L.used + Me, g_e, dec, hk == 0, lane);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the decision (lane 0) is in LDS
    __builtin_amdgcn_wave_barrier();
    const DecodeDecision dd = dec;
    apply_head<T, DH>(s, b, hk, dd, ke, ve, kn_row, vn_row, j, g_e, lane, nnorm_e, nnorm_s, &newrows[0][0], rpk);
    if (hk == 0) {
      // metadata of the sequence, and the next record's snapshot of it
      const DStepWs wn = dstep_ws(rec_out, b, Hkv, Me, Ms);
      const bool ow_e = Me > 0 && dd.ow_e, keep_e = Me > 0 && dd.keep_e, keep_s = Ms > 0 && dd.keep_s;
      const int ie = Me > 0 ? dd.idx_e : -1, is = Ms > 0 ? dd.idx_s : -1;
      for (int m = lane; m < Me + Ms; m += 64)
        wn.used[m] = L.used[m] | ((ow_e && m == ie) || (keep_s && m == Me + is) ? 1 : 0);
      for (int m = lane; m < Me; m += 64) wn.last[m] = (keep_e && m == ie) ? pos - W : L.last[m];
      if (lane == 0) {
        *wn.g_e = jn == j ? g_new[b] : s.g_recent[(int64_t)b * W + jn];
        commit_decode_meta(s, b, dd, j, pos - W, g_new[b]);
      }
    }
    // visibility bytes of the bank slots, with the slots this update fills
#pragma unroll
    for (int k = 0; k < kAlBank; ++k) {
      const int m = lane + 64 * k;
      const bool fill = (Me > 0 && dd.ow_e && m == dd.idx_e) || (Ms > 0 && dd.keep_s && m == Me + dd.idx_s);
      if (m < Me + Ms) al_lds[W + m] = fill ? (uint8_t)1 : (uint8_t)alb[k];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): rewritten norm rows in LDS
    __builtin_amdgcn_wave_barrier();
    // the record dots of the norm rows this update rewrote: exact row on
    // lane 0, summary row on lane 1
    // (one call on operands chosen per lane, so the two chains run side by
    // side rather than one after the other)
    if (lane < 2) {
      const bool ex = lane == 0;
      if (ex ? (Me > 0 && dd.ow_e) : (Ms > 0 && dd.keep_s))
        fix_lds[lane] = Elt<T>::rnd(lane_dot_cpu_order<T, DH / 8>(ex ? nnorm_e : nnorm_s, ex ? vnrm : knrm,
                                                                   ex ? DH : LF));
    }
  }
  if (wv == 3) {
    // the bank wave's two bank tiles (rows the update rewrote are replaced
    // from LDS after the barrier)
    issue(kt2(0), false, kf0, vv0);
    issue(kt2(1), false, kf1, vv1);
  }
  __syncthreads();  // the decision, new rows, bank visibility bytes and record dots in LDS
  if (wv == 3) {
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[c] = __builtin_bit_cast(bf16x8_t, reinterpret_cast<const uint4*>(vt_smem[3])[c * 64 + lane]);
  }

  // ---- phase 2: exact and summary slots; rows this step's update rewrote
  // come from LDS in every tile
  {
    const int re = Me > 0 && dec.ow_e ? W + dec.idx_e : -1;
    const int rs = Ms > 0 && dec.keep_s ? W + Me + dec.idx_s : -1;
    auto patch = [&](int kt, bf16x8_t (&kf)[NC], uint4 (&vv)[4]) {
      const int rk = kt + n;
      if (rk == re || rk == rs) {
        const T* src = newrows[rk == re ? 0 : 2];
#pragma unroll
        for (int c = 0; c < NC; ++c) kf[c] = *reinterpret_cast<const bf16x8_t*>(src + 32 * c + 8 * g4);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int rv = kt + 4 * (kgl & 3) + jj;
        if (rv == re || rv == rs) vv[jj] = *reinterpret_cast<const uint4*>(newrows[rv == re ? 1 : 3] + 8 * dcl);
      }
    };
    auto step2 = [&](int i, bf16x8_t (&kf)[NC], uint4 (&vv)[4]) {
      const int kt = kt2(i);
      patch(kt, kf, vv);
      const int vm = tile_mask(kt);
      __builtin_amdgcn_sched_barrier(0);
      consume(kf, vv, vm);
      issue(kt2(i + 2), false, kf, vv);
    };
    for (int i = 0; i < n2_w; i += 2) {
      step2(i, kf0, vv0);
      if (i + 1 >= n2_w) break;
      step2(i + 1, kf1, vv1);
    }
  }
  // ---- merge the 4 waves (rows r < R), epilogue (the bank stage is free)
  float* red_o = reinterpret_cast<float*>(ds_u);  // [NW][R][DH + 4]
  l_i = xsum32(xsum16(l_i));
  if (g4 == 0) {
    red_m[wv][n] = m_i;
    red_l[wv][n] = l_i;
  }
  if (n < R) {
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) red_o[(wv * R + n) * (DH + 4) + 16 * mt + 4 * g4 + jj] = o[mt][jj];
  }
  __syncthreads();
  // the next record's dots of head hk; the rewritten rows' from the bank wave
  {
    float* out_e = rec_out + (int64_t)b * words + (int64_t)hk * Me;
    float* out_s = rec_out + (int64_t)b * words + (int64_t)Hkv * Me + (int64_t)hk * Ms;
    const int ie = Me > 0 && dec.ow_e ? dec.idx_e : -1;
    const int is = Ms > 0 && dec.keep_s ? dec.idx_s : -1;
    for (int m = threadIdx.x; m < Me + Ms; m += blockDim.x) {
      if (m < Me) out_e[m] = m == ie ? fix_lds[0] : dots_lds[m];
      else out_s[m - Me] = m - Me == is ? fix_lds[1] : dots_lds[m];
    }
  }
  for (int orow = wv, r_pf = 0; orow < G; orow += NW, ++r_pf) {
    const int h = hk * G + orow;
    float os[NV], on[NV], y[NV];
    bool act[NV];
    int dd[NV];
    float M[2] = {-INFINITY, -INFINITY}, Ls[2] = {0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int r = st * G + orow;
#pragma unroll
      for (int w = 0; w < NW; ++w) M[st] = fmaxf(M[st], red_m[w][r]);
      const float Mu = M[st] == -INFINITY ? 0.f : M[st];
#pragma unroll
      for (int w = 0; w < NW; ++w) Ls[st] += red_l[w][r] * exp2f(red_m[w][r] - Mu);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = d < DH;
      dd[i] = act[i] ? d : 0;
      float acc[2] = {0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int r = st * G + orow;
        const float Mu = M[st] == -INFINITY ? 0.f : M[st];
#pragma unroll
        for (int w = 0; w < NW; ++w) acc[st] += red_o[(w * R + r) * (DH + 4) + dd[i]] * exp2f(red_m[w][r] - Mu);
        acc[st] = Ls[st] > 0.f ? acc[st] / Ls[st] : 0.f;
      }
      os[i] = act[i] ? acc[0] : 0.f;
      on[i] = act[i] ? acc[1] : 0.f;
    }
    const float lam = bf2f((bf16_t)(r_pf == 0 ? lam_r[0] : r_pf == 1 ? lam_r[1] : ((const T*)a.lam)[b * a.lam_sb + h * a.lam_sh]));
    float w_pf[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) w_pf[i] = bf2f((bf16_t)w_r[i]);
    diff_norm_w<NV>(y, os, on, act, lam, a.rms_w ? w_pf : nullptr, a.eps, DH);
    T* orow_p = (T*)a.out + b * a.o_sb + h * a.o_sh;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) orow_p[dd[i]] = f2bf(y[i]);
  }
}

// ------------------------------------------------------------ prefill tiles
// Workgroup = (query block of 16*NQ, KV head, batch), NW = G*NQ waves;
// wave w owns head g = w / NQ and queries q0 + 16*(w % NQ) + [0,16) as two
// 16-row tiles (signal, noise).
template <int DH, int NW>
__global__ __launch_bounds__(NW * 64) void attn_tile_bf16(const coda_attn_desc a, int NQ) {
  constexpr int NC = DH / 32, NM = DH / 16, KT = 64;
  constexpr int KROW = DH * 2 + 16;  // padded K row bytes
  __shared__ __attribute__((aligned(16))) char k_smem[KT * KROW];
  __shared__ __attribute__((aligned(16))) char v_smem[4 * VtLayout<DH>::kTileBytes];
  const int qb = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int G = a.H / a.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int n = lane & 15, g4 = lane >> 4;
  const int g = wv / NQ, qsub = wv % NQ, h = hk * G + g;
  const int q0 = qb * 16 * NQ + 16 * qsub;
  const int qrow = q0 + n;
  const bool qlive = qrow < a.Lq;
  const float scale = (a.sm_scale > 0.f ? a.sm_scale : rsqrtf((float)DH)) * kLog2e;

  bf16x8_t qf[2][NC];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (qlive) prep_q8<bf16_t>(a, b, h, qrow, 32 * c + 8 * g4, s, x);
      qf[s][c] = pack8(x);
    }
  float m_i[2] = {-INFINITY, -INFINITY}, l_i[2] = {0.f, 0.f};
  f32x4 o[2][NM];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < NM; ++i) o[s][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // visibility bytes of the prefix (the host guarantees Lp <= kMaxRowsPrefix)
  __shared__ uint8_t al_lds[kMaxRowsPrefix];
  for (int i = tid; i < a.Lp; i += NW * 64) al_lds[i] = a.allowed ? a.allowed[(int64_t)b * a.al_sb + i] : (uint8_t)1;
  const int Lk = a.Lp + a.Lb;
  // last key any query of this workgroup can see
  const int qlast = min(a.Lq - 1, qb * 16 * NQ + 16 * NQ - 1);
  const int coff = a.causal == 2 ? 0 : a.Lb - a.Lq;
  const int klim = a.causal ? min(Lk, a.Lp + qlast + coff + 1) : Lk;
  constexpr int DCH = DH / 8;
  const int nthreads = NW * 64;

  for (int k0 = 0; k0 < klim; k0 += KT) {
    __syncthreads();
    // K tile: 64 keys x DCH chunks of 16 bytes, row-major (padded rows)
    for (int i = tid; i < KT * DCH; i += nthreads) {
      const int kk = i / DCH, dc = i % DCH;
      const int kidx = k0 + kk;
      uint4 u = uint4{0, 0, 0, 0};
      if (kidx < Lk) u = *reinterpret_cast<const uint4*>(key_ptr<bf16_t>(a, b, hk, kidx, false) + 8 * dc);
      *reinterpret_cast<uint4*>(k_smem + kk * KROW + dc * 16) = u;
    }
    // V tile: 16 key groups x DCH chunks, transposed into 4 sub-tiles
    for (int i = tid; i < 16 * DCH; i += nthreads) {
      const int kg = i / DCH, dc = i % DCH;
      uint4 vv[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int kidx = k0 + 4 * kg + jj;
        vv[jj] = kidx < Lk ? *reinterpret_cast<const uint4*>(key_ptr<bf16_t>(a, b, hk, kidx, true) + 8 * dc)
                           : uint4{0, 0, 0, 0};
      }
      store_vt<DH>(v_smem + (kg >> 2) * VtLayout<DH>::kTileBytes, kg & 3, 8 * dc, vv);
    }
    __syncthreads();
#pragma unroll
    for (int sub = 0; sub < KT / 16; ++sub) {
      const int kt = k0 + 16 * sub;
      if (kt >= klim) break;
      f32x4 st[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 u = *reinterpret_cast<const uint4*>(k_smem + (16 * sub + n) * KROW + (32 * c + 8 * g4) * 2);
        const bf16x8_t kf = __builtin_bit_cast(bf16x8_t, u);
        st[0] = mfma_k32(kf, qf[0][c], st[0]);
        st[1] = mfma_k32(kf, qf[1][c], st[1]);
      }
      bool vis[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kidx = kt + 4 * g4 + j;
        const int jb = kidx - a.Lp;
        vis[j] = kidx < a.Lp ? al_lds[kidx] != 0
                             : (jb < a.Lb && (!a.causal || jb <= qrow + (a.causal == 2 ? 0 : a.Lb - a.Lq)));
      }
      short4_t pf[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float sv[4], tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sv[j] = vis[j] ? st[s][j] * scale : -INFINITY;
          tmax = fmaxf(tmax, sv[j]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(m_i[s], tmax);
        const float muse = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = exp2f(m_i[s] - muse);
        float p[4], ps = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p[j] = bf2f(f2bf(exp2f(sv[j] - muse)));
          ps += p[j];
        }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l_i[s] = l_i[s] * alpha + ps;
        m_i[s] = mnew;
        pf[s] = pack4(p[0], p[1], p[2], p[3]);
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) o[s][mt] *= alpha;
      }
      const char* vsub = v_smem + sub * VtLayout<DH>::kTileBytes;
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) {
        const uint2 cell = *reinterpret_cast<const uint2*>(vsub + VtLayout<DH>::off(g4, 16 * mt + n));
        const short4_t vf = __builtin_bit_cast(short4_t, cell);
        o[0][mt] = mfma_k16(vf, pf[0], o[0][mt]);
        o[1][mt] = mfma_k16(vf, pf[1], o[1][mt]);
      }
    }
  }
  // epilogue in registers: lane holds channels 16 mt + 4 g4 + j of row n
  constexpr int NV = NM * 4;
  float os[NV], on[NV], y[NV];
  bool act[NV];
  int dd[NV];
#pragma unroll
  for (int mt = 0; mt < NM; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = mt * 4 + j;
      dd[i] = 16 * mt + 4 * g4 + j;
      act[i] = true;
      os[i] = l_i[0] > 0.f ? o[0][mt][j] / l_i[0] : 0.f;
      on[i] = l_i[1] > 0.f ? o[1][mt][j] / l_i[1] : 0.f;
    }
  const float lam = qlive ? bf2f(((const bf16_t*)a.lam)[b * a.lam_sb + h * a.lam_sh + qrow * a.lam_sl]) : 0.f;
  diff_norm<bf16_t, NV>(y, os, on, act, lam, (const bf16_t*)a.rms_w, dd, a.eps, DH, false, 16, 32);
  if (qlive) {
    bf16_t* orow_p = (bf16_t*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)qrow * a.o_sl;
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) {
      uint2 u;
      u.x = (uint32_t)f2bf(y[mt * 4 + 0]) | ((uint32_t)f2bf(y[mt * 4 + 1]) << 16);
      u.y = (uint32_t)f2bf(y[mt * 4 + 2]) | ((uint32_t)f2bf(y[mt * 4 + 3]) << 16);
      *reinterpret_cast<uint2*>(orow_p + 16 * mt + 4 * g4) = u;
    }
  }
}

// s_waitcnt vmcnt(n) for a run-time n in [0, 15] (the count is an immediate)
__device__ __forceinline__ void vm_wait(int n) {
  switch (n) {
#define CODA_VMW(k) \
  case k: __builtin_amdgcn_s_waitcnt(((k) & 15) | 0x0f70); break;
    CODA_VMW(0) CODA_VMW(1) CODA_VMW(2) CODA_VMW(3) CODA_VMW(4) CODA_VMW(5) CODA_VMW(6) CODA_VMW(7)
    CODA_VMW(8) CODA_VMW(9) CODA_VMW(10) CODA_VMW(11) CODA_VMW(12) CODA_VMW(13) CODA_VMW(14) CODA_VMW(15)
#undef CODA_VMW
    default: __builtin_amdgcn_s_waitcnt(0x0f70); break;
  }
}

// ------------------------------------------------------------ prefill flash tiles, 32-row MFMA
// The tiles of the MFMA path for prefill chunks and unbounded attention
// (head_dim 64 / 128, attn_f3_bf16).  Workgroup = (query block, KV head,
// sequence); wave
// w owns head g = w / NQ and 16 queries, BOTH streams: the wave's 32 MFMA
// rows are the 16 signal queries (rows 0-15) and the same 16 queries
// rotated into the noise stream (rows 16-31).  Every K / V fragment a wave
// reads from LDS therefore feeds a 32 x 32 x 16 product (twice the FLOPs
// per LDS byte of a 16-row wave), and the epilogue finds O_noise one
// permlane swap away (lanes l and l ^ 16).
//   S^T = K Q^T per 32-key block kb: A = K fragment (32 keys x 16 channels,
//     lane l: key l % 32, channels 8 (l / 32) ..+8, one contiguous 16-byte
//     read: K sits in LDS in fragment order), B = Q^T (lane l: row l % 32,
//     the same channels), D: lane l holds row l % 32 and keys
//     8 (j / 4) + 4 (l / 32) + j % 4 of the block in register j.
//   O^T += V^T P^T per 16-key step (kb, ph): B = registers 8 ph .. 8 ph + 7
//     of S^T block kb (already the B layout, with k-slot i standing for key
//     16 ph + 8 (i / 4) + 4 (l / 32) + i % 4), A = V^T with the same key
//     order: two ds_read_b64_tr_b16 of rows 4 (l / 32) + 0..3 and + 8, at
//     channel 32 db + l % 32.  V is row-major in LDS with 16-byte chunks
//     XOR-swizzled per row (F2Layout::vchunk) so each transposed read
//     touches every bank group.
// Online softmax per row with a lazy rescale (the running max moves only
// when a tile's max exceeds it by more than 2^8); P rounded to bf16 by the
// hardware conversion.
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma_32x32x16(const bf16x8_t& a, const bf16x8_t& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ds_read_b128 issued by hand at an immediate offset (see lds_read_tr16_at)
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));
template <int OFF>
__device__ __forceinline__ u32x4v_t lds_read_b128_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  u32x4v_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int N>
__device__ __forceinline__ void lds_wait_b128(u32x4v_t& a) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(N));
}
template <int N>
__device__ __forceinline__ void lds_wait2_n(uint2& a, uint2& b) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}

template <int DH>
struct F2Layout {
  static constexpr int KT = 64;                  // keys per tile
  static constexpr int NKS = DH / 16;            // 16-channel steps of S^T
  static constexpr int NDB = DH / 32;            // 32-channel blocks of O^T
  static constexpr int KBYTES = 2 * NKS * 1024;  // K tile: fragments (kb, ks)
  static constexpr int ROWB = DH * 2;            // V row (one key)
  static constexpr int CPR = DH / 8;             // 16-byte chunks per V row
  static constexpr int VBYTES = KT * ROWB;
  static constexpr int RPI = 1024 / ROWB;        // V rows per 1 KiB direct load
  static constexpr int KCH = 2 * NKS, VCH = VBYTES / 1024;
  static constexpr int LDS = 2 * (KBYTES + VBYTES);  // two tiles in flight
  // stored chunk of chunk c of V row r (an involution): the 64-byte
  // segments of the eight rows one transposed read touches land in
  // distinct bank groups, two rows a group
  static __host__ __device__ __forceinline__ int vchunk(int r, int c) {
    return DH == 128 ? (c ^ (4 * (r & 3))) : (c ^ (4 * ((r >> 1) & 1)));
  }
};

// ------------------------------------------------------------ prefill flash tiles, pipelined
// attn_f3_bf16: the 32-row tiles above (32 MFMA rows per wave: 16 queries x
// both streams; S^T = K Q^T and O^T += V^T P^T as 32 x 32 x 16 products),
// software-pipelined so the matrix and vector pipes work at the same time
// within each wave.  Iteration it, with S(it) already masked and its row
// max folded into the running max:
//   phase A: the 16 products of S(it + 1) (tile it + 1's K fragments),
//            each followed by the exp / row sum / bf16 packing of two of
//            this lane's 32 entries of P(it);
//   phase C: the 4 NDB products of O += V(it)^T P(it), each followed by the
//            mask and running-max work of two entries of S(it + 1);
//   then the lazy rescale (only when a row max moves by more than 2^8).
// NS = 4: four tiles live in LDS (it, it + 1, and it + 2, it + 3 loading),
// so one barrier per tile suffices and a tile's loads have two iterations
// to land; 128 KiB, one workgroup a CU.  NS = 2: K and V in two buffers
// each, K one tile ahead (iteration it reads K(it + 1) and V(it) while
// K(it + 2) and V(it + 1) load into the buffers of K(it) and V(it - 1));
// 64 KiB, so two workgroups of 4 waves share a CU and one's prologue,
// epilogue and barriers overlap the other's products; a tile's loads have
// one iteration to land.
// Whole tiles inside the prefix or the block load from a wave-uniform base
// plus per-lane offsets.
static constexpr int kTabRows = 64;  // query rows whose RoPE tables attn_f3_bf16 stages in LDS
template <int DH>
constexpr int f3_tab_pitch() { return DH / 2 + 8; }  // table row pitch in LDS (bf16)
// NS = 2: the tables sit in the second V buffer and may run past it
template <int DH>
constexpr int f3_table_offset() { return 2 * F2Layout<DH>::KBYTES + F2Layout<DH>::VBYTES; }
template <int DH, int NS>
constexpr size_t f3_lds_bytes() {
  constexpr size_t tiles = (size_t)NS * (F2Layout<DH>::KBYTES + F2Layout<DH>::VBYTES);
  constexpr size_t tabs = f3_table_offset<DH>() + 2 * 2 * (size_t)kTabRows * f3_tab_pitch<DH>() + 2 * 2 * 8 * (DH / 2);
  return NS == 4 || tabs < tiles ? tiles : tabs;
}

// Chunks of a prefill call in one launch (coda_prefill_attn_chunks):
// blockIdx.y = chunk c_first + y, covering queries [t0, t0 + Lq) of the
// call, t0 = c blk, Lq = min(blk, L - t0); its block keys are the call's
// keys [t0 - win, t0 + Lq) with win = min(t0, W) (the ring window, in time
// order, then the chunk itself, lower-right causal); its prefix is bank
// snapshot y (prefix pointers and visibility bytes advanced by y strides).
// n == 0: one chunk, as the descriptor says.
struct ChunkGeom {
  int n, c_first, blk, L, W, pad;
  int64_t snap_stride;  // elements from one snapshot's K / V to the next
  int64_t al_stride;    // bytes from one snapshot's visibility bytes to the next
};
template <int DH>
__device__ __forceinline__ coda_attn_desc chunk_view(const coda_attn_desc& a0, const ChunkGeom& cg) {
  if (cg.n == 0) return a0;
  coda_attn_desc a = a0;
  const int y = blockIdx.y;
  const int64_t t0 = (int64_t)(cg.c_first + y) * cg.blk;
  const int Lq = min(cg.blk, cg.L - (int)t0);
  const int win = min((int)t0, cg.W);
  using B = const bf16_t*;
  a.q = (B)a0.q + t0 * a0.q_sl;
  a.lam = (B)a0.lam + t0 * a0.lam_sl;
  a.out = (bf16_t*)a0.out + t0 * a0.o_sl;
  if (a0.rope_cos) {
    a.rope_cos = (B)a0.rope_cos + t0 * (DH / 2);
    a.rope_sin = (B)a0.rope_sin + t0 * (DH / 2);
  }
  a.kb = (B)a0.kb + (t0 - win) * a0.b_sl;
  a.vb = (B)a0.vb + (t0 - win) * a0.b_sl;
  a.Lq = Lq;
  a.Lb = win + Lq;
  a.kp = (B)a0.kp + y * cg.snap_stride;
  a.vp = (B)a0.vp + y * cg.snap_stride;
  if (a0.allowed) a.allowed = a0.allowed + y * cg.al_stride;
  return a;
}

template <int DH, int NW, int QM, bool TB, int NS>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void attn_f3_bf16(
    const coda_attn_desc a_, int NQ, int nqb, int npairs, ChunkGeom cg) {
  const coda_attn_desc a = chunk_view<DH>(a_, cg);
  using Lay = F2Layout<DH>;
  static_assert(NS == 2 || NS == 4, "tile stages");
  static_assert(!TB || QM == 0 || QM == 1, "tables staged for the RoPE + rotation query cases");
  constexpr int kTabPitch = f3_tab_pitch<DH>();
  constexpr int KT = Lay::KT, NKS = Lay::NKS, NDB = Lay::NDB, KCH = Lay::KCH, VCH = Lay::VCH;
  constexpr int KCW = (KCH + NW - 1) / NW, VCW = (VCH + NW - 1) / NW;
  static_assert(KCH % NW == 0 && VCH % NW == 0, "tile pieces split evenly over the waves");
  constexpr int STAGE = Lay::KBYTES + Lay::VBYTES;
  extern __shared__ __attribute__((aligned(16))) char f3_smem[];
  __shared__ __attribute__((aligned(16))) uint8_t al_lds[kMaxRowsPrefix];
  __shared__ __attribute__((aligned(16))) float w_lds[DH];
  // each wave's 16 lambda values (through LDS: a register across the tile
  // loop would spill)
  __shared__ float lam_lds[NW * 16];
  // TB: cos / sin rows of the workgroup's queries, cos / sin of its heads'
  // noise angles.  NS 2: in the second V buffer (its first tile load goes
  // out after the barrier that follows every wave's table reads)
  constexpr bool TBS = TB && NS == 4;
  __shared__ __attribute__((aligned(16))) bf16_t tab_rope_s[TBS ? 2 : 1][TBS ? kTabRows * kTabPitch : 8];
  __shared__ __attribute__((aligned(16))) bf16_t tab_th_s[TBS ? 2 : 1][TBS ? 8 * (DH / 2) : 8];
  bf16_t* const tab_rope0 = TBS ? &tab_rope_s[0][0] : (bf16_t*)(f3_smem + f3_table_offset<DH>());
  bf16_t* const tab_rope1 = TBS ? &tab_rope_s[1][0] : tab_rope0 + kTabRows * kTabPitch;
  bf16_t* const tab_th0 = TBS ? &tab_th_s[0][0] : tab_rope0 + 2 * kTabRows * kTabPitch;
  bf16_t* const tab_th1 = TBS ? &tab_th_s[1][0] : tab_th0 + 8 * (DH / 2);

  const int id = blockIdx.x;
  int qb, pair;
  if (npairs % 8 == 0) {
    const int local = id >> 3;
    pair = (id & 7) + 8 * (local / nqb);
    qb = local % nqb;
  } else {
    pair = id / nqb;
    qb = id % nqb;
  }
  // causal: the q-blocks with the most keys go out first, so the last
  // workgroups of the launch are short ones
  if (a_.causal) qb = nqb - 1 - qb;
  const int hk = pair % a.Hkv, b = pair / a.Hkv;
  const int G = a.H / a.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hl = lane >> 5;
  const int strm = n >> 4, qn = n & 15;
  const int g = wv / NQ, qsub = wv % NQ, h = hk * G + g;
  const int q0 = qb * 16 * NQ + 16 * qsub;
  const int qrow = q0 + qn;
  const float scale = (a.sm_scale > 0.f ? a.sm_scale : rsqrtf((float)DH)) * kLog2e;
  const int Lk = a.Lp + a.Lb;
  const int coff = a.causal == 2 ? 0 : a.Lb - a.Lq;
  const int q_hi = min(a.Lq - 1, qb * 16 * NQ + 16 * NQ - 1);
  const int klim = a.causal ? min(Lk, a.Lp + q_hi + coff + 1) : Lk;
  const int ntile = (klim + KT - 1) / KT;

  const bf16_t* kpb = a.Lp > 0 ? (const bf16_t*)a.kp + b * a.p_sb + hk * a.p_sh : nullptr;
  const bf16_t* vpb = a.Lp > 0 ? (const bf16_t*)a.vp + b * a.p_sb + hk * a.p_sh : nullptr;
  const bf16_t* kbb = a.Lb > 0 ? (const bf16_t*)a.kb + b * a.b_sb + hk * a.b_sh : nullptr;
  const bf16_t* vbb = a.Lb > 0 ? (const bf16_t*)a.vb + b * a.b_sb + hk * a.b_sh : nullptr;
  const int psl = (int)a.p_sl, bsl = (int)a.b_sl;

  // ---- tile loads: K fragment ci = wv + NW j is (kb, ks) = (ci / NKS,
  // ci % NKS): key 32 kb + k_r, channels 16 ks + k_c; V piece vi = wv + NW j:
  // row RPI vi + v_r, the channels of its stored chunk.  Per-lane byte
  // offsets from the tile's first row (31 bits: checked by the launcher).
  const int k_r = lane & 31, k_c = 8 * (lane >> 5);
  const int v_r = lane / Lay::CPR, v_c = 8 * Lay::vchunk(v_r, lane % Lay::CPR);
  const uint32_t kofP = 2u * (uint32_t)(k_r * psl + k_c), kofB = 2u * (uint32_t)(k_r * bsl + k_c);
  const uint32_t vofP = 2u * (uint32_t)(v_r * psl + v_c), vofB = 2u * (uint32_t)(v_r * bsl + v_c);
  // K / V buffers of tile t
  auto kbuf = [&](int t) -> char* {
    return NS == 4 ? f3_smem + (t % 4) * STAGE : f3_smem + (t & 1) * Lay::KBYTES;
  };
  auto vbuf = [&](int t) -> char* {
    return NS == 4 ? f3_smem + (t % 4) * STAGE + Lay::KBYTES : f3_smem + 2 * Lay::KBYTES + (t & 1) * Lay::VBYTES;
  };
  // tile t's K (WK) and / or V (WV) pieces of this wave
  auto tile_part = [&](auto wk_c, auto wv_c, int t) {
    constexpr bool WK = decltype(wk_c)::value, WV = decltype(wv_c)::value;
    const int kt0 = t * KT;
    char* kd = kbuf(t);
    char* vd = vbuf(t);
    const bool in_p = kt0 + KT <= a.Lp, in_b = kt0 >= a.Lp && kt0 + KT <= Lk;
    if (in_p || in_b) {
      const char* kb0 = in_p ? (const char*)(kpb + (int64_t)kt0 * psl) : (const char*)(kbb + (int64_t)(kt0 - a.Lp) * bsl);
      const char* vb0 = in_p ? (const char*)(vpb + (int64_t)kt0 * psl) : (const char*)(vbb + (int64_t)(kt0 - a.Lp) * bsl);
      const int sl2 = 2 * (in_p ? psl : bsl);
      const uint32_t kof = in_p ? kofP : kofB, vof = in_p ? vofP : vofB;
      if constexpr (WK) {
#pragma unroll
        for (int j = 0; j < KCW; ++j) {
          const int ci = wv + NW * j, kb = ci / NKS, ks = ci % NKS;
          lds_load16(kb0 + (int64_t)(32 * kb) * sl2 + 32 * ks + kof, kd + ci * 1024);
        }
      }
      if constexpr (WV) {
#pragma unroll
        for (int j = 0; j < VCW; ++j) {
          const int vi = wv + NW * j;
          lds_load16(vb0 + (int64_t)(Lay::RPI * vi) * sl2 + vof, vd + vi * 1024);
        }
      }
    } else {
      // a tile across the prefix / block boundary or the end: per row
      // (rows past Lk read row 0, a valid row, and are masked)
      auto row_of = [&](const bf16_t* pb, const bf16_t* bb, int kidx) {
        kidx = kidx < Lk ? kidx : 0;
        return kidx < a.Lp ? pb + (int64_t)kidx * psl : bb + (int64_t)(kidx - a.Lp) * bsl;
      };
      if constexpr (WK) {
#pragma unroll
        for (int j = 0; j < KCW; ++j) {
          const int ci = wv + NW * j, kb = ci / NKS, ks = ci % NKS;
          lds_load16(row_of(kpb, kbb, kt0 + 32 * kb + k_r) + 16 * ks + k_c, kd + ci * 1024);
        }
      }
      if constexpr (WV) {
#pragma unroll
        for (int j = 0; j < VCW; ++j) {
          const int vi = wv + NW * j;
          lds_load16(row_of(vpb, vbb, kt0 + Lay::RPI * vi + v_r) + v_c, vd + vi * 1024);
        }
      }
    }
  };
  using TrueC = std::integral_constant<bool, true>;
  using FalseC = std::integral_constant<bool, false>;
  auto tile_load = [&](int t) { tile_part(TrueC{}, TrueC{}, t); };
  constexpr int LPT = KCW + VCW;  // direct loads per wave and tile

  // ---- prologue.  VMEM loads complete in issue order, so the loads the
  // query math waits for go out first and tiles 0, 1, 2 behind them.  The
  // compiler cannot tell which LDS bytes a direct global->LDS load writes,
  // so it makes any LDS access the kernel code issues after one wait for
  // all of them: the visibility bytes and the norm weight reach LDS before
  // the tile loads go out, and nothing between those loads and the first
  // product touches LDS but the hand-issued fragment reads.
  // Visibility bytes: every wave loads the prefix's bytes (16 a lane, up to
  // kMaxRowsPrefix), folds them into `allvis` (bit e: the 32 keys [32 e,
  // 32 e + 32) are all visible, a key past the prefix counting as hidden)
  // and wave 0 stores them to LDS for the per-entry mask.
  constexpr int ALC = kMaxRowsPrefix / (16 * 64);  // 16-byte chunks per lane
  uint4 al_c[ALC];
  bf16_t w_raw;
  uint64_t allvis = 0;
  // queries of this lane: row n (stream strm of query qrow), channels
  // 16 ks + 8 hl .. + 8: RoPE with the eager-op rounding, then for the noise
  // stream the per-head rotation (primitives.py:58-113), unless the noise
  // queries are given.  QM fixes the case at compile time (0: interleaved
  // RoPE + rotation, 1: half-split RoPE + rotation, 2: given noise queries,
  // no RoPE, 3: any, decided at run time), so the common cases are
  // straight-line code: every load unconditional and from a valid address
  // (the signal and noise lanes of a query read the same row in the same
  // instruction, one memory access), both streams' math on every lane and
  // a select, no wait inside a branch.
  bf16x8_t qf[NKS];
  bf16_t lam_raw;
  {
    using E = Elt<bf16_t>;
    constexpr int half = DH / 2;
    const bool noise = strm == 1;
    const bool given = QM == 2 || (QM == 3 && a.q_noise != nullptr);
    const bool rope = QM == 0 || QM == 1 || (QM == 3 && a.rope_cos != nullptr);
    const bool inter = QM == 0 || (QM == 3 && a.rope_interleaved != 0);
    const bool qlive = qrow < a.Lq;
    const int qi = qlive ? qrow : 0;
    const bf16_t* qrow_sig = (const bf16_t*)a.q + b * a.q_sb + h * a.q_sh + (int64_t)qi * a.q_sl;
    const bf16_t* qr = (given && noise)
                           ? (const bf16_t*)a.q_noise + b * a.qn_sb + h * a.qn_sh + (int64_t)qi * a.qn_sl
                           : qrow_sig;
    // RoPE applies to the query rows this lane loads unless they are given
    // noise queries (QM 3 with both)
    const bool rope_lane = rope && !(given && noise);
    const bf16_t* csr = rope ? (const bf16_t*)a.rope_cos + (int64_t)qi * half : nullptr;
    const bf16_t* snr = rope ? (const bf16_t*)a.rope_sin + (int64_t)qi * half : nullptr;
    const bf16_t* thc = !given ? (const bf16_t*)a.theta_cos + (int64_t)h * half : nullptr;
    const bf16_t* ths = !given ? (const bf16_t*)a.theta_sin + (int64_t)h * half : nullptr;
    // QM 0 / 1 (RoPE and the noise rotation): the signal and noise lanes of
    // a query split its channel steps, NOWN each (the signal lane the first
    // half, the noise lane the second), rope and rotate their own, and trade
    // with one permlane16 swap: the signal lane sends the rotated values the
    // noise lane needs and gets the roped values it needs
    constexpr bool SPLIT = QM == 0 || QM == 1;
    constexpr int NOWN = SPLIT ? NKS / 2 : NKS;
    const int ks_base = SPLIT ? NOWN * strm : 0;
    uint4 uq[NOWN], up[NOWN], rc[NOWN], rs[NOWN];
    uint2 rc2[NOWN], rs2[NOWN], tcs[NOWN], tsn[NOWN];
    // TB: the workgroup's RoPE rows (its 16 NQ queries) and noise angles
    // (its G heads) load once per workgroup, 16-byte pieces spread over the
    // threads, and reach the lanes through LDS: per-lane table loads were
    // most of the prologue's load instructions, and a CU's prologue is
    // bound by how many it can have in flight
    constexpr int TCH = half / 8;  // 16-byte pieces of a table row
    constexpr int TPT = (2 * kTabRows * TCH + 2 * 8 * TCH + NW * 64 - 1) / (NW * 64);
    uint4 tv[TPT];
    const int nrow = 16 * NQ, nrope = 2 * nrow * TCH, ntab = nrope + 2 * G * TCH;
    // piece c of a table: (which, row, 16-byte piece) by shifts (G and the
    // row count are powers of two here, TCH a power of two)
    static_assert((TCH & (TCH - 1)) == 0, "table pieces per row");
    constexpr int lg_tch = __builtin_ctz(TCH);
    const int lg_g = __builtin_ctz(G), lg_row = __builtin_ctz(nrow);
    if constexpr (TB) {
#pragma unroll
      for (int u = 0; u < TPT; ++u) {
        // (threads past the last piece reload it)
        const int c = min(tid + NW * 64 * u, ntab - 1);
        const bool th = c >= nrope;
        const int cc = th ? c - nrope : c;
        const int lgn = th ? lg_g : lg_row;
        const int which = cc >> (lgn + lg_tch), rr = (cc >> lg_tch) & ((1 << lgn) - 1), ch = cc & (TCH - 1);
        const bf16_t* src = th ? (const bf16_t*)(which ? a.theta_sin : a.theta_cos) + (int64_t)(hk * G + rr) * half + 8 * ch
                               : (const bf16_t*)(which ? a.rope_sin : a.rope_cos) +
                                     (int64_t)min(qb * 16 * NQ + rr, a.Lq - 1) * half + 8 * ch;
        tv[u] = NW * 64 * u < ntab ? *reinterpret_cast<const uint4*>(src) : uint4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < NOWN; ++u) {
      const int d0 = 16 * (ks_base + u) + 8 * hl;
      uq[u] = *reinterpret_cast<const uint4*>(qr + d0);
      if (rope && !inter) up[u] = *reinterpret_cast<const uint4*>(qr + (d0 < half ? d0 + half : d0 - half));
      if constexpr (!TB) {
        if (rope && inter) {
          rc2[u] = *reinterpret_cast<const uint2*>(csr + d0 / 2);
          rs2[u] = *reinterpret_cast<const uint2*>(snr + d0 / 2);
        }
        if (rope && !inter) {
          const int f0 = d0 < half ? d0 : d0 - half;
          rc[u] = *reinterpret_cast<const uint4*>(csr + f0);
          rs[u] = *reinterpret_cast<const uint4*>(snr + f0);
        }
        if (!given) {
          tcs[u] = *reinterpret_cast<const uint2*>(thc + d0 / 2);
          tsn[u] = *reinterpret_cast<const uint2*>(ths + d0 / 2);
        }
      }
    }
    lam_raw = ((const bf16_t*)a.lam)[b * a.lam_sb + h * a.lam_sh + (int64_t)qi * a.lam_sl];
    // visibility bytes of the prefix and the norm weight, behind the
    // queries (without visibility bytes, or past the row, a 16-byte read of
    // the queries keeps the load unconditional; its value is replaced)
    {
      const bool have = a.allowed != nullptr && (a.al_sb % 16) == 0 && ((uintptr_t)a.allowed % 16) == 0 &&
                        (a.Lp % 16) == 0;
      const uint8_t* alp = have ? a.allowed + (int64_t)b * a.al_sb : (const uint8_t*)a.q;
#pragma unroll
      for (int c = 0; c < ALC; ++c) {
        const int i0 = 16 * (lane + 64 * c);
        al_c[c] = *reinterpret_cast<const uint4*>(alp + (have && i0 + 16 <= a.Lp ? i0 : 0));
      }
      const bf16_t wl = (a.rms_w ? (const bf16_t*)a.rms_w : (const bf16_t*)a.q)[a.rms_w ? (tid & (DH - 1)) : 0];
      w_raw = a.rms_w ? wl : (bf16_t)0x3f80;
      const bool slow = a.allowed != nullptr && !have;
      if (slow) {
        // visibility bytes that are not 16-byte aligned: one load a byte
        // (their own branch, so the usual path has no load in it)
#pragma unroll
        for (int c = 0; c < ALC; ++c) {
          const int i0 = 16 * (lane + 64 * c);
          uint32_t wd[4] = {0, 0, 0, 0};
          for (int i = 0; i < 16; ++i)
            if (i0 + i < a.Lp) wd[i >> 2] |= (uint32_t)a.allowed[(int64_t)b * a.al_sb + i0 + i] << (8 * (i & 3));
          al_c[c] = uint4{wd[0], wd[1], wd[2], wd[3]};
        }
      }
#pragma unroll
      for (int c = 0; c < ALC; ++c) {
        const int i0 = 16 * (lane + 64 * c);
        // a prefix key is visible when its byte is nonzero (every prefix key
        // without visibility bytes; the per-entry mask reads bytes of keys
        // inside the prefix only); the chunk's 16 keys are all visible when
        // the chunk lies inside the prefix and has no zero byte (a word has
        // one exactly when (w - 0x01010101) & ~w & 0x80808080 is nonzero)
        const uint4 v = a.allowed == nullptr ? uint4{0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u} : al_c[c];
        al_c[c] = v;
        const uint32_t z = ((v.x - 0x01010101u) & ~v.x) | ((v.y - 0x01010101u) & ~v.y) |
                           ((v.z - 0x01010101u) & ~v.z) | ((v.w - 0x01010101u) & ~v.w);
        const bool all16 = i0 + 16 <= a.Lp && (z & 0x80808080u) == 0u;
        // 16-byte chunk k of this group is lane k: block e of the group is
        // chunks 2e, 2e + 1, so bit e of the group's 32 is (bit 2e & bit
        // 2e + 1) of the ballot, gathered from the even bits
        uint64_t x = __ballot(all16);
        x &= x >> 1;
        x &= 0x5555555555555555ull;
        x = (x | (x >> 1)) & 0x3333333333333333ull;
        x = (x | (x >> 2)) & 0x0f0f0f0f0f0f0f0full;
        x = (x | (x >> 4)) & 0x00ff00ff00ff00ffull;
        x = (x | (x >> 8)) & 0x0000ffff0000ffffull;
        x = (x | (x >> 16)) & 0x00000000ffffffffull;
        allvis |= x << (32 * c);
      }
      if (wv == 0) {
#pragma unroll
        for (int c = 0; c < ALC; ++c) {
          const int i0 = 16 * (lane + 64 * c);
          if (i0 < a.Lp) *reinterpret_cast<uint4*>(al_lds + i0) = al_c[c];
        }
      }
      if (tid < DH) w_lds[tid] = bf2f(w_raw);
      if (lane < 16) lam_lds[wv * 16 + lane] = bf2f(lam_raw);
    }
    if constexpr (TB) {
      // tables to LDS (rows padded by 16 bytes, so the 16 query rows of a
      // wave's reads spread over the banks), then each lane reads its
      // entries, before any direct global->LDS load is in flight
#pragma unroll
      for (int u = 0; u < TPT; ++u) {
        const int c = tid + NW * 64 * u;
        if (c < ntab) {
          const bool th = c >= nrope;
          const int cc = th ? c - nrope : c;
          const int lgn = th ? lg_g : lg_row;
          const int which = cc >> (lgn + lg_tch), rr = (cc >> lg_tch) & ((1 << lgn) - 1), ch = cc & (TCH - 1);
          bf16_t* dst = th ? (which ? tab_th1 : tab_th0) + rr * half + 8 * ch
                           : (which ? tab_rope1 : tab_rope0) + rr * kTabPitch + 8 * ch;
          *reinterpret_cast<uint4*>(dst) = tv[u];
        }
      }
      __syncthreads();
      const int rl = 16 * qsub + qn;
#pragma unroll
      for (int u = 0; u < NOWN; ++u) {
        const int d0 = 16 * (ks_base + u) + 8 * hl;
        if (inter) {
          rc2[u] = *reinterpret_cast<const uint2*>(tab_rope0 + rl * kTabPitch + d0 / 2);
          rs2[u] = *reinterpret_cast<const uint2*>(tab_rope1 + rl * kTabPitch + d0 / 2);
        } else {
          const int f0 = d0 < half ? d0 : d0 - half;
          rc[u] = *reinterpret_cast<const uint4*>(tab_rope0 + rl * kTabPitch + f0);
          rs[u] = *reinterpret_cast<const uint4*>(tab_rope1 + rl * kTabPitch + f0);
        }
        tcs[u] = *reinterpret_cast<const uint2*>(tab_th0 + g * half + d0 / 2);
        tsn[u] = *reinterpret_cast<const uint2*>(tab_th1 + g * half + d0 / 2);
      }
    }
    // tiles 0 .. NS-2 behind everything else (NS 2: K(0), K(1), V(0))
    if constexpr (NS == 4) {
#pragma unroll
      for (int t = 0; t < NS - 1; ++t)
        if (t < ntile) tile_load(t);
    } else {
      if (ntile > 0) tile_part(TrueC{}, FalseC{}, 0);
      if (ntile > 1) tile_part(TrueC{}, FalseC{}, 1);
      if (ntile > 0) tile_part(FalseC{}, TrueC{}, 0);
    }
#pragma unroll
    for (int u = 0; u < NOWN; ++u) {
      const int d0 = 16 * (ks_base + u) + 8 * hl;
      uint32_t w[4] = {uq[u].x, uq[u].y, uq[u].z, uq[u].w};
      if (rope && inter) {
        // pairs (2p, 2p+1) rotated by angle d0/2 + p: one bf16 dot2 per
        // output (fp32 products and sum, one rounding)
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t r = rot_pair(w[pp], pp >> 1 ? rc2[u].y : rc2[u].x, pp >> 1 ? rs2[u].y : rs2[u].x, pp & 1);
          w[pp] = rope_lane ? r : w[pp];
        }
      }
      if (rope && !inter) {
        // half-split pairs (d, d +- Dh/2): x cos + rotate_half(x) sin
        float x[8], cc[8], ss[8], y[8];
        unpack8(uq[u], x);
        unpack8(rc[u], cc);
        unpack8(rs[u], ss);
        unpack8(up[u], y);
        const bool lo = d0 < half;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float rt = lo ? -y[j] : y[j];
          x[j] = E::rnd(E::rnd(x[j] * cc[j]) + E::rnd(rt * ss[j]));
        }
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) w[pp] = rope_lane ? pk_bf16(x[2 * pp], x[2 * pp + 1]) : w[pp];
      }
      if constexpr (SPLIT) {
        // this lane's roped values (r) and their rotation (t); the swap
        // leaves the signal lane r of step u and r of step u + NOWN (its
        // partner's), the noise lane t of step u (its partner's) and t of
        // step u + NOWN
        uint32_t lo4[4], hi4[4];
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t t = rot_pair(w[pp], pp >> 1 ? tcs[u].y : tcs[u].x, pp >> 1 ? tsn[u].y : tsn[u].x, pp & 1);
          const auto sw = __builtin_amdgcn_permlane16_swap(w[pp], t, false, false);
          lo4[pp] = (uint32_t)sw[0];
          hi4[pp] = (uint32_t)sw[1];
        }
        // (a row past Lq read row 0: finite values, and its output is not
        // stored)
        qf[u] = __builtin_bit_cast(bf16x8_t, uint4{lo4[0], lo4[1], lo4[2], lo4[3]});
        qf[u + NOWN] = __builtin_bit_cast(bf16x8_t, uint4{hi4[0], hi4[1], hi4[2], hi4[3]});
      } else {
        if (!given) {
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) {
            const uint32_t r = rot_pair(w[pp], pp >> 1 ? tcs[u].y : tcs[u].x, pp >> 1 ? tsn[u].y : tsn[u].x, pp & 1);
            w[pp] = noise ? r : w[pp];
          }
        }
        qf[u] = __builtin_bit_cast(bf16x8_t, qlive ? uint4{w[0], w[1], w[2], w[3]} : uint4{0, 0, 0, 0});
      }
    }
  }

  // V transposed-read cells: for each channel block db, rows 4 hl +
  // (p16 >> 2) of a 16-key step, channels 32 db + 16 (grp & 1) + 4 (p16 &
  // 3), stored chunk swizzled (F2Layout::vchunk)
  const int grp = lane >> 4, p16 = lane & 15;
  const int vrow = 4 * (grp >> 1) + (p16 >> 2);
  int v_off[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    v_off[db] = vrow * Lay::ROWB + 16 * Lay::vchunk(vrow, 4 * db + 2 * (grp & 1) + ((p16 & 3) >> 1)) + 8 * (p16 & 1);
  // key kt0 + 32 kb + kk(j) of register j; a block key is visible while
  // kidx <= thr (causal / end), a prefix key when its byte is set
  const int thr = min(Lk - 1, a.causal ? a.Lp + qrow + coff : Lk - 1);
  auto kk = [](int j) { return 8 * (j >> 2) + (j & 3); };

  float m_s = -INFINITY, l_s = 0.f;
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16{};

  f32x16 st[2][2];  // S of two tiles: [parity][key block]
  // per-entry masking a tile needs: 1 = the end / causal threshold only,
  // 2 = also hidden prefix slots (visibility bytes), 0 = none
  auto tile_mask_mode = [&](int kt0) {
    const bool thr_m = kt0 + KT > Lk || (a.causal && kt0 + KT - 1 > a.Lp + q0 + coff);
    bool al_m = false;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int pk0 = kt0 + 32 * kb;
      al_m |= pk0 < a.Lp && !((allvis >> (pk0 >> 5)) & 1);
    }
    return al_m ? 2 : thr_m ? 1 : 0;
  };
  // (branch-free: every lane reads a byte of the LDS copy, a valid one
  // past the prefix, and selects)
  auto mask_entry = [&](float v, int kt0, int kb, int j, auto mode_c) {
    const int kidx = kt0 + 32 * kb + 4 * hl + kk(j);
    const int thr_ok = kidx <= thr;
    if constexpr (decltype(mode_c)::value == 1) {
      return thr_ok ? v : -INFINITY;
    } else {
      const int byte = al_lds[min(kidx, kMaxRowsPrefix - 1)];
      const int pre = kidx < a.Lp;
      return ((pre & (byte != 0)) | ((pre ^ 1) & thr_ok)) ? v : -INFINITY;
    }
  };
  // a tile's mask in place, one straight-line loop per mode
  auto mask_tile = [&](auto par_c, int kt0, int mode) {
    constexpr int P = decltype(par_c)::value;
    if (mode == 1) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) st[P][kb][j] = mask_entry(st[P][kb][j], kt0, kb, j, std::integral_constant<int, 1>{});
    } else if (mode == 2) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) st[P][kb][j] = mask_entry(st[P][kb][j], kt0, kb, j, std::integral_constant<int, 2>{});
    }
  };
  // running-max update from a tile's masked scores (lanes l and l ^ 32
  // share a row), with the lazy rescale of O and the row sum
  auto fold_max = [&](float mx) {
    const float tsc = xmax32(mx) * scale;
    if (__ballot(tsc > m_s + 8.f)) {
      const float mnew = fmaxf(m_s, tsc);
      const float alpha = mnew == -INFINITY ? 1.f : fast_exp2(m_s - mnew);
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] *= alpha;
      l_s *= alpha;
      m_s = mnew;
    }
  };

  // ---- S(0), masked, max folded
  if (ntile > 0) {
    if constexpr (NS == 4)
      vm_wait(LPT * (min(ntile, NS - 1) - 1));
    else
      vm_wait(ntile > 1 ? KCW + VCW : VCW);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    const uint32_t ka = lds_addr(f3_smem) + 16 * lane;
    u32x4v_t kr[4];
    auto k_issue = [&](auto f_c) {
      constexpr int f = decltype(f_c)::value;
      if constexpr (f < 2 * NKS) kr[f % 4] = lds_read_b128_at<((f % 2) * NKS + f / 2) * 1024>(ka);
    };
    k_issue(std::integral_constant<int, 0>{});
    k_issue(std::integral_constant<int, 1>{});
    k_issue(std::integral_constant<int, 2>{});
    static_for<2 * NKS>([&](auto f_c) {
      constexpr int f = decltype(f_c)::value, ks = f / 2, kb = f % 2;
      k_issue(std::integral_constant<int, f + 3>{});
      lds_wait_b128<(f + 3 < 2 * NKS) ? 3 : (2 * NKS - 1 - f)>(kr[f % 4]);
      st[0][kb] = mfma_32x32x16(__builtin_bit_cast(bf16x8_t, kr[f % 4]), qf[ks], ks == 0 ? f32x16{} : st[0][kb]);
      __builtin_amdgcn_sched_barrier(0);
    });
    mask_tile(std::integral_constant<int, 0>{}, 0, tile_mask_mode(0));
    float mx = st[0][0][0];
#pragma unroll
    for (int j = 1; j < 16; ++j) mx = fmaxf(mx, st[0][0][j]);
#pragma unroll
    for (int j = 0; j < 16; ++j) mx = fmaxf(mx, st[0][1][j]);
    fold_max(mx);
  }

  // one pipelined iteration; PAR = it % 2 selects the S registers
  auto iteration = [&](auto par_c, int it) {
    constexpr int PAR = decltype(par_c)::value, NXT = 1 - PAR;
    const bool has_next = it + 1 < ntile;
    const int kt0 = it * KT, kt1 = kt0 + KT;
    // tile it + 1 has landed and every wave has finished iteration it - 1
    // (so tile it - 1's buffer may take tile it + 2)
    if constexpr (NS == 4) {
      if (has_next) {
        vm_wait(it + 2 < ntile ? LPT : 0);
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_s_barrier();
        if (it + 3 < ntile) tile_load(it + 3);
      }
    } else {
      // K(it + 1) and V(it), the only loads in flight, have landed and every
      // wave has finished iteration it - 1 (so K(it)'s buffer may take
      // K(it + 2) and V(it - 1)'s V(it + 1))
      vm_wait(0);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_s_barrier();
      if (it + 2 < ntile) tile_part(TrueC{}, FalseC{}, it + 2);
      if (has_next) tile_part(FalseC{}, TrueC{}, it + 1);
    }
    const float mu = m_s == -INFINITY ? 0.f : m_s;
    uint32_t pw[16];  // P(it) as bf16 pairs: word e / 2 holds entries e, e + 1 (e = 16 kb + j)
    float ls = 0.f;
    auto p_pair = [&](int e) {
      const int kb = e >> 4, j = e & 15;
      const float p0 = fast_exp2(fmaf(st[PAR][kb][j], scale, -mu));
      const float p1 = fast_exp2(fmaf(st[PAR][kb][j + 1], scale, -mu));
      pw[e >> 1] = pk_bf16(p0, p1);
      // (plain adds: a dot2 does not issue beside a running product)
      ls += p0 + p1;
    };
    // ---- phase A: S(it + 1) products, each with one pair of P(it).  Wave
    // priorities: phase A 1, phase C 2, everything else 0, so that where
    // two waves share a SIMD the one in its product-heavy phase issues its
    // products first and the other fills the vector pipe (measured: 2-4%)
    __builtin_amdgcn_s_setprio(1);
    if (has_next) {
      const uint32_t ka = lds_addr(kbuf(it + 1)) + 16 * lane;
      u32x4v_t kr[4];
      auto k_issue = [&](auto f_c) {
        constexpr int f = decltype(f_c)::value;
        if constexpr (f < 2 * NKS) kr[f % 4] = lds_read_b128_at<((f % 2) * NKS + f / 2) * 1024>(ka);
      };
      k_issue(std::integral_constant<int, 0>{});
      k_issue(std::integral_constant<int, 1>{});
      k_issue(std::integral_constant<int, 2>{});
      static_for<2 * NKS>([&](auto f_c) {
        constexpr int f = decltype(f_c)::value, ks = f / 2, kb = f % 2;
        k_issue(std::integral_constant<int, f + 3>{});
        lds_wait_b128<(f + 3 < 2 * NKS) ? 3 : (2 * NKS - 1 - f)>(kr[f % 4]);
        st[NXT][kb] = mfma_32x32x16(__builtin_bit_cast(bf16x8_t, kr[f % 4]), qf[ks], ks == 0 ? f32x16{} : st[NXT][kb]);
        if constexpr (2 * f < 32) p_pair(2 * f);
        if constexpr (2 * NKS == 8 && 2 * f + 16 < 32) p_pair(2 * f + 16);  // head_dim 64: two pairs a product
        __builtin_amdgcn_sched_barrier(0);
      });
    } else {
#pragma unroll
      for (int e = 0; e < 32; e += 2) p_pair(e);
    }
    l_s += ls;
    // ---- S(it + 1)'s mask, where the tile needs one (rare: the tile on the
    // causal diagonal, the end, hidden prefix slots)
    if (has_next) mask_tile(std::integral_constant<int, NXT>{}, kt1, tile_mask_mode(kt1));
    // ---- phase C: O += V(it)^T P(it), each product with the running max
    // of two entries of S(it + 1) (four at head_dim 64; a stale S when
    // there is no next tile, whose max is then dropped)
    float mx = -INFINITY;
    __builtin_amdgcn_s_setprio(2);
    {
      const uint32_t va = lds_addr(vbuf(it));
      constexpr int NPV = 4 * NDB;
      uint2 rd[3][2];
      auto v_issue = [&](auto q_c) {
        constexpr int q = decltype(q_c)::value;
        if constexpr (q < NPV) {
          constexpr int p = q / NDB, db = q % NDB;
          constexpr int ROW0 = 16 * p * Lay::ROWB, ROW8 = ROW0 + 8 * Lay::ROWB;
          rd[q % 3][0] = lds_read_tr16_at<ROW0>(va + v_off[db]);
          rd[q % 3][1] = lds_read_tr16_at<ROW8>(va + v_off[db]);
        }
      };
      v_issue(std::integral_constant<int, 0>{});
      v_issue(std::integral_constant<int, 1>{});
      static_for<NPV>([&](auto q_c) {
        constexpr int q = decltype(q_c)::value;
        constexpr int p = q / NDB, db = q % NDB, b3 = q % 3;
        lds_wait2_n<(q + 1 < NPV) ? 2 : 0>(rd[b3][0], rd[b3][1]);
        const bf16x8_t va8 = __builtin_bit_cast(bf16x8_t, uint4{rd[b3][0].x, rd[b3][0].y, rd[b3][1].x, rd[b3][1].y});
        const uint4 pf = uint4{pw[4 * p], pw[4 * p + 1], pw[4 * p + 2], pw[4 * p + 3]};
        o[db] = mfma_32x32x16(va8, __builtin_bit_cast(bf16x8_t, pf), o[db]);
        constexpr int PER = 32 / NPV;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          constexpr int e0 = PER * q;
          mx = fmaxf(mx, st[NXT][(e0 + u) >> 4][(e0 + u) & 15]);
        }
        __builtin_amdgcn_sched_barrier(0);
        v_issue(std::integral_constant<int, q + 2>{});
        __builtin_amdgcn_sched_barrier(0);
      });
    }
    __builtin_amdgcn_s_setprio(0);
    if (has_next) fold_max(mx);
  };
  for (int it = 0; it < ntile; it += 2) {
    iteration(std::integral_constant<int, 0>{}, it);
    if (it + 1 < ntile) iteration(std::integral_constant<int, 1>{}, it + 1);
  }

  // ---- epilogue: lane holds row n's channels 32 db + 8 (j / 4) + 4 hl +
  // j % 4.  Noise lanes (n >= 16) round O_noise to bf16; one permlane swap
  // hands it to the signal lane l ^ 16; y = O_signal - lam rnd(O_noise),
  // then the HeadwiseRMSNorm and weight in fp32, one rounding at the store.
  const float l_tot = xsum32(l_s);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float lam = lam_lds[wv * 16 + qn];
  float y[NDB][16];
  float sq = 0.f;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      const uint32_t mine = pk_bf16(o[db][j] * inv, o[db][j + 1] * inv);
      const auto r = __builtin_amdgcn_permlane16_swap(mine, mine, false, false);
      const uint32_t nz = (uint32_t)r[1];
      const float on0 = bf2f((bf16_t)(nz & 0xffffu)), on1 = bf2f((bf16_t)(nz >> 16));
      y[db][j] = fmaf(-lam, on0, o[db][j] * inv);
      y[db][j + 1] = fmaf(-lam, on1, o[db][j + 1] * inv);
      sq = fmaf(y[db][j], y[db][j], sq);
      sq = fmaf(y[db][j + 1], y[db][j + 1], sq);
    }
  if (a.rms_w) {
    sq = xsum32(sq);
    const float rr = 1.0f / sqrtf(sq / (float)DH + a.eps);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const float4 wv4 = *reinterpret_cast<const float4*>(w_lds + 32 * db + 8 * jq + 4 * hl);
        y[db][4 * jq + 0] *= rr * wv4.x;
        y[db][4 * jq + 1] *= rr * wv4.y;
        y[db][4 * jq + 2] *= rr * wv4.z;
        y[db][4 * jq + 3] *= rr * wv4.w;
      }
  }
  if (strm == 0 && qrow < a.Lq) {
    bf16_t* orow_p = (bf16_t*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)qrow * a.o_sl;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        uint2 u;
        u.x = pk_bf16(y[db][4 * jq + 0], y[db][4 * jq + 1]);
        u.y = pk_bf16(y[db][4 * jq + 2], y[db][4 * jq + 3]);
        *reinterpret_cast<uint2*>(orow_p + 32 * db + 8 * jq + 4 * hl) = u;
      }
  }
}

// ------------------------------------------------------------ host side
static int rows_nsplit(const coda_attn_desc* d) {
  const int Lk = d->Lp + d->Lb;
  const int pairs = d->B * d->Hkv;
  if (pairs >= 512) return 1;
  int ns = (512 + pairs - 1) / pairs;
  const int max_ns = (Lk + 63) / 64;
  ns = ns < max_ns ? ns : max_ns;
  return ns < 1 ? 1 : ns;
}

static bool use_rows(const coda_attn_desc* d) {
  return d->dtype == CODA_BF16 && 2 * (d->H / d->Hkv) * d->Lq <= 16;
}

static int validate(const coda_attn_desc* d) {
  CODA_REQUIRE(d != nullptr, "coda_diff_attn_fwd: null descriptor");
  CODA_REQUIRE(d->dtype == CODA_F32 || d->dtype == CODA_BF16,
               "coda_diff_attn_fwd: dtype must be CODA_F32 or CODA_BF16 (got %d)", d->dtype);
  CODA_REQUIRE(d->B >= 0 && d->H > 0 && d->Hkv > 0 && d->Lq >= 0,
               "coda_diff_attn_fwd: bad sizes B=%d H=%d Hkv=%d Lq=%d", d->B, d->H, d->Hkv, d->Lq);
  CODA_REQUIRE(d->H % d->Hkv == 0, "coda_diff_attn_fwd: H=%d not a multiple of Hkv=%d", d->H, d->Hkv);
  CODA_REQUIRE(d->Dh == 32 || d->Dh == 64 || d->Dh == 128,
               "coda_diff_attn_fwd: head_dim %d unsupported (32, 64, 128)", d->Dh);
  const int G = d->H / d->Hkv;
  CODA_REQUIRE(G <= 8, "coda_diff_attn_fwd: %d query heads per KV head unsupported (max 8)", G);
  CODA_REQUIRE(d->Lp >= 0 && d->Lb >= 0, "coda_diff_attn_fwd: negative key count");
  CODA_REQUIRE(d->Lp == 0 || (d->kp && d->vp), "coda_diff_attn_fwd: prefix keys missing");
  CODA_REQUIRE(d->Lb == 0 || (d->kb && d->vb), "coda_diff_attn_fwd: block keys missing");
  CODA_REQUIRE(d->causal >= 0 && d->causal <= 2, "coda_diff_attn_fwd: causal mode %d unknown", d->causal);
  CODA_REQUIRE(d->causal != 1 || d->Lb >= d->Lq || d->Lb == 0,
               "coda_diff_attn_fwd: lower-right causal block needs Lb >= Lq (Lb=%d Lq=%d)", d->Lb, d->Lq);
  CODA_REQUIRE(d->q && d->lam && d->out, "coda_diff_attn_fwd: q, lam, out are required");
  CODA_REQUIRE(d->q_noise || (d->theta_cos && d->theta_sin),
               "coda_diff_attn_fwd: need q_noise or theta tables");
  CODA_REQUIRE(!d->rope_cos == !d->rope_sin, "coda_diff_attn_fwd: rope_cos/rope_sin come in pairs");
  CODA_REQUIRE(d->Lp + d->Lb < (1 << 30), "coda_diff_attn_fwd: too many keys");
  CODA_REQUIRE(d->Lp <= kMaxRowsPrefix, "coda_diff_attn_fwd: prefix of %d slots (max %d)", d->Lp,
               kMaxRowsPrefix);
  return CODA_OK;
}

}  // namespace coda

using namespace coda;

extern "C" int coda_attn_workspace_bytes(const coda_attn_desc* d, size_t* bytes) {
  int rc = validate(d);
  if (rc) return rc;
  CODA_REQUIRE(bytes != nullptr, "coda_attn_workspace_bytes: null out pointer");
  *bytes = 0;
  if (use_rows(d)) {
    const int ns = rows_nsplit(d);
    if (ns > 1) *bytes = (size_t)d->B * d->Hkv * ns * 16 * (d->Dh + 2) * sizeof(float);
  }
  return CODA_OK;
}

// the flash kernel's per-lane load offsets are 31-bit byte counts from a
// tile's first row (or from the prefix / block start on a boundary tile)
static bool flash_offsets_fit(const coda_attn_desc* d) {
  const int64_t lim = (int64_t)1 << 30;  // elements
  return (d->Lp == 0 || (d->p_sl >= 0 && ((int64_t)d->Lp + 64) * d->p_sl < lim)) &&
         (d->Lb == 0 || (d->b_sl >= 0 && ((int64_t)d->Lb + 64) * d->b_sl < lim));
}

// pipelined 32-row flash tiles: NW waves, G heads x NW / G groups of 16
// queries, NS tile stages; QM the query case (see attn_f3_bf16)
template <int DH, int QM, bool TB, int NW, int NS>
static int launch_f3_nw(const coda_attn_desc* d, hipStream_t st, int G, const ChunkGeom& cg) {
  const int npairs = d->B * d->Hkv;
  const int NQ = NW / G;
  const int nblk = (d->Lq + 16 * NQ - 1) / (16 * NQ);
  const size_t lds = f3_lds_bytes<DH, NS>();
  int rc = lds_limit<attn_f3_bf16<DH, NW, QM, TB, NS>>(lds, "coda_diff_attn_fwd");
  if (rc) return rc;
  hipLaunchKernelGGL((attn_f3_bf16<DH, NW, QM, TB, NS>), dim3(nblk * npairs, cg.n > 0 ? cg.n : 1), dim3(NW * 64),
                     lds, st, *d, NQ, nblk, npairs, cg);
  return check_launch("attn_f3_bf16");
}
// compute units of the current device (read once per device)
static int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}
// 4-wave workgroups with two tile stages (two a CU) for G <= 4 (a 4-wave
// workgroup still holds every head of its KV head), except a one-launch grid
// whose 8-wave workgroups fill the CUs once (at least one a CU, fewer than
// two): it keeps 8 waves and four stages, whose deeper prefetch serves a
// grid that starts all at once (measured: a block-256 chunk at B = 4, 36 vs
// 38 us; 4 waves win for grouped launches, small grids and configs[3]'s
// 4096 workgroups)
template <int DH, int QM, bool TB>
static int launch_f3_qm(const coda_attn_desc* d, hipStream_t st, int G, const ChunkGeom& cg) {
  if (G <= 4) {
    const int64_t rows8 = 16 * (8 / G);
    const int64_t n8 = (d->Lq + rows8 - 1) / rows8 * d->B * d->Hkv * (cg.n > 0 ? cg.n : 1);
    const int64_t cus = device_cus();
    if (cg.n > 1 || n8 < cus || n8 >= 2 * cus) return launch_f3_nw<DH, QM, TB, 4, 2>(d, st, G, cg);
  }
  return launch_f3_nw<DH, QM, TB, 8, 4>(d, st, G, cg);
}
template <int DH>
static int launch_f3(const coda_attn_desc* d, hipStream_t st, int G, const ChunkGeom& cg = ChunkGeom{}) {
  // the RoPE + rotation cases stage their tables in LDS while the
  // workgroup's 16 * 8 / G query rows fit (G >= 2)
  const bool tb = 16 * (8 / G) <= kTabRows && G <= 8;
  if (!d->q_noise && d->rope_cos) {
    if (d->rope_interleaved)
      return tb ? launch_f3_qm<DH, 0, true>(d, st, G, cg) : launch_f3_qm<DH, 0, false>(d, st, G, cg);
    return tb ? launch_f3_qm<DH, 1, true>(d, st, G, cg) : launch_f3_qm<DH, 1, false>(d, st, G, cg);
  }
  if (d->q_noise && !d->rope_cos) return launch_f3_qm<DH, 2, false>(d, st, G, cg);
  return launch_f3_qm<DH, 3, false>(d, st, G, cg);
}
template <int DH>
static int launch_attn(const coda_attn_desc* d, hipStream_t st) {
  const int G = d->H / d->Hkv;
  if (d->dtype == CODA_F32) {
    hipLaunchKernelGGL((attn_generic<float, DH>), dim3(d->Lq, d->Hkv, d->B), dim3(256), 0, st, *d);
    return check_launch("attn_generic<f32>");
  }
  if (use_rows(d)) {
    const int ns = rows_nsplit(d);
    const int Lk = d->Lp + d->Lb;
    int per = ((Lk + ns - 1) / ns + 15) / 16 * 16;
    if (per < 16) per = 16;
    const int ns_eff = Lk > 0 ? (Lk + per - 1) / per : 1;
    if (ns_eff > 1) {
      size_t need = (size_t)d->B * d->Hkv * ns_eff * 16 * (d->Dh + 2) * sizeof(float);
      if (!d->workspace || d->workspace_bytes < need)
        return fail(CODA_ESMALL, "coda_diff_attn_fwd: workspace %zu < %zu bytes", d->workspace_bytes, need);
    }
    hipLaunchKernelGGL((attn_rows_bf16<DH>), dim3(ns_eff > 0 ? ns_eff : 1, d->Hkv, d->B), dim3(256), 0, st, *d, per,
                       (float*)d->workspace);
    int rc = check_launch("attn_rows_bf16");
    if (rc || ns_eff <= 1) return rc;
    hipLaunchKernelGGL((attn_rows_merge<DH>), dim3(d->Hkv, d->B), dim3(256), 0, st, *d, ns_eff,
                       (const float*)d->workspace);
    return check_launch("attn_rows_merge");
  }
  if constexpr (DH >= 64) {
    if ((G == 8 || G == 4 || G == 2 || G == 1) && flash_offsets_fit(d)) return launch_f3<DH>(d, st, G);
  }
  const int NQ = G >= 4 ? 1 : 4 / G;
  const int nblk = (d->Lq + 16 * NQ - 1) / (16 * NQ);
  if (G == 8) {
    hipLaunchKernelGGL((attn_tile_bf16<DH, 8>), dim3(nblk, d->Hkv, d->B), dim3(512), 0, st, *d, NQ);
  } else if (G == 4 || G == 2 || G == 1) {
    hipLaunchKernelGGL((attn_tile_bf16<DH, 4>), dim3(nblk, d->Hkv, d->B), dim3(256), 0, st, *d, NQ);
  } else {
    return fail(CODA_EUNSUP, "coda_diff_attn_fwd: G=%d with Lq=%d unsupported for bf16 tiles", G, d->Lq);
  }
  return check_launch("attn_tile_bf16");
}

extern "C" int coda_prefill_attn_chunks(const coda_attn_desc* d, int n_chunks, int c_first, int blk, int L, int W,
                                        int64_t snap_stride, int64_t al_stride, void* stream) {
  CODA_REQUIRE(d != nullptr, "coda_prefill_attn_chunks: null descriptor");
  CODA_REQUIRE(n_chunks > 0 && c_first >= 0 && blk > 0 && W >= 0 && L > (int64_t)(c_first + n_chunks - 1) * blk,
               "coda_prefill_attn_chunks: chunks %d .. %d of %d tokens in blocks of %d", c_first,
               c_first + n_chunks - 1, L, blk);
  // the descriptor as for the widest chunk (a full block behind a full
  // window): every chunk's view lies within it
  coda_attn_desc w = *d;
  w.Lq = blk < L ? blk : L;
  w.Lb = W + w.Lq;
  int rc = validate(&w);
  if (rc) return rc;
  const int G = w.H / w.Hkv;
  CODA_REQUIRE(w.dtype == CODA_BF16 && w.Dh >= 64 && (G == 8 || G == 4 || G == 2 || G == 1) && w.causal == 1 &&
                   !use_rows(&w) && flash_offsets_fit(&w) && !w.q_noise && w.rope_cos,
               "coda_prefill_attn_chunks: needs bf16, head_dim >= 64, G in {1, 2, 4, 8}, the lower-right causal "
               "block, queries roped in-kernel and more than one query row per block");
  CODA_REQUIRE(snap_stride >= 0 && al_stride >= 0, "coda_prefill_attn_chunks: negative snapshot stride");
  if (w.B == 0) return CODA_OK;
  ChunkGeom cg{n_chunks, c_first, blk, L, W, 0, snap_stride, al_stride};
  hipStream_t st = (hipStream_t)stream;
  return w.Dh == 64 ? launch_f3<64>(&w, st, G, cg) : launch_f3<128>(&w, st, G, cg);
}

extern "C" int coda_diff_attn_fwd(const coda_attn_desc* d, void* stream) {
  int rc = validate(d);
  if (rc) return rc;
  if (d->B == 0 || d->Lq == 0) return CODA_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (d->Dh) {
    case 32: return launch_attn<32>(d, st);
    case 64: return launch_attn<64>(d, st);
    default: return launch_attn<128>(d, st);
  }
}

// ------------------------------------------------------------ decode step
// Full ring (the steady state): the bank update runs from a routing record
// (decode_bank_kernel, one workgroup per (head, sequence)), which also
// writes the record of the next token, then the attention kernel reads the
// updated cache.  The workspace holds two records, picked by the parity of
// the token position, followed by the attention kernel's scratch.
static bool step_routed(const coda_bank_desc* s, int ring_filled) {
  return ring_filled >= s->W && (s->Me > 0 || s->Ms > 0);
}

// bytes of one routing record (all sequences), 256-byte aligned
static size_t route_record_bytes(const coda_bank_desc* s) {
  return (sizeof(float) * (size_t)s->B * dstep_words(s->Hkv, s->Me, s->Ms) + 255) & ~(size_t)255;
}

static int validate_step(const coda_bank_desc* s, const coda_attn_desc* a) {
  int rc = validate(a);
  if (rc) return rc;
  CODA_REQUIRE(s != nullptr, "coda_decode_step: null state descriptor");
  const int Lbuf = s->W + s->Me + s->Ms;
  CODA_REQUIRE(a->dtype == s->dtype && a->B == s->B && a->Hkv == s->Hkv && a->Dh == s->Dh,
               "coda_decode_step: attention and state descriptors disagree (dtype/B/Hkv/Dh)");
  CODA_REQUIRE(a->Lq == 1 && a->Lb == 0 && a->Lp == Lbuf && a->kp == s->k_buf && a->vp == s->v_buf,
               "coda_decode_step: attention must read one query over the state cache (Lq=1, Lb=0, Lp=Lbuf)");
  CODA_REQUIRE(a->p_sl == s->Dh && a->p_sh == (int64_t)Lbuf * s->Dh && a->p_sb == (int64_t)s->Hkv * Lbuf * s->Dh,
               "coda_decode_step: state cache must be contiguous (B, Hkv, Lbuf, Dh)");
  return CODA_OK;
}

// the fused decode step kernel: bf16, a full ring, every row of a head's
// plane in the LDS visibility copy, all query rows in one MFMA tile
// CODA_DECODE_FUSED=0 sends every decode step through the bank kernel +
// split attention launches (read at every call, so that one process can
// compare the two paths)
static bool fused_step_enabled() {
  const char* e = getenv("CODA_DECODE_FUSED");
  return !(e && e[0] == '0');
}
static bool fused_step_ok(const coda_bank_desc* s, const coda_attn_desc* a) {
  const int G = a->H / a->Hkv;
  return fused_step_enabled() && s->dtype == CODA_BF16 && (s->Dh == 64 || s->Dh == 128) && 2 * G <= 16 && s->W >= 16 &&
         s->Me + s->Ms <= kFusedMaxBank && s->W + s->Me + s->Ms <= kMaxRowsPrefix && 2 * s->lf == s->Dh &&
         a->causal == 0 && a->allowed != nullptr;
}

template <int DH>
static int launch_fused_step(const coda_bank_desc* s, const coda_attn_desc* a, const void* k_new, const void* v_new,
                             int64_t nb_sb, int64_t nb_sh, const float* g_new, int j, int64_t pos,
                             const float* rec_in, float* rec_out, hipStream_t st, RopeK rk) {
  const int R = 2 * (a->H / a->Hkv);
  // record, two rewritten norm rows, ke / ve / vnrm / knrm; then the merge
  size_t lds = sizeof(float) * (size_t)dstep_words(s->Hkv, s->Me, s->Ms) + 2 * 2 * (size_t)DH + 4 * sizeof(float) * DH;
  const size_t red = (size_t)4 * R * (DH + 4) * sizeof(float);
  lds = lds > red ? lds : red;
  if (lds > 120 * 1024) return fail(CODA_EUNSUP, "coda_decode_step: bank of %d + %d rows too large", s->Me, s->Ms);
  const int rc = lds_limit<decode_step_bf16<DH>>(lds, "coda_decode_step");
  if (rc) return rc;
  hipLaunchKernelGGL((decode_step_bf16<DH>), dim3(s->Hkv, s->B), dim3(256), lds, st, *a, *s, (const bf16_t*)k_new,
                     (const bf16_t*)v_new, nb_sb, nb_sh, g_new, j, pos, rec_in, rec_out, rk);
  return check_launch("decode_step_bf16");
}

extern "C" int coda_decode_step_workspace_bytes(const coda_bank_desc* s, const coda_attn_desc* a, size_t* bytes) {
  int rc = validate_step(s, a);
  if (rc) return rc;
  CODA_REQUIRE(bytes != nullptr, "coda_decode_step_workspace_bytes: null out pointer");
  size_t att = 0;
  rc = coda_attn_workspace_bytes(a, &att);
  if (rc) return rc;
  *bytes = 2 * route_record_bytes(s) + att;
  return CODA_OK;
}

// The decode step; raw_k: k_new comes before RoPE and the kernels rope it
// with the query's tables (the token's own position in a write-then-attend
// step) wherever they write or read it.
static int decode_step_impl(const coda_bank_desc* s, const coda_attn_desc* a, const void* k_new, const void* v_new,
                            int64_t nb_sb, int64_t nb_sh, const float* g_new, int ring_idx, int ring_filled,
                            int64_t pos, void* workspace, size_t workspace_bytes, int* routed, void* stream,
                            bool raw_k, const char* who) {
  int rc = validate_step(s, a);
  if (rc) return rc;
  RopeK rk{nullptr, nullptr, 0};
  if (raw_k) {
    CODA_REQUIRE(a->rope_cos && a->rope_sin,
                 "%s: a raw new K is roped with the query's tables: rope_cos / rope_sin of the attention descriptor "
                 "missing", who);
    CODA_REQUIRE((uintptr_t)a->rope_cos % 16 == 0 && (uintptr_t)a->rope_sin % 16 == 0,
                 "%s: RoPE tables must be 16-byte aligned", who);
    rk = RopeK{a->rope_cos, a->rope_sin, a->rope_interleaved ? 1 : 2};
  }
  const int have_route = routed != nullptr && *routed != 0;
  if (routed) *routed = 0;
  hipStream_t st = (hipStream_t)stream;
  const size_t rec = route_record_bytes(s);
  coda_attn_desc d = *a;
  if (!step_routed(s, ring_filled)) {
    // ring still filling (or no banks): bank kernel, then the attention kernel
    rc = decode_write_impl(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st, rk, who);
    if (rc) return rc;
    d.workspace = workspace;
    d.workspace_bytes = workspace_bytes;
    return coda_diff_attn_fwd(&d, stream);
  }
  CODA_REQUIRE(k_new && v_new && g_new, "coda_decode_step: new token pointers missing");
  CODA_REQUIRE(ring_idx >= 0 && ring_idx < s->W, "coda_decode_step: ring_idx %d outside [0, %d)", ring_idx, s->W);
  CODA_REQUIRE(s->k_buf && s->v_buf && s->allowed && s->g_recent, "coda_decode_step: state buffers missing");
  CODA_REQUIRE(s->Me == 0 || (s->mem_last && s->exact_v_norm), "coda_decode_step: exact bank buffers missing");
  CODA_REQUIRE(s->Ms == 0 || (s->sum_lf_k_norm && s->eta), "coda_decode_step: summary bank buffers missing");
  CODA_REQUIRE(2 * s->lf == s->Dh, "coda_decode_step: lf %d unsupported (must be Dh/2)", s->lf);
  size_t att = 0;
  rc = coda_attn_workspace_bytes(a, &att);
  if (rc) return rc;
  if (!workspace || workspace_bytes < 2 * rec + att)
    return fail(CODA_ESMALL, "coda_decode_step: workspace %zu < %zu bytes", workspace_bytes, 2 * rec + att);
  if (s->B == 0) return CODA_OK;
  float* rec_in = (float*)((char*)workspace + (pos & 1) * rec);
  float* rec_out = (float*)((char*)workspace + ((pos + 1) & 1) * rec);
  if (!have_route) {
    rc = launch_decode_route(s, ring_idx, rec_in, st);
    if (rc) return rc;
  }
  if (fused_step_ok(s, a)) {
    rc = s->Dh == 128
             ? launch_fused_step<128>(s, a, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, pos, rec_in, rec_out, st, rk)
             : launch_fused_step<64>(s, a, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, pos, rec_in, rec_out, st, rk);
    if (rc == CODA_OK && routed) *routed = 1;
    return rc;
  }
  rc = launch_decode_bank(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, pos, rec_in, rec_out, st, rk);
  if (rc) return rc;
  d.workspace = (char*)workspace + 2 * rec;
  d.workspace_bytes = workspace_bytes - 2 * rec;
  rc = coda_diff_attn_fwd(&d, stream);
  if (rc == CODA_OK && routed) *routed = 1;
  return rc;
}

extern "C" int coda_decode_step(const coda_bank_desc* s, const coda_attn_desc* a, const void* k_new, const void* v_new,
                                int64_t nb_sb, int64_t nb_sh, const float* g_new, int ring_idx, int ring_filled,
                                int64_t pos, void* workspace, size_t workspace_bytes, int* routed, void* stream) {
  return decode_step_impl(s, a, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, workspace,
                          workspace_bytes, routed, stream, false, "coda_decode_step");
}

extern "C" int coda_decode_step_raw_k(const coda_bank_desc* s, const coda_attn_desc* a, const void* k_new,
                                      const void* v_new, int64_t nb_sb, int64_t nb_sh, const float* g_new,
                                      int ring_idx, int ring_filled, int64_t pos, void* workspace,
                                      size_t workspace_bytes, int* routed, void* stream) {
  return decode_step_impl(s, a, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, workspace,
                          workspace_bytes, routed, stream, true, "coda_decode_step_raw_k");
}
