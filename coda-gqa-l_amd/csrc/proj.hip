// Projection front end of the bounded layer on gfx950: one GEMM of the
// token rows against the packed [q | k | v | lambda | write-gate] weights
// (bf16 MFMA, fp32 accumulation), with the epilogues of the reference's
// eager ops fused into the tile's store (attention.py:396-410, 592-608):
//   q, v    (+ bias) rounded to bf16;
//   k       (+ bias) rounded to bf16, then RoPE with the tables of the row's
//           position, one bf16 rounding per op (primitives.py:83-113);
//   lambda  sigmoid(bf16(acc + bias)) in bf16;
//   gate    sigmoid(bf16(acc + bias)) in bf16, stored as float32.
// The tile computes C^T = W X^T: MFMA A operand = weight rows (features), B
// operand = token rows, so each lane holds 4 consecutive features of one
// token (the RoPE pairs of a head sit in one lane; the half-split layout
// is packed with each pair (i, i + Dh/2) on adjacent weight rows).
#include "common.h"


namespace coda {

typedef __bf16 pbf16x8_t __attribute__((ext_vector_type(8)));
typedef float pf32x4 __attribute__((ext_vector_type(4)));
typedef float pf32x2 __attribute__((ext_vector_type(2)));

static constexpr int kProjKT = 64;        // k per LDS stage
static constexpr int kProjPitch = 72;     // LDS row pitch (bf16): 144 bytes, conflict-free fragment reads

__device__ __forceinline__ float proj_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

// Epilogue of features f .. f + 3 (f a multiple of 4) of token row m:
// the fp32 accumulators plus bias, rounded and routed to q / k (RoPE) / v /
// lambda / gate
__device__ __forceinline__ void proj_store4(const coda_proj_desc& d, int f, int m, pf32x4 v) {
  using E = Elt<bf16_t>;
  const int Fq = d.H * d.Dh, Fk = d.Hkv * d.Dh, half = d.Dh / 2;
  const int o_k = Fq, o_v = Fq + Fk, o_l = Fq + 2 * Fk, o_g = o_l + d.H;
  if (f + 3 < o_l) {  // q / k / v: the linear's bias (zero where it has none)
    const float4 bb = *reinterpret_cast<const float4*>(d.bias + f);
    v[0] += bb.x;
    v[1] += bb.y;
    v[2] += bb.z;
    v[3] += bb.w;
  }
  if (f + 3 < o_k) {  // q
    uint2 w;
    w.x = (uint32_t)E::st(v[0]) | ((uint32_t)E::st(v[1]) << 16);
    w.y = (uint32_t)E::st(v[2]) | ((uint32_t)E::st(v[3]) << 16);
    *reinterpret_cast<uint2*>((bf16_t*)d.q + (int64_t)m * d.q_sm + f) = w;
  } else if (f >= o_k && f + 3 < o_v) {  // k: two RoPE pairs
    const int kf = f - o_k, hk = kf / d.Dh, c = kf % d.Dh, prow = m % d.L;
    const bool inter = d.rope_interleaved != 0;
    const bf16_t* cs = (const bf16_t*)d.rope_cos;
    const bf16_t* sn = (const bf16_t*)d.rope_sin;
    bf16_t* krow = (bf16_t*)d.k + (int64_t)m * d.k_sm + (int64_t)hk * d.Dh;
    float r[4];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const int p = c / 2 + pp;  // pair index
      const float cc = E::ld(cs[(int64_t)prow * half + p]), ss = E::ld(sn[(int64_t)prow * half + p]);
      rope_pair_t<bf16_t>(E::rnd(v[2 * pp]), E::rnd(v[2 * pp + 1]), cc, ss, inter, r[2 * pp], r[2 * pp + 1]);
    }
    if (inter) {
      uint2 w;
      w.x = (uint32_t)E::st(r[0]) | ((uint32_t)E::st(r[1]) << 16);
      w.y = (uint32_t)E::st(r[2]) | ((uint32_t)E::st(r[3]) << 16);
      *reinterpret_cast<uint2*>(krow + c) = w;
    } else {  // packed pairs (p, p + half): channels c/2, c/2 + 1 and the same + half
      const int p = c / 2;
      *reinterpret_cast<uint32_t*>(krow + p) = (uint32_t)E::st(r[0]) | ((uint32_t)E::st(r[2]) << 16);
      *reinterpret_cast<uint32_t*>(krow + p + half) = (uint32_t)E::st(r[1]) | ((uint32_t)E::st(r[3]) << 16);
    }
  } else if (f >= o_v && f + 3 < o_l) {  // v
    uint2 w;
    w.x = (uint32_t)E::st(v[0]) | ((uint32_t)E::st(v[1]) << 16);
    w.y = (uint32_t)E::st(v[2]) | ((uint32_t)E::st(v[3]) << 16);
    *reinterpret_cast<uint2*>((bf16_t*)d.v + (int64_t)m * d.v_sm + (f - o_v)) = w;
  } else {  // lambda / write gate, one feature at a time
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int ff = f + rr;
      if (ff < o_l || ff >= o_g + (d.gate ? 1 : 0)) continue;
      const float lin = E::rnd(v[rr] + d.bias[ff]);
      const float sg = E::rnd(proj_sigmoid(lin));
      if (ff < o_g) ((bf16_t*)d.lam)[(int64_t)m * d.lam_sm + (ff - o_l)] = E::st(sg);
      else d.g[m] = sg;
    }
  }
}

// Workgroup tile: NTF features x MTT tokens; WF x WT waves, wave tile
// (NTF / WF) x (MTT / WT) in 16 x 16 MFMA blocks.  K staged through LDS in
// kProjKT slices, double-buffered through registers.
template <int NTF, int MTT, int WF, int WT>
__global__ __launch_bounds__(64 * WF * WT) void proj_gemm_bf16(const coda_proj_desc d, int n_feat) {
  using E = Elt<bf16_t>;
  constexpr int NT = 64 * WF * WT;
  constexpr int BF = NTF / WF / 16, BT = MTT / WT / 16;
  constexpr int ROWS = NTF + MTT, CH = kProjKT / 8, PER = ROWS * CH / NT;
  static_assert(ROWS * CH % NT == 0, "whole 16-byte pieces per thread");
  extern __shared__ __attribute__((aligned(16))) bf16_t proj_lds[];  // [2][ROWS * kProjPitch]
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int wf = wv % WF, wt = wv / WF;
  const int f0 = blockIdx.x * NTF, m0 = blockIdx.y * MTT;
  const bf16_t* W = (const bf16_t*)d.w;
  const bf16_t* X = (const bf16_t*)d.x;
  // this thread's pieces: row r of the stage (features first, then
  // tokens), 16-byte chunk c; rows past the matrices read row 0 / M - 1
  const bf16_t* src[PER];
  int dst[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = t + u * NT, r = i / CH, c = i % CH;
    if (r < NTF) {
      const int f = min(f0 + r, n_feat - 1);
      src[u] = W + (int64_t)f * d.D + 8 * c;
    } else {
      const int m = min(m0 + r - NTF, d.M - 1);
      src[u] = X + (int64_t)m * d.x_sm + 8 * c;
    }
    dst[u] = r * kProjPitch + 8 * c;
  }
  uint4 reg[PER];
  auto load = [&](int kb) {
#pragma unroll
    for (int u = 0; u < PER; ++u) reg[u] = *reinterpret_cast<const uint4*>(src[u] + kb * kProjKT);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER; ++u) *reinterpret_cast<uint4*>(&proj_lds[buf * ROWS * kProjPitch + dst[u]]) = reg[u];
  };
  pf32x4 acc[BF][BT];
#pragma unroll
  for (int i = 0; i < BF; ++i)
#pragma unroll
    for (int j = 0; j < BT; ++j) acc[i][j] = pf32x4{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, kq = lane >> 4;
  const int nk = d.D / kProjKT;
  load(0);
  store(0);
  __syncthreads();
  for (int kb = 0; kb < nk; ++kb) {
    if (kb + 1 < nk) load(kb + 1);
    const bf16_t* L = proj_lds + (kb & 1) * ROWS * kProjPitch;
#pragma unroll
    for (int s = 0; s < kProjKT / 32; ++s) {
      pbf16x8_t a[BF], b[BT];
#pragma unroll
      for (int i = 0; i < BF; ++i)
        a[i] = *reinterpret_cast<const pbf16x8_t*>(L + ((wf * BF + i) * 16 + r16) * kProjPitch + 32 * s + 8 * kq);
#pragma unroll
      for (int j = 0; j < BT; ++j)
        b[j] = *reinterpret_cast<const pbf16x8_t*>(L + (NTF + (wt * BT + j) * 16 + r16) * kProjPitch + 32 * s +
                                                   8 * kq);
#pragma unroll
      for (int i = 0; i < BF; ++i)
#pragma unroll
        for (int j = 0; j < BT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kb + 1 < nk) store((kb + 1) & 1);
    __syncthreads();
  }
  // ---- epilogue: lane holds features fb + 4 g4 .. + 3 of token tb + (lane & 15)
#pragma unroll
  for (int j = 0; j < BT; ++j) {
    const int m = m0 + (wt * BT + j) * 16 + r16;
    if (m >= d.M) continue;
#pragma unroll
    for (int i = 0; i < BF; ++i) proj_store4(d, f0 + (wf * BF + i) * 16 + 4 * kq, m, acc[i][j]);
  }
  if (!d.gate && blockIdx.x == 0)
    for (int m = m0 + t; m < min(d.M, m0 + MTT); m += NT) d.g[m] = 1.f;
}

// Few token rows (M <= 64): the weights are the traffic.  A workgroup owns
// 16 features over all of K: wave w of 8 takes k in [w K/8, (w + 1) K/8)
// and streams its 16 weight rows and the token rows of that range straight
// from memory into MFMA fragments (16 bytes per lane and k-step, LA steps
// ahead), one 16 x 16 accumulator per 16 tokens; the 8 partials meet in LDS
// and are summed in wave order (deterministic), then the epilogue runs on
// 64 MT lanes.  No workspace, no cross-workgroup exchange.  Weights cross
// HBM once; the token rows (at most 512 KiB) are read by every workgroup
// from L2.
static constexpr int kRowsLA = 4;  // k-steps of loads in flight ahead of the products
// RB row blocks of 16 features per wave: the token rows a wave loads feed
// RB products each.  TILED: W in fragment tiles (coda_project_pack), where
// the operand of row block fb at k-step ks is the KiB at (fb D/32 + ks) 512
// elements, lane l's 16 bytes at 8 l; else row-major with row stride w_sm.
template <int NS, int MT, int RB, bool TILED>
__device__ __forceinline__ void rows_partial(const bf16_t* __restrict__ W, int64_t w_sm, int n_feat,
                                             const bf16_t* __restrict__ X, int64_t x_sm, int M, int f0,
                                             pf32x4* part) {
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, r16 = lane & 15, kq = lane >> 4;
  const int k0 = wv * (NS * 32) + 8 * kq;
  const bf16_t* wr[RB];
  // element step between k-steps: 32 columns, or one tile
  constexpr int WS = TILED ? 512 : 32;
#pragma unroll
  for (int i = 0; i < RB; ++i)
    wr[i] = TILED ? W + ((int64_t)(f0 / 16 + i) * (8 * NS) + wv * NS) * 512 + 8 * lane
                  : W + (int64_t)min(f0 + 16 * i + r16, n_feat - 1) * w_sm + k0;
  const bf16_t* xr[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) xr[j] = X + (int64_t)min(16 * j + r16, M - 1) * x_sm + k0;
  pbf16x8_t a[kRowsLA][RB], b[kRowsLA][MT];
  auto load = [&](int s) {
#pragma unroll
    for (int i = 0; i < RB; ++i) a[s % kRowsLA][i] = *reinterpret_cast<const pbf16x8_t*>(wr[i] + WS * s);
#pragma unroll
    for (int j = 0; j < MT; ++j) b[s % kRowsLA][j] = *reinterpret_cast<const pbf16x8_t*>(xr[j] + 32 * s);
  };
  pf32x4 acc[RB][MT];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kRowsLA && s < NS; ++s) load(s);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    pbf16x8_t as[RB], bs[MT];
#pragma unroll
    for (int i = 0; i < RB; ++i) as[i] = a[s % kRowsLA][i];
#pragma unroll
    for (int j = 0; j < MT; ++j) bs[j] = b[s % kRowsLA][j];
    if (s + kRowsLA < NS) load(s + kRowsLA);
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as[i], bs[j], acc[i][j], 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) part[((wv * RB + i) * MT + j) * 64 + lane] = acc[i][j];
  __syncthreads();
}
// Sum of the 8 waves' partials for (row block i, token block j, lane l) =
// item 64 (MT i + j) + l: features f0 + 16 i + 4 (l / 16) .. + 3 of token
// 16 j + l % 16
template <int MT, int RB>
__device__ __forceinline__ pf32x4 rows_sum(const pf32x4* part, int item) {
  const int ij = item >> 6, l = item & 63;
  pf32x4 sum = part[ij * 64 + l];
#pragma unroll
  for (int w = 1; w < 8; ++w) sum += part[(w * RB * MT + ij) * 64 + l];
  return sum;
}

template <int NS, int MT, int RB, bool TILED>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void proj_rows_bf16(
    const coda_proj_desc d, int n_feat) {
  __shared__ pf32x4 part[8 * RB * MT * 64];
  const int f0 = blockIdx.x * 16 * RB;
  rows_partial<NS, MT, RB, TILED>((const bf16_t*)d.w, d.D, n_feat, (const bf16_t*)d.x, d.x_sm, d.M, f0, part);
  const int t = threadIdx.x;
  if (!d.gate && blockIdx.x == 0 && t < d.M) d.g[t] = 1.f;
  for (int item = t; item < 64 * MT * RB; item += 512) {
    const pf32x4 sum = rows_sum<MT, RB>(part, item);
    const int i = (item >> 6) / MT, j = (item >> 6) % MT, l = item & 63;
    const int m = 16 * j + (l & 15), f = f0 + 16 * i + 4 * (l >> 4);
    if (m < d.M && f < n_feat) proj_store4(d, f, m, sum);
  }
}

template <int NS, int RB, bool TILED>
static int launch_rows_t(const coda_proj_desc* d, int n_feat, hipStream_t st) {
  const dim3 grid((n_feat + 16 * RB - 1) / (16 * RB));
  if (d->M <= 16) hipLaunchKernelGGL((proj_rows_bf16<NS, 1, RB, TILED>), grid, dim3(512), 0, st, *d, n_feat);
  else if (d->M <= 32) hipLaunchKernelGGL((proj_rows_bf16<NS, 2, RB, TILED>), grid, dim3(512), 0, st, *d, n_feat);
  else hipLaunchKernelGGL((proj_rows_bf16<NS, 4, RB, TILED>), grid, dim3(512), 0, st, *d, n_feat);
  return check_launch("proj_rows_bf16");
}
template <int NS, int RB>
static int launch_rows_rb(const coda_proj_desc* d, int n_feat, hipStream_t st) {
  return d->w_layout == 1 ? launch_rows_t<NS, RB, true>(d, n_feat, st) : launch_rows_t<NS, RB, false>(d, n_feat, st);
}
// 16 RB features per workgroup: RB 2 up to 16 k-steps per wave (K <= 4096),
// RB 4 beyond (measured fastest at the 7B and 70B shapes, batch 1 .. 64)
template <int NS>
static int launch_rows_ns(const coda_proj_desc* d, int n_feat, hipStream_t st) {
  return launch_rows_rb<NS, (NS <= 16 ? 2 : 4)>(d, n_feat, st);
}
static int launch_rows(const coda_proj_desc* d, int n_feat, hipStream_t st) {
  switch (d->D / 256) {
    case 2: return launch_rows_ns<2>(d, n_feat, st);
    case 4: return launch_rows_ns<4>(d, n_feat, st);
    case 8: return launch_rows_ns<8>(d, n_feat, st);
    case 16: return launch_rows_ns<16>(d, n_feat, st);
    case 32: return launch_rows_ns<32>(d, n_feat, st);
    default: return -1;
  }
}
// one thread per 16-byte piece of the tiled copy
__global__ __launch_bounds__(256) void proj_pack_kernel(const bf16_t* __restrict__ w, int n_feat, int D, int64_t w_sm,
                                                        bf16_t* __restrict__ out, int64_t n_pieces) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_pieces) return;
  const int l = (int)(i & 63), r = l & 15, q = l >> 4;
  const int64_t tile = i >> 6;
  const int ksteps = D / 32;
  const int64_t fb = tile / ksteps;
  const int ks = (int)(tile % ksteps);
  const int64_t f = fb * 16 + r;
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (f < n_feat) v = *reinterpret_cast<const uint4*>(w + f * w_sm + 32 * ks + 8 * q);
  *reinterpret_cast<uint4*>(out + 8 * i) = v;
}

static bool rows_path(int D) {
  return D >= 512 && D <= 8192 && D % 256 == 0 && ((D / 256) & (D / 256 - 1)) == 0;
}

template <int NTF, int MTT, int WF, int WT>
static int launch_proj(const coda_proj_desc* d, int n_feat, hipStream_t st) {
  const dim3 grid((n_feat + NTF - 1) / NTF, (d->M + MTT - 1) / MTT);
  const size_t lds = 2 * sizeof(bf16_t) * (NTF + MTT) * kProjPitch;
  const int rc = lds_limit<proj_gemm_bf16<NTF, MTT, WF, WT>>(lds, "coda_project");
  if (rc) return rc;
  hipLaunchKernelGGL((proj_gemm_bf16<NTF, MTT, WF, WT>), grid, dim3(64 * WF * WT), lds, st, *d, n_feat);
  return check_launch("proj_gemm_bf16");
}

}  // namespace coda

using namespace coda;

extern "C" int coda_project(const coda_proj_desc* d, void* stream) {
  CODA_REQUIRE(d != nullptr, "coda_project: null descriptor");
  CODA_REQUIRE(d->dtype == CODA_BF16, "coda_project: bf16 only");
  CODA_REQUIRE(d->M >= 0 && d->M <= 64, "coda_project: %d token rows; the front end serves decode-shaped inputs "
               "(at most 64 rows), many rows are library GEMMs", d->M);
  CODA_REQUIRE(d->D > 0 && d->D % kProjKT == 0, "coda_project: D=%d must be a positive multiple of %d", d->D,
               kProjKT);
  CODA_REQUIRE(d->H > 0 && d->Hkv > 0 && d->Dh > 0 && d->Dh % 4 == 0 && d->L > 0,
               "coda_project: bad sizes H=%d Hkv=%d Dh=%d L=%d", d->H, d->Hkv, d->Dh, d->L);
  CODA_REQUIRE(d->x && d->w && d->bias && d->rope_cos && d->rope_sin && d->q && d->k && d->v && d->lam && d->g,
               "coda_project: pointer missing");
  CODA_REQUIRE(((uintptr_t)d->bias % 16) == 0, "coda_project: bias must be 16-byte aligned");
  CODA_REQUIRE(d->x_sm % 8 == 0 && ((uintptr_t)d->x % 16) == 0 && ((uintptr_t)d->w % 16) == 0,
               "coda_project: x / w rows must be 16-byte aligned");
  CODA_REQUIRE(d->q_sm % 4 == 0 && d->k_sm % 4 == 0 && d->v_sm % 4 == 0 && ((uintptr_t)d->q % 8) == 0 &&
                   ((uintptr_t)d->k % 8) == 0 && ((uintptr_t)d->v % 8) == 0,
               "coda_project: q / k / v rows must be 8-byte aligned");
  if (d->M == 0) return CODA_OK;
  const int n_feat = d->H * d->Dh + 2 * d->Hkv * d->Dh + d->H + (d->gate ? 1 : 0);
  hipStream_t st = (hipStream_t)stream;
  // K 512 .. 8192, a power of two times 256: row tiles over all of K (no
  // workspace); else 64 x 64 tiles over K
  CODA_REQUIRE(d->w_layout == 0 || (d->w_layout == 1 && rows_path(d->D)),
               "coda_project: weight layout %d with D=%d (tiles serve the row kernel's D only)", d->w_layout, d->D);
  if (rows_path(d->D)) return launch_rows(d, n_feat, st);
  return launch_proj<64, 64, 4, 1>(d, n_feat, st);
}

extern "C" int coda_project_pack(const void* w, int n_feat, int D, int64_t w_sm, void* out, void* stream) {
  CODA_REQUIRE(w && out && n_feat > 0 && D > 0 && w_sm >= D, "coda_project_pack: bad arguments");
  if (!rows_path(D)) return fail(CODA_EUNSUP, "coda_project_pack: D=%d does not take the row kernel", D);
  CODA_REQUIRE(w_sm % 8 == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)out % 16) == 0,
               "coda_project_pack: rows must be 16-byte aligned");
  // rows padded to a multiple of 64: the row kernel reads up to 4 row
  // blocks per workgroup past the last feature
  const int64_t n_pieces = (int64_t)((n_feat + 63) / 64) * 4 * (D / 32) * 64;
  hipLaunchKernelGGL(proj_pack_kernel, dim3((unsigned)((n_pieces + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)w, n_feat, D, w_sm, (bf16_t*)out, n_pieces);
  return check_launch("proj_pack_kernel");
}

extern "C" int coda_project_workspace_bytes(const coda_proj_desc* d, size_t* bytes) {
  CODA_REQUIRE(d != nullptr && bytes != nullptr, "coda_project_workspace_bytes: null pointer");
  *bytes = 0;
  return CODA_OK;
}
