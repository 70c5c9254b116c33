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

#include <atomic>
#include <chrono>

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

// Few token rows (M <= 64): the weights are the traffic, so every load of
// a workgroup is issued at once.  Workgroup (tile, ks) takes 128 features x
// all rows over k in [512 ks, 512 ks + 512): wave w's 16 weight rows go
// straight from global memory into its 16 A fragments (16 bytes per lane
// and k-step), the 64 token rows once into LDS (B fragments, shared by the
// 8 waves).  With KS = D / 512 > 1 each workgroup stores its fp32 partial
// tile (agent-scope atomic stores, the threads adjacent: one 512-byte run
// per wave and value pair), and the last of the KS workgroups of a tile to
// arrive (a counter per tile tagged with the launch's epoch, so it needs no
// clearing) sums the KS partials in split order and runs the epilogue:
// the result does not depend on arrival order.
static constexpr int kDecKR = 512;                 // k per workgroup
static constexpr int kDecPitch = kDecKR + 8;       // LDS row pitch (bf16)
__global__ __launch_bounds__(512) void proj_decode_bf16(const coda_proj_desc d, int n_feat, float* part,
                                                        unsigned long long* cnt, unsigned long long epoch) {
  using E = Elt<bf16_t>;
  constexpr int NT = 512, NS = kDecKR / 32, BT = 4, NP = BT * 2;
  extern __shared__ __attribute__((aligned(16))) bf16_t xs_lds[];  // [64][kDecPitch]
  __shared__ int last_s;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, r16 = lane & 15, kq = lane >> 4;
  const int KS = gridDim.y, ks = blockIdx.y;
  const int f0 = blockIdx.x * 128;
  const int k0 = ks * kDecKR;
  const bf16_t* W = (const bf16_t*)d.w;
  const bf16_t* X = (const bf16_t*)d.x;
  // A fragments: weight row f0 + 16 wv + r16, k0 + 32 s + 8 kq
  pbf16x8_t a[NS];
  {
    const bf16_t* wr = W + (int64_t)min(f0 + 16 * wv + r16, n_feat - 1) * d.D + k0 + 8 * kq;
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) a[s2] = *reinterpret_cast<const pbf16x8_t*>(wr + 32 * s2);
  }
  // token rows [0, 64) x k [k0, k0 + 512) into LDS, 8 pieces per thread
  {
    uint4 xv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = t + u * NT, r = i >> 6, c = i & 63;
      xv[u] = *reinterpret_cast<const uint4*>(X + (int64_t)min(r, d.M - 1) * d.x_sm + k0 + 8 * c);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = t + u * NT, r = i >> 6, c = i & 63;
      *reinterpret_cast<uint4*>(xs_lds + r * kDecPitch + 8 * c) = xv[u];
    }
  }
  __syncthreads();
  pf32x4 acc[BT];
#pragma unroll
  for (int j = 0; j < BT; ++j) acc[j] = pf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < NS; ++s2) {
    pbf16x8_t b[BT];
#pragma unroll
    for (int j = 0; j < BT; ++j)
      b[j] = *reinterpret_cast<const pbf16x8_t*>(xs_lds + (16 * j + r16) * kDecPitch + 32 * s2 + 8 * kq);
#pragma unroll
    for (int j = 0; j < BT; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s2], b[j], acc[j], 0, 0, 0);
  }
  if (!d.gate && blockIdx.x == 0 && ks == 0 && t < d.M) d.g[t] = 1.f;
  if (KS > 1) {
    const int64_t tile = blockIdx.x;
    unsigned long long* pw = reinterpret_cast<unsigned long long*>(part);
#pragma unroll
    for (int j = 0; j < BT; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const pf32x2 pr = {acc[j][2 * h], acc[j][2 * h + 1]};
        __hip_atomic_store(pw + ((tile * KS + ks) * NP + j * 2 + h) * NT + t,
                           __builtin_bit_cast(unsigned long long, pr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0) {
      unsigned long long* w = cnt + tile;
      unsigned long long old = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), nv;
      for (;;) {
        nv = (old >> 8) == epoch ? old + 1ull : ((epoch << 8) | 1ull);
        if (__hip_atomic_compare_exchange_strong(w, &old, nv, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
          break;
      }
      last_s = (int)(nv & 0xff) == KS;
    }
    __syncthreads();
    if (!last_s) return;
#pragma unroll
    for (int j = 0; j < BT; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const unsigned long long* p0 = pw + ((tile * KS) * NP + j * 2 + h) * NT + t;
        pf32x2 sum = __builtin_bit_cast(pf32x2, __hip_atomic_load(p0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        for (int q = 1; q < KS; ++q)
          sum += __builtin_bit_cast(pf32x2, __hip_atomic_load(p0 + (int64_t)q * NP * NT, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT));
        acc[j][2 * h] = sum[0];
        acc[j][2 * h + 1] = sum[1];
      }
  }
  // epilogue of features f0 + 16 wv + 4 kq .. + 3, tokens 16 j + r16
#pragma unroll
  for (int j = 0; j < BT; ++j) {
    const int m = 16 * j + r16;
    if (m < d.M) proj_store4(d, f0 + 16 * wv + 4 * kq, m, acc[j]);
  }
}

// Workspace of proj_decode_bf16 with KS = D / 512 > 1: the partial tiles
// and one counter per 128-feature tile.
static size_t proj_ws_bytes(int n_feat, int D) {
  const size_t tiles = (size_t)((n_feat + 127) / 128), KS = (size_t)(D / 512);
  return tiles * KS * 512 * 16 * sizeof(float) + tiles * sizeof(unsigned long long);  // 16 partials per thread
}
static unsigned long long proj_epoch() {
  static std::atomic<unsigned long long> ep{
      (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count() * 0x2545F4914F6CDD1Dull};
  return ep.fetch_add(1, std::memory_order_relaxed) & ((1ull << 56) - 1);
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
  // D a multiple of 512: every load of a workgroup at once, K split in
  // 512-wide ranges; else 64 x 64 tiles over K
  if (d->D % kDecKR == 0) {
    const int KS = d->D / kDecKR, tiles = (n_feat + 127) / 128;
    float* part = nullptr;
    unsigned long long* cnt = nullptr;
    if (KS > 1) {
      const size_t need = proj_ws_bytes(n_feat, d->D);
      CODA_REQUIRE(d->workspace && d->workspace_bytes >= need && ((uintptr_t)d->workspace % 16) == 0,
                   "coda_project: workspace %zu < %zu bytes (coda_project_workspace_bytes)", d->workspace_bytes, need);
      part = (float*)d->workspace;
      cnt = (unsigned long long*)(part + (size_t)tiles * KS * 512 * 16);
    }
    const size_t lds = sizeof(bf16_t) * 64 * kDecPitch;
    const int rc = lds_limit<proj_decode_bf16>(lds, "coda_project");
    if (rc) return rc;
    hipLaunchKernelGGL(proj_decode_bf16, dim3(tiles, KS), dim3(512), lds, st, *d, n_feat, part, cnt,
                       KS > 1 ? proj_epoch() : 0ull);
    return check_launch("proj_decode_bf16");
  }
  return launch_proj<64, 64, 4, 1>(d, n_feat, st);
}

extern "C" int coda_project_workspace_bytes(const coda_proj_desc* d, size_t* bytes) {
  CODA_REQUIRE(d != nullptr && bytes != nullptr, "coda_project_workspace_bytes: null pointer");
  const int n_feat = d->H * d->Dh + 2 * d->Hkv * d->Dh + d->H + (d->gate ? 1 : 0);
  *bytes = (d->M <= 64 && d->D % 512 == 0 && d->D > 512) ? proj_ws_bytes(n_feat, d->D) : 0;
  return CODA_OK;
}
