// Device-side building blocks of bank maintenance shared by the bank
// kernels (banks.hip) and the decode attention kernel (attn.hip), which
// applies one head's bank update in its prologue.
//
// Every arithmetic step that feeds a decision or a stored value repeats the
// rounding of the reference's eager CPU ops (src/coda_gqa_l/memory_banks.py;
// one rounding to the element type per torch op, fp32 accumulation inside
// matmul / mean / norm / scatter_add).
#pragma once

#include "common.h"

#include <math.h>

namespace coda {

// Active bank sizes: the caller's device words when it keeps them on the
// device (dynamic expansion without host syncs), else the descriptor's ints
__device__ __forceinline__ int act_exact(const coda_bank_desc& s) { return s.active ? s.active[0] : s.active_exact; }
__device__ __forceinline__ int act_summary(const coda_bank_desc& s) {
  return s.active ? s.active[1] : s.active_summary;
}

static constexpr int64_t kNegBig = -(int64_t(1) << 62);
static constexpr int64_t kPosBig = int64_t(1) << 62;

template <typename T>
__device__ __forceinline__ float eps_r() {
  return Elt<T>::rnd(1e-6f);
}
template <typename T>
__device__ __forceinline__ float neg_fill() {
  return Elt<T>::rnd(-1e9f);
}

// Wave reductions for order-free combines (max / min with index ties,
// or, and): DPP within 16-lane rows (xor 1, xor 2, half-row mirror, row
// mirror), then the gfx950 permlane swaps across rows (16, 32), which
// hand both lanes of a pair the same two values in the same order.  Every
// lane ends with the result.
// (value, index) arg-max with first-occurrence ties, across a wave.
__device__ __forceinline__ void argmax_step(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  argmax_step(v, i, dpp_f<0xB1>(v), dpp_i<0xB1>(i));
  argmax_step(v, i, dpp_f<0x4E>(v), dpp_i<0x4E>(i));
  argmax_step(v, i, dpp_f<0x141>(v), dpp_i<0x141>(i));
  argmax_step(v, i, dpp_f<0x140>(v), dpp_i<0x140>(i));
  {
    const Pair2 pv = swap16(__builtin_bit_cast(int, v)), pi = swap16(i);
    v = __builtin_bit_cast(float, pv.a);
    i = pi.a;
    argmax_step(v, i, __builtin_bit_cast(float, pv.b), pi.b);
  }
  {
    const Pair2 pv = swap32(__builtin_bit_cast(int, v)), pi = swap32(i);
    v = __builtin_bit_cast(float, pv.a);
    i = pi.a;
    argmax_step(v, i, __builtin_bit_cast(float, pv.b), pi.b);
  }
}
__device__ __forceinline__ void argmin64_step(int64_t& v, int& i, int64_t ov, int oi) {
  if (ov < v || (ov == v && oi < i)) { v = ov; i = oi; }
}
template <int CTRL>
__device__ __forceinline__ int64_t dpp_i64(int64_t v) {
  const int lo = dpp_i<CTRL>((int)(uint32_t)v), hi = dpp_i<CTRL>((int)(v >> 32));
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ void wave_argmin_i64(int64_t& v, int& i) {
  argmin64_step(v, i, dpp_i64<0xB1>(v), dpp_i<0xB1>(i));
  argmin64_step(v, i, dpp_i64<0x4E>(v), dpp_i<0x4E>(i));
  argmin64_step(v, i, dpp_i64<0x141>(v), dpp_i<0x141>(i));
  argmin64_step(v, i, dpp_i64<0x140>(v), dpp_i<0x140>(i));
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const Pair2 lo = st ? swap32((int)(uint32_t)v) : swap16((int)(uint32_t)v);
    const Pair2 hi = st ? swap32((int)(v >> 32)) : swap16((int)(v >> 32));
    const Pair2 pi = st ? swap32(i) : swap16(i);
    v = (int64_t)(((uint64_t)(uint32_t)hi.a << 32) | (uint32_t)lo.a);
    i = pi.a;
    argmin64_step(v, i, (int64_t)(((uint64_t)(uint32_t)hi.b << 32) | (uint32_t)lo.b), pi.b);
  }
}
__device__ __forceinline__ int wave_or(int v) {
  v |= dpp_i<0xB1>(v);
  v |= dpp_i<0x4E>(v);
  v |= dpp_i<0x141>(v);
  v |= dpp_i<0x140>(v);
  Pair2 p = swap16(v);
  v = p.a | p.b;
  p = swap32(v);
  return p.a | p.b;
}
__device__ __forceinline__ int wave_and(int v) {
  v &= dpp_i<0xB1>(v);
  v &= dpp_i<0x4E>(v);
  v &= dpp_i<0x141>(v);
  v &= dpp_i<0x140>(v);
  Pair2 p = swap16(v);
  v = p.a & p.b;
  p = swap32(v);
  return p.a & p.b;
}
__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, dpp_i<0xB1>(v));
  v = min(v, dpp_i<0x4E>(v));
  v = min(v, dpp_i<0x141>(v));
  v = min(v, dpp_i<0x140>(v));
  Pair2 p = swap16(v);
  v = min(p.a, p.b);
  p = swap32(v);
  return min(p.a, p.b);
}

__device__ __forceinline__ void atomic_add_i64(int64_t* p, int64_t v) {
  if (p && v) atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v);
}

// Sum of squares of one row held by one wave (lane owns channels lane + 64 i,
// i < NV; the channels with act set are the contiguous range [LO, LO + len),
// LO a multiple of 8), summed in the order of torch's CPU last-dim 2-norm on
// x86 (ATen ReduceOpsKernel.cpp, norm_two_reduce_step into one 8-wide fp32
// accumulator vector): row channels r < nv = len - len % VW (VW = 8 fp32 /
// 16 bf16 elements per input vector) go to accumulator r % 8 in increasing
// order with fused multiply-adds, the eight accumulators are added in
// order, then each remaining channel adds its rounded square.  Every lane
// gets the sum.
template <typename T, int NV, int LO = 0>
__device__ __forceinline__ float wave_sumsq_cpu_order(const float (&x)[NV], const bool (&act)[NV]) {
  static_assert(LO % 8 == 0 && LO < 64 * NV, "band offset must be a multiple of 8 inside the row");
  constexpr int VW = sizeof(T) == 2 ? 16 : 8;
  int len = 0;
#pragma unroll
  for (int i = 0; i < NV; ++i) len += __popcll(__ballot(act[i]));
  const int nv = len - len % VW;
  const int j = threadIdx.x & 7;
  // accumulator j on lanes j, j + 8, ... (lane j's copy is read); row
  // channel r0 + j lives in register (LO + r0) / 64, lane (LO + r0) % 64 + j.
  // Every cross-lane fetch is issued before the chain starts: fetched one
  // at a time, each waits out the full LDS-crossbar latency
  constexpr int NR = (64 * NV - LO) / 8;
  float vals[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) vals[k] = __shfl(x[(LO + 8 * k) >> 6], ((LO + 8 * k) & 63) + j, 64);
  __builtin_amdgcn_sched_barrier(0);
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < NR; ++k)
    if (8 * k + j < nv) acc = fmaf(vals[k], vals[k], acc);
  float ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 0));
#pragma unroll
  for (int q = 1; q < 8; ++q)
    ss = ss + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), q));
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int k0 = max(LO + nv, 64 * i), k1 = min(LO + len, 64 * i + 64);
    for (int k = k0; k < k1; ++k) {
      const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x[i]), k - 64 * i));
      ss = ss + v * v;
    }
  }
  return ss;
}

// F.normalize(x, dim=-1, eps=1e-6) of one row held by one wave (lane owns
// channels lane + 64 i, i < NV; active channels [LO, LO + len)): fp32 sum of
// squares in the CPU order above, norm rounded to the element type,
// clamp_min(eps), rounded division.
template <typename T, int NV, int LO = 0>
__device__ __forceinline__ void wave_unit(float (&x)[NV], const bool (&act)[NV]) {
  using E = Elt<T>;
  const float ss = wave_sumsq_cpu_order<T, NV, LO>(x, act);
  const float den = fmaxf(E::rnd(sqrtf(ss)), eps_r<T>());
#pragma unroll
  for (int i = 0; i < NV; ++i) x[i] = act[i] ? E::rnd(x[i] / den) : 0.f;
}

template <typename T>
__device__ __forceinline__ void load8f(const T* p, float x[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf2f((bf16_t)(w[i] & 0xffffu));
      x[2 * i + 1] = bf2f((bf16_t)(w[i] >> 16));
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
}

// One step of a routing dot in torch's CPU bf16 matmul order (oneDNN on
// AVX512-BF16 hosts, the x86 VDPBF16PS accumulation): channel pairs (2i,
// 2i+1) in increasing i, the odd channel's product added first; bf16
// products are exact in fp32, so each add is one fused multiply-add.
__device__ __forceinline__ float dot_pair(float acc, float u0, float x0, float u1, float x1) {
  acc = fmaf(u1, x1, acc);
  return fmaf(u0, x0, acc);
}
__device__ __forceinline__ float dot8_pairs(float acc, const float* u, const float (&x)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(u);
  const float4 c = *reinterpret_cast<const float4*>(u + 4);
  acc = dot_pair(acc, a.x, x[0], a.y, x[1]);
  acc = dot_pair(acc, a.z, x[2], a.w, x[3]);
  acc = dot_pair(acc, c.x, x[4], c.y, x[5]);
  return dot_pair(acc, c.z, x[6], c.w, x[7]);
}

// dot(u, row) by one lane over len channels (a multiple of 8): row of T in
// device memory, u fp32 (16-byte aligned, LDS or registers' backing).
// Loads run PF 16-byte pieces ahead of the chain.  Unrounded.
template <typename T, int PF = 4>
__device__ __forceinline__ float lane_dot_cpu_order(const T* row, const float* u, int len) {
  float acc = 0.f;
  const int n8 = len >> 3;
  for (int c0 = 0; c0 < n8; c0 += PF) {
    float x[PF][8];
#pragma unroll
    for (int k = 0; k < PF; ++k) load8f<T>(row + 8 * min(c0 + k, n8 - 1), x[k]);
#pragma unroll
    for (int k = 0; k < PF; ++k)
      if (c0 + k < n8) acc = dot8_pairs(acc, u + 8 * (c0 + k), x[k]);
  }
  return acc;
}

// out[item] = rnd(dot(vec(item), mat_row(item))) for items enumerated by the
// caller through `row_ptr(item)` / `vec_ptr(item)`; len a multiple of 8.
// One lane per item (the chain is sequential in the CPU order), items
// wave * 64 + lane + 64 n_waves k.
template <typename T, typename RowF, typename VecF, typename OutF>
__device__ __forceinline__ void wave_dots(int n_items, int len, int wave, int n_waves, int lane, RowF row_ptr,
                                          VecF vec_ptr, OutF out) {
  for (int item = wave * 64 + lane; item < n_items; item += 64 * n_waves)
    out(item, Elt<T>::rnd(lane_dot_cpu_order<T>(row_ptr(item), vec_ptr(item), len)));
}

// ------------------------------------------------------------ decode decision
// Outcome of the exact and summary decisions for one evicted token.
struct DecodeDecision {
  int idx_e, ow_e, keep_e;
  int idx_s, keep_s, new_s;
};

// Exact bank decision for one token by one wave (memory_banks.py:240-290):
// de[h * Me + m] per-head cosine dots (rounded), used[m] (0/1) and last[m]
// the bank metadata before the update.  Lane 0 writes dec; with `count`
// it also adds the metrics / frustration counters.
template <typename T>
__device__ __forceinline__ void decide_exact(const coda_bank_desc& s, const float* de, const int* used,
                                             const int64_t* last, float g_e, DecodeDecision& dec, bool count,
                                             int lane) {
  using E = Elt<T>;
  const int Me = s.Me, Ae = act_exact(s), Hkv = s.Hkv;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  int any_used = 0, free_i = 0x7fffffff;
  int64_t lv = kPosBig + 1;
  int li = 0x7fffffff;
  for (int m = lane; m < Me; m += 64) {
    float acc = 0.f;
    for (int h = 0; h < Hkv; ++h) acc += de[h * Me + m];
    float sc = E::rnd(acc / (float)Hkv);
    const bool u = used[m] != 0;
    if (m >= Ae || !u) sc = neg_fill<T>();
    if (sc > bv || (sc == bv && m < bi)) { bv = sc; bi = m; }
    if (m < Ae && u) any_used = 1;
    if (m < Ae && !u && m < free_i) free_i = m;
    const int64_t lk = (m < Ae && u) ? last[m] : kPosBig;
    if (lk < lv || (lk == lv && m < li)) { lv = lk; li = m; }
  }
  wave_argmax(bv, bi);
  any_used = wave_or(any_used);
  free_i = wave_min_i(free_i);
  wave_argmin_i64(lv, li);
  if (lane == 0) {
    const bool keep = s.gated ? (g_e >= s.tau_exact) : true;
    const bool novel = !any_used || bv < E::rnd(s.tau_novel);
    const bool hit = any_used && bv >= E::rnd(s.tau_match);
    const bool free_exists = free_i != 0x7fffffff;
    const int idx = novel ? (free_exists ? free_i : li) : bi;
    const bool ow = (s.refresh_on_hit ? (novel || hit) : novel) && keep;
    dec.idx_e = idx;
    dec.ow_e = ow;
    dec.keep_e = keep;
    if (count) {
      if (s.metrics) {
        if (s.gated && !keep) atomic_add_i64(s.metrics + CODA_CNT_TOKENS_GATED_OUT, 1);
        if (hit) atomic_add_i64(s.metrics + CODA_CNT_EXACT_HITS, 1);
        if (novel && keep) atomic_add_i64(s.metrics + CODA_CNT_EXACT_INSERTS, 1);
        if (ow) atomic_add_i64(s.metrics + CODA_CNT_EXACT_OVERWRITES, 1);
      }
      if (s.frustrated && novel && keep && !free_exists) atomic_add_i64(s.frustrated + 0, 1);
    }
  }
}

// Summary bank routing for one token by one wave (memory_banks.py:352-392):
// ds[h * Ms + m] per-head LF-key dots, used[m] summary used bits before the
// update.
template <typename T>
__device__ __forceinline__ void decide_summary(const coda_bank_desc& s, const float* ds, const int* used, float g_e,
                                               DecodeDecision& dec, bool count, int lane) {
  using E = Elt<T>;
  const int Ms = s.Ms, As = act_summary(s), Hkv = s.Hkv;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int m = lane; m < Ms; m += 64) {
    float acc = 0.f;
    for (int h = 0; h < Hkv; ++h) acc += ds[h * Ms + m];
    float sc = E::rnd(acc / (float)Hkv);
    if (m >= As) sc = neg_fill<T>();
    if (sc > bv || (sc == bv && m < bi)) { bv = sc; bi = m; }
  }
  wave_argmax(bv, bi);
  const bool keep = s.gated ? (g_e >= s.tau_summary) : true;
  int all_used = 1;
  for (int m = lane; m < As; m += 64)
    if (!(used[m] != 0 || (keep && m == bi))) all_used = 0;
  all_used = wave_and(all_used);
  if (lane == 0) {
    dec.idx_s = bi;
    dec.keep_s = keep;
    dec.new_s = used[bi] == 0;
    if (count) {
      if (s.metrics) {
        if (keep) atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_UPDATES, 1);
        if (s.overwrite_on_insert && dec.new_s && keep) atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_INSERTS, 1);
      }
      if (s.frustrated) {
        if (!all_used) atomic_add_i64(s.frustrated + 1, 1);
        if (keep) atomic_add_i64(s.frustrated + 2, 1);
      }
    }
  }
}

// One element loaded into a 32-bit register as raw bits, and its value.
__device__ __forceinline__ uint32_t raw_ld(const bf16_t* p) { return *p; }
__device__ __forceinline__ uint32_t raw_ld(const float* p) { return __builtin_bit_cast(uint32_t, *p); }
template <typename T>
__device__ __forceinline__ float raw_f(uint32_t u);
template <>
__device__ __forceinline__ float raw_f<bf16_t>(uint32_t u) { return bf2f((bf16_t)u); }
template <>
__device__ __forceinline__ float raw_f<float>(uint32_t u) { return __builtin_bit_cast(float, u); }

// Bank writes of one head for one evicted token, by one wave; every old
// row this head needs (exact slot, summary slot) and the new token are
// loaded together, then:
//   exact  : new = mem + w * (k_e - mem), w = one-hot(idx) * overwrite,
//            V-norm cache row refreshed
//   summary: eta = eta_h (* gate) (1 if new) * keep;
//            K_LF += eta * (k_e_LF * energy - K_LF), V += eta * (v_e - V),
//            LF-K-norm cache row refreshed
//   ring   : slot j <- new token
// (memory_banks.py:296-331, :381-416, :214-222).  ke / ve: the evicted
// row of head h as floats; kn_src / vn_src: the new token of head h (its K
// roped here first when rk.mode != 0).
// With patch_e / patch_s (may be null) the refreshed V-norm row and LF-K-norm
// row are also written to those copies (rows of DH and LF elements).
template <typename T, int DH>
__device__ __forceinline__ void apply_head(const coda_bank_desc& s, int b, int h, const DecodeDecision& dec,
                                           const float* ke, const float* ve, const T* kn_src, const T* vn_src,
                                           int j, float g_e, int lane, T* patch_e = nullptr,
                                           T* patch_s = nullptr, T* rows_out = nullptr, RopeK rk = RopeK{nullptr, nullptr, 0}) {
  using E = Elt<T>;
  constexpr int NV = (DH + 63) / 64;
  const int Hkv = s.Hkv, W = s.W, Me = s.Me, Ms = s.Ms, lf = s.lf, LF = DH - lf;
  const int Lbuf = W + Me + Ms;
  T* kb = (T*)s.k_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;
  T* vb = (T*)s.v_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;
  const bool do_e = Me > 0 && dec.ow_e;
  const bool do_s = Ms > 0 && dec.keep_s;
  const int idx_e = Me > 0 ? dec.idx_e : 0, idx_s = Ms > 0 ? dec.idx_s : 0;
  T* kre = kb + (int64_t)(W + idx_e) * DH;
  T* vre = vb + (int64_t)(W + idx_e) * DH;
  T* krs = kb + (int64_t)(W + Me + idx_s) * DH;
  T* vrs = vb + (int64_t)(W + Me + idx_s) * DH;
  float mke[NV], mve[NV], mks[NV], mvs[NV], kn[NV], vn[NV];
  // every load in one batch (eta included), unconditional from
  // valid rows (the new token's where a bank row is not rewritten) and raw:
  // a conditional load, or a conversion next to the load, waits for it
  const float eta_h = Ms > 0 ? s.eta[h] : 0.f;
  const T* lke = do_e ? kre : kn_src;
  const T* lve = do_e ? vre : vn_src;
  const T* lks = do_s ? krs : kn_src;
  const T* lvs = do_s ? vrs : vn_src;
  uint32_t r_ke[NV], r_ve[NV], r_ks[NV], r_vs[NV], r_kn[NV], r_vn[NV], r_kp[NV], r_c[NV], r_s[NV];
  // a raw new K: its partner elements and table entries load with the rest
  // (from valid addresses: the row itself when there is no RoPE)
  const bool rope = rk.mode != 0;
  const T* rcs = rope ? (const T*)rk.cs : kn_src;
  const T* rsn = rope ? (const T*)rk.sn : kn_src;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = min(lane + 64 * i, DH - 1);
    r_ke[i] = raw_ld(lke + d);
    r_ve[i] = raw_ld(lve + d);
    r_ks[i] = raw_ld(lks + d);
    r_vs[i] = raw_ld(lvs + d);
    r_kn[i] = raw_ld(kn_src + d);
    r_vn[i] = raw_ld(vn_src + d);
    r_kp[i] = raw_ld(kn_src + (rope ? rope_k_partner(d, DH, rk.mode) : d));
    r_c[i] = raw_ld(rcs + (rope ? rope_k_table(d, DH, rk.mode) : 0));
    r_s[i] = raw_ld(rsn + (rope ? rope_k_table(d, DH, rk.mode) : 0));
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    mke[i] = do_e ? raw_f<T>(r_ke[i]) : 0.f;
    mve[i] = do_e ? raw_f<T>(r_ve[i]) : 0.f;
    mks[i] = do_s ? raw_f<T>(r_ks[i]) : 0.f;
    mvs[i] = do_s ? raw_f<T>(r_vs[i]) : 0.f;
    kn[i] = raw_f<T>(r_kn[i]);
    if (rope)
      kn[i] = rope_k_elem<T>(kn[i], raw_f<T>(r_kp[i]), raw_f<T>(r_c[i]), raw_f<T>(r_s[i]),
                             min(lane + 64 * i, DH - 1), DH, rk.mode);
    vn[i] = raw_f<T>(r_vn[i]);
  }
  if (do_e) {
    float nv[NV];
    bool act[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = d < DH;
      nv[i] = 0.f;
      if (act[i]) {
        const T kv = E::st(mke[i] + E::rnd(ke[d] - mke[i]));
        kre[d] = kv;
        nv[i] = E::rnd(mve[i] + E::rnd(ve[d] - mve[i]));
        vre[d] = E::st(nv[i]);
        if (rows_out) {
          rows_out[d] = kv;
          rows_out[DH + d] = E::st(nv[i]);
        }
      }
    }
    wave_unit<T, NV>(nv, act);
    T* nr = (T*)s.exact_v_norm + (((int64_t)b * Hkv + h) * Me + idx_e) * DH;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) {
        nr[lane + 64 * i] = E::st(nv[i]);
        if (patch_e) patch_e[lane + 64 * i] = E::st(nv[i]);
      }
  }
  if (do_s) {
    float eta = eta_h;
    if (s.gated) eta = E::rnd(eta * E::rnd(g_e));
    if (s.overwrite_on_insert && dec.new_s) eta = 1.f;
    float nk[NV];
    bool act[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = false;
      nk[i] = 0.f;
      if (d < DH) {
        const T vv = E::st(mvs[i] + E::rnd(eta * E::rnd(ve[d] - mvs[i])));
        vrs[d] = vv;
        if (rows_out) {
          rows_out[3 * DH + d] = vv;
          rows_out[2 * DH + d] = E::st(mks[i]);
        }
        if (d >= lf) {
          const float dk = E::rnd(E::rnd(ke[d] * s.energy_scale) - mks[i]);
          nk[i] = E::rnd(mks[i] + E::rnd(eta * dk));
          krs[d] = E::st(nk[i]);
          if (rows_out) rows_out[2 * DH + d] = E::st(nk[i]);
          act[i] = true;
        }
      }
    }
    wave_unit<T, NV, DH / 2>(nk, act);  // the LF band: channels [lf, DH), lf = DH / 2
    T* nr = (T*)s.sum_lf_k_norm + (((int64_t)b * Hkv + h) * Ms + idx_s) * LF;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) {
        nr[lane + 64 * i - lf] = E::st(nk[i]);
        if (patch_s) patch_s[lane + 64 * i - lf] = E::st(nk[i]);
      }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = lane + 64 * i;
    if (d < DH) {
      kb[(int64_t)j * DH + d] = E::st(kn[i]);
      vb[(int64_t)j * DH + d] = E::st(vn[i]);
    }
  }
}

// Per-sequence metadata after a decode update (one thread): used bits of
// the written slots, the LRU stamp, the ring gate, and the decision record
// when the caller asked for one.
__device__ __forceinline__ void commit_decode_meta(const coda_bank_desc& s, int b, const DecodeDecision& dec, int j,
                                                   int64_t pos_e, float g_new) {
  const int W = s.W, Me = s.Me, Ms = s.Ms;
  uint8_t* al = s.allowed + (int64_t)b * (W + Me + Ms);
  if (Me > 0) {
    if (dec.ow_e) al[W + dec.idx_e] = 1;
    if (dec.keep_e) s.mem_last[(int64_t)b * Me + dec.idx_e] = pos_e;
  }
  if (Ms > 0 && dec.keep_s) al[W + Me + dec.idx_s] = 1;
  s.g_recent[(int64_t)b * W + j] = g_new;
  if (s.trace) {
    int32_t* tr = s.trace + 4 * (int64_t)b;
    tr[0] = Me > 0 ? dec.idx_e : -1;
    tr[1] = Me > 0 ? ((dec.ow_e ? 1 : 0) | (dec.keep_e ? 2 : 0)) : 0;
    tr[2] = Ms > 0 ? dec.idx_s : -1;
    tr[3] = Ms > 0 ? ((dec.keep_s ? 1 : 0) | (dec.new_s ? 2 : 0)) : 0;
  }
}

// Routing record of one decode step, per sequence (4-byte words):
//   dots  [Hkv][Me + Ms] f32  per-head exact / summary cosine dots (rounded)
//   used  [Me + Ms] i32       bank used bits before the update
//   last  [Me] i64            LRU stamps before the update (8-byte aligned)
//   g_e   f32                 gate of the evicted ring slot
// padded to a multiple of 4 words, so every record is 16-byte aligned and
// moves to LDS in 16-byte pieces.
__host__ __device__ __forceinline__ int dstep_words(int Hkv, int Me, int Ms) {
  const int a = Hkv * (Me + Ms) + (Me + Ms);
  return (((a + 1) & ~1) + 2 * Me + 1 + 3) & ~3;
}
struct DStepWs {
  float* dots;
  int32_t* used;
  int64_t* last;
  float* g_e;
};
__host__ __device__ __forceinline__ DStepWs dstep_ws(float* ws, int b, int Hkv, int Me, int Ms) {
  float* base = ws + (int64_t)b * dstep_words(Hkv, Me, Ms);
  DStepWs w;
  w.dots = base;
  w.used = reinterpret_cast<int32_t*>(base + Hkv * (Me + Ms));
  const int a = Hkv * (Me + Ms) + (Me + Ms);
  w.last = reinterpret_cast<int64_t*>(base + ((a + 1) & ~1));
  w.g_e = base + ((a + 1) & ~1) + 2 * Me;
  return w;
}

// LDS of one (sequence, head) decode bank update: record [words] f32 |
// norm stage [Me*DH + Ms*LF] T | ke, ve, vnrm, knrm [DH] f32.
__host__ __device__ __forceinline__ size_t dbank_stage_elems(int DH, int Me, int Ms, int lf) {
  return ((size_t)Me * DH + (size_t)Ms * (DH - lf) + 7) & ~(size_t)7;
}
__host__ __device__ __forceinline__ size_t dbank_lds(const coda_bank_desc& s) {
  const size_t es = s.dtype == CODA_BF16 ? 2 : 4;
  return sizeof(float) * (size_t)dstep_words(s.Hkv, s.Me, s.Ms) + es * dbank_stage_elems(s.Dh, s.Me, s.Ms, s.lf) +
         sizeof(float) * 4 * (size_t)s.Dh;
}

// Copy nbytes (a multiple of 16) global -> LDS with direct loads by one
// wave (1 KiB per instruction, lane l the bytes [16 l, 16 l + 16)); the
// loads count in vmcnt.
__device__ __forceinline__ void wave_copy_lds(void* dst, const void* src, int nbytes, int lane) {
  for (int c = 0; c < nbytes; c += 1024)
    if (c + 16 * lane < nbytes)
      __builtin_amdgcn_global_load_lds((const char*)src + c + 16 * lane,
                                       (__attribute__((address_space(3))) void*)((char*)dst + c), 16, 0, 0);
}

// Routing dots of head h for evicting ring slot j of sequence b, by the
// 256 threads of a workgroup (every thread must call it): the evicted row
// (k, v) goes to LDS as floats (ke, ve: DH each), its unit V and unit LF-K
// band (vnrm: DH, knrm: LF) are formed by waves 0-1, then waves 0-1 take the
// dots with head h's exact V-norm cache rows (out_e[Me]) and waves 2-3 with
// its summary LF-K-norm rows (out_s[Ms]), each rounded to T
// (memory_banks.py:240-252, :352-364 per head, before the head mean).
template <typename T, int DH>
__device__ __forceinline__ void route_head_dots(const coda_bank_desc& s, int b, int h, int j, float* ke, float* ve,
                                                float* vnrm, float* knrm, float* out_e, float* out_s) {
  using E = Elt<T>;
  constexpr int NV = (DH + 63) / 64;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int Hkv = s.Hkv, W = s.W, Me = s.Me, Ms = s.Ms, lf = s.lf, LF = DH - lf;
  const int Lbuf = W + Me + Ms;
  const T* kr = (const T*)s.k_buf + (((int64_t)b * Hkv + h) * Lbuf + j) * DH;
  const T* vr = (const T*)s.v_buf + (((int64_t)b * Hkv + h) * Lbuf + j) * DH;
  for (int d = t; d < DH; d += 256) {
    ke[d] = E::ld(kr[d]);
    ve[d] = E::ld(vr[d]);
  }
  __syncthreads();
  if (wv < 2) {
    const bool is_v = wv == 0;
    if ((is_v && Me > 0) || (!is_v && Ms > 0)) {
      const int len = is_v ? DH : LF;
      float x[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lane + 64 * i;
        act[i] = d < len;
        x[i] = act[i] ? (is_v ? ve[d] : ke[lf + d]) : 0.f;
      }
      wave_unit<T, NV>(x, act);
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) (is_v ? vnrm : knrm)[lane + 64 * i] = x[i];
    }
  }
  __syncthreads();
  if (wv < 2 && Me > 0) {
    const T* en = (const T*)s.exact_v_norm + ((int64_t)b * Hkv + h) * Me * DH;
    wave_dots<T>(
        Me, DH, wv, 2, lane, [&](int it) { return en + (int64_t)it * DH; }, [&](int) { return (const float*)vnrm; },
        [&](int it, float v) { out_e[it] = v; });
  }
  if (wv >= 2 && Ms > 0) {
    const T* sn = (const T*)s.sum_lf_k_norm + ((int64_t)b * Hkv + h) * Ms * LF;
    wave_dots<T>(
        Ms, LF, wv - 2, 2, lane, [&](int it) { return sn + (int64_t)it * LF; },
        [&](int) { return (const float*)knrm; }, [&](int it, float v) { out_s[it] = v; });
  }
}

// Host launchers of decode_route_kernel, decode_bank_kernel and
// decode_write_kernel (defined with the bank kernels); rk: the new K's RoPE
// when it is handed over raw.
int launch_decode_route(const coda_bank_desc* s, int j, float* ws, hipStream_t st);
int launch_decode_bank(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb, int64_t nb_sh,
                       const float* g_new, int j, int64_t pos, const float* rec_in, float* rec_out, hipStream_t st,
                       RopeK rk);
int decode_write_impl(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb, int64_t nb_sh,
                      const float* g_new, int ring_idx, int ring_filled, int64_t pos, hipStream_t st, RopeK rk,
                      const char* who);

}  // namespace coda
