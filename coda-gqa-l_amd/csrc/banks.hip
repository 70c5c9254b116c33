// Bank maintenance of the bounded cache on gfx950: ring FIFO, exact bank
// (V-cosine novelty filter, first-free / LRU victim, delta writeback, LRU
// stamps) and summary bank (LF-K cosine routing, weighted accumulation,
// gated EMA), for one decode token and for one prefill chunk.
//
// Every arithmetic step that feeds a decision or a stored value repeats the
// rounding of the reference's eager CPU ops (memory_banks.py; one rounding
// to the element type per torch op, fp32 accumulation inside matmul / mean
// / norm / scatter_add), so slot decisions and written bytes are identical
// to the reference given identical inputs and state.
//
// Layout (contiguous): k_buf/v_buf [B][Hkv][Lbuf][Dh], Lbuf = W + Me + Ms,
// slots [0,W) ring, [W,W+Me) exact bank, [W+Me,Lbuf) summary bank.
#include "common.h"
#include "select.h"

#include <math.h>

#include <algorithm>
#include <vector>

namespace coda {

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

// (value, index) arg-max with first-occurrence ties, across a wave.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
  }
}
__device__ __forceinline__ void wave_argmin_i64(int64_t& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int64_t ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (ov < v || (ov == v && oi < i)) { v = ov; i = oi; }
  }
}
__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_and(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v &= __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ void atomic_add_i64(int64_t* p, int64_t v) {
  if (p && v) atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v);
}

// F.normalize(x, dim=-1, eps=1e-6) of one row held by one wave (lane owns
// channels lane + 64 i, i < NV): fp32 sum of squares, norm rounded to the
// element type, clamp_min(eps), rounded division.
template <typename T, int NV>
__device__ __forceinline__ void wave_unit(float (&x)[NV], const bool (&act)[NV]) {
  using E = Elt<T>;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (act[i]) ss = fmaf(x[i], x[i], ss);
  ss = wave_sum(ss);
  const float den = fmaxf(E::rnd(sqrtf(ss)), eps_r<T>());
#pragma unroll
  for (int i = 0; i < NV; ++i) x[i] = act[i] ? E::rnd(x[i] / den) : 0.f;
}

// Dots of rows of a [rows][len] device matrix (element T) against one fp32
// vector in LDS, cooperatively by a wave: `len/8` lanes per row, 8 channels
// per lane (one 16-byte load), group reduction by xor shuffles.
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

// out[item] = rnd(dot(vec(item), mat_row(item))), items enumerated by the
// caller through `row_ptr(item)` / `vec_ptr(item)`; len in {16,32,64,128}.
template <typename T, typename RowF, typename VecF, typename OutF>
__device__ __forceinline__ void wave_dots(int n_items, int len, int wave, int n_waves, int lane, RowF row_ptr,
                                          VecF vec_ptr, OutF out) {
  const int lpi = len >> 3;          // lanes per item
  const int ipw = 64 / lpi;          // items per wave step
  const int grp = lane / lpi, sub = lane % lpi;
  for (int base = wave * ipw; base < n_items; base += n_waves * ipw) {
    const int item = base + grp;
    float acc = 0.f;
    if (item < n_items) {
      float x[8];
      load8f<T>(row_ptr(item) + 8 * sub, x);
      const float* v = vec_ptr(item) + 8 * sub;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf(v[j], x[j], acc);
    }
    for (int o = lpi >> 1; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (item < n_items && sub == 0) out(item, Elt<T>::rnd(acc));
  }
}

struct DecodeDecision {
  int idx_e, ow_e, keep_e;
  int idx_s, keep_s, new_s;
};

// ------------------------------------------------------------ decode
// One workgroup (512 threads) per sequence b.  Reference: _write_one,
// _exact_update_one, _summary_update_one (memory_banks.py:183-432).
template <typename T, int DH>
__global__ __launch_bounds__(512) void decode_write_kernel(const coda_bank_desc s, const T* __restrict__ k_new,
                                                           const T* __restrict__ v_new, int64_t nb_sb,
                                                           int64_t nb_sh, const float* __restrict__ g_new,
                                                           int j, int filled, int64_t pos) {
  using E = Elt<T>;
  constexpr int NWV = 8, NT = 512, NV = (DH + 63) / 64;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  __shared__ DecodeDecision dec;
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int Hkv = s.Hkv, W = s.W, Me = s.Me, Ms = s.Ms, lf = s.lf, LF = DH - lf;
  const int Lbuf = W + Me + Ms;
  T* kb = (T*)s.k_buf + (int64_t)b * Hkv * Lbuf * DH;
  T* vb = (T*)s.v_buf + (int64_t)b * Hkv * Lbuf * DH;
  uint8_t* al = s.allowed + (int64_t)b * Lbuf;
  const T* kn_src = k_new + b * nb_sb;
  const T* vn_src = v_new + b * nb_sb;

  if (filled < W) {
    for (int i = t; i < Hkv * DH; i += NT) {
      const int h = i / DH, d = i % DH;
      kb[((int64_t)h * Lbuf + filled) * DH + d] = kn_src[h * nb_sh + d];
      vb[((int64_t)h * Lbuf + filled) * DH + d] = vn_src[h * nb_sh + d];
    }
    if (t == 0) {
      s.g_recent[(int64_t)b * W + filled] = g_new[b];
      al[filled] = 1;
    }
    return;
  }

  // LDS: ke, ve [Hkv][DH]; vn [Hkv][DH]; kn [Hkv][LF]; de [Hkv][Me]; ds [Hkv][Ms]
  float* ke = smem;
  float* ve = ke + Hkv * DH;
  float* vnrm = ve + Hkv * DH;
  float* knrm = vnrm + Hkv * DH;
  float* de = knrm + Hkv * LF;
  float* dsum = de + Hkv * Me;
  for (int i = t; i < Hkv * DH; i += NT) {
    const int h = i / DH, d = i % DH;
    ke[i] = E::ld(kb[((int64_t)h * Lbuf + j) * DH + d]);
    ve[i] = E::ld(vb[((int64_t)h * Lbuf + j) * DH + d]);
  }
  const float g_e = s.g_recent[(int64_t)b * W + j];
  const int64_t pos_e = pos - W;
  __syncthreads();
  // unit rows: exact V (full) and summary K (LF band), one wave per row
  for (int r = wv; r < 2 * Hkv; r += NWV) {
    const bool is_v = r < Hkv;
    if (is_v && Me == 0) continue;
    if (!is_v && Ms == 0) continue;
    const int h = is_v ? r : r - Hkv;
    const int len = is_v ? DH : LF;
    float x[NV];
    bool act[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = d < len;
      x[i] = act[i] ? (is_v ? ve[h * DH + d] : ke[h * DH + lf + d]) : 0.f;
    }
    wave_unit<T, NV>(x, act);
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) (is_v ? vnrm[h * DH + lane + 64 * i] : knrm[h * LF + lane + 64 * i]) = x[i];
  }
  __syncthreads();
  // per-head cosine dots against the norm caches
  if (Me > 0) {
    const T* en = (const T*)s.exact_v_norm + (int64_t)b * Hkv * Me * DH;
    wave_dots<T>(
        Hkv * Me, DH, wv, NWV, lane, [&](int it) { return en + (int64_t)it * DH; },
        [&](int it) { return (const float*)(vnrm + (it / Me) * DH); }, [&](int it, float v) { de[it] = v; });
  }
  if (Ms > 0) {
    const T* sn = (const T*)s.sum_lf_k_norm + (int64_t)b * Hkv * Ms * LF;
    wave_dots<T>(
        Hkv * Ms, LF, wv, NWV, lane, [&](int it) { return sn + (int64_t)it * LF; },
        [&](int it) { return (const float*)(knrm + (it / Ms) * LF); }, [&](int it, float v) { dsum[it] = v; });
  }
  __syncthreads();
  if (wv == 0 && Me > 0) {
    // exact decision (memory_banks.py:240-290)
    const int Ae = s.active_exact;
    const uint8_t* used = al + W;
    const int64_t* last = s.mem_last + (int64_t)b * Me;
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
    {
      int fi = free_i;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) fi = min(fi, __shfl_xor(fi, o, 64));
      free_i = fi;
    }
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
      if (s.metrics) {
        if (s.gated && !keep) atomic_add_i64(s.metrics + CODA_CNT_TOKENS_GATED_OUT, 1);
        if (hit) atomic_add_i64(s.metrics + CODA_CNT_EXACT_HITS, 1);
        if (novel && keep) atomic_add_i64(s.metrics + CODA_CNT_EXACT_INSERTS, 1);
        if (ow) atomic_add_i64(s.metrics + CODA_CNT_EXACT_OVERWRITES, 1);
      }
      if (s.frustrated && novel && keep && !free_exists) atomic_add_i64(s.frustrated + 0, 1);
    }
  }
  if (wv == 1 && Ms > 0) {
    // summary routing (memory_banks.py:352-392)
    const int As = s.active_summary;
    const uint8_t* used = al + W + Me;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    int all_used = 1;
    for (int m = lane; m < Ms; m += 64) {
      float acc = 0.f;
      for (int h = 0; h < Hkv; ++h) acc += dsum[h * Ms + m];
      float sc = E::rnd(acc / (float)Hkv);
      if (m >= As) sc = neg_fill<T>();
      if (sc > bv || (sc == bv && m < bi)) { bv = sc; bi = m; }
    }
    wave_argmax(bv, bi);
    const bool keep = s.gated ? (g_e >= s.tau_summary) : true;
    for (int m = lane; m < As; m += 64)
      if (!(used[m] != 0 || (keep && m == bi))) all_used = 0;
    all_used = wave_and(all_used);
    if (lane == 0) {
      dec.idx_s = bi;
      dec.keep_s = keep;
      dec.new_s = used[bi] == 0;
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
  __syncthreads();
  // exact write: w = one-hot(idx) * overwrite; new = mem + w * (k - mem)
  if (Me > 0) {
    const int idx = dec.idx_e;
    if (dec.ow_e) {
      for (int h = wv; h < Hkv; h += NWV) {
        T* kr = kb + ((int64_t)h * Lbuf + W + idx) * DH;
        T* vr = vb + ((int64_t)h * Lbuf + W + idx) * DH;
        float nv[NV];
        bool act[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int d = lane + 64 * i;
          act[i] = d < DH;
          nv[i] = 0.f;
          if (act[i]) {
            const float mk = E::ld(kr[d]), mv = E::ld(vr[d]);
            kr[d] = E::st(mk + E::rnd(ke[h * DH + d] - mk));
            nv[i] = E::rnd(mv + E::rnd(ve[h * DH + d] - mv));
            vr[d] = E::st(nv[i]);
          }
        }
        wave_unit<T, NV>(nv, act);
        T* nr = (T*)s.exact_v_norm + (((int64_t)b * Hkv + h) * Me + idx) * DH;
#pragma unroll
        for (int i = 0; i < NV; ++i)
          if (act[i]) nr[lane + 64 * i] = E::st(nv[i]);
      }
      if (t == 0) al[W + idx] = 1;
    }
    if (t == 0 && dec.keep_e) s.mem_last[(int64_t)b * Me + idx] = pos_e;
  }
  // summary write: eta = sigmoid(logit_h) (* gate) (1 if new) * keep
  if (Ms > 0 && dec.keep_s) {
    const int idx = dec.idx_s;
    for (int h = wv; h < Hkv; h += NWV) {
      float eta = E::rnd(1.f / (1.f + expf(-s.eta_logit[h])));
      if (s.gated) eta = E::rnd(eta * E::rnd(g_e));
      if (s.overwrite_on_insert && dec.new_s) eta = 1.f;
      T* kr = kb + ((int64_t)h * Lbuf + W + Me + idx) * DH;
      T* vr = vb + ((int64_t)h * Lbuf + W + Me + idx) * DH;
      float nk[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lane + 64 * i;
        act[i] = d < LF;
        nk[i] = 0.f;
        if (d < DH) {
          const float mv = E::ld(vr[d]);
          vr[d] = E::st(mv + E::rnd(eta * E::rnd(ve[h * DH + d] - mv)));
        }
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lf + lane + 64 * i;
        if (act[i]) {
          const float mk = E::ld(kr[d]);
          const float dk = E::rnd(E::rnd(ke[h * DH + d] * s.energy_scale) - mk);
          nk[i] = E::rnd(mk + E::rnd(eta * dk));
          kr[d] = E::st(nk[i]);
        }
      }
      wave_unit<T, NV>(nk, act);
      T* nr = (T*)s.sum_lf_k_norm + (((int64_t)b * Hkv + h) * Ms + idx) * LF;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) nr[lane + 64 * i] = E::st(nk[i]);
    }
    if (t == 0) al[W + Me + idx] = 1;
  }
  __syncthreads();
  // ring overwrite of the evicted slot
  for (int i = t; i < Hkv * DH; i += NT) {
    const int h = i / DH, d = i % DH;
    kb[((int64_t)h * Lbuf + j) * DH + d] = kn_src[h * nb_sh + d];
    vb[((int64_t)h * Lbuf + j) * DH + d] = vn_src[h * nb_sh + d];
  }
  if (t == 0) s.g_recent[(int64_t)b * W + j] = g_new[b];
}

// ------------------------------------------------------------ block plan
// One wave per (chunk, sequence); lane 0 runs the libstdc++-order selection
// on the chunk's evicted gates staged in LDS.  Gates of the virtual
// sequence S = [initial ring (time order) | g_seq].
struct PlanGeom {
  int W, L, block, Lr0, ring_head, kE, kS, doE, doS, Kmax, B;
};

__global__ __launch_bounds__(64) void block_plan_kernel(const float* __restrict__ g_ring,
                                                        const float* __restrict__ g_seq, int64_t g_sb,
                                                        PlanGeom p, int32_t* __restrict__ plan) {
  extern __shared__ __attribute__((aligned(16))) char psmem[];
  sel::Item<float>* items = reinterpret_cast<sel::Item<float>*>(psmem);
  const int c = blockIdx.x, b = blockIdx.y;
  const int t0 = c * p.block;
  const int blk = min(p.block, p.L - t0);
  // ring occupancy at the start of chunk c
  const int64_t seen = (int64_t)p.Lr0 + t0;
  const int Lr = (int)min<int64_t>(p.W, seen);
  const int total = Lr + blk;
  const int keep_len = min(p.W, total);
  const int n_ev = total - keep_len;
  int32_t* out = plan + ((int64_t)c * p.B + b) * p.Kmax;
  if (n_ev <= 0) return;
  int K;
  if (p.doE && p.doS) K = max(min(p.kE, n_ev), min(p.kS, n_ev));
  else if (p.doE) K = min(p.kE, n_ev);
  else if (p.doS) K = min(p.kS, n_ev);
  else return;
  const int64_t base = seen - Lr;  // S index of evicted token 0
  for (int i = threadIdx.x; i < n_ev; i += 64) {
    const int64_t si = base + i;
    float g;
    if (si < p.Lr0) {
      const int slot = (p.Lr0 == p.W) ? (int)((p.ring_head + si) % p.W) : (int)si;
      g = g_ring[(int64_t)b * p.W + slot];
    } else {
      g = g_seq[(int64_t)b * g_sb + (si - p.Lr0)];
    }
    items[i] = sel::Item<float>{g, (int64_t)i};
  }
  __syncthreads();
  if (threadIdx.x == 0) sel::topk_order<float>(items, n_ev, K, true, false);
  __syncthreads();
  for (int i = threadIdx.x; i < K; i += 64) out[i] = (int32_t)items[i].i;
}

// ------------------------------------------------------------ block write
// Workspace layout per call (4-byte words), T = max(Te, Ts):
//   dot_e [B][Hkv][Te][Me] f32   per-head exact cosine dots (rounded)
//   dot_s [B][Hkv][Ts][Ms] f32   per-head summary cosine dots (rounded)
//   dec   [B][3][T] i32          idx_e, ow | touch << 1, idx_s
//   wtok  [B][Ts] f32            summary weight (rounded to the element type)
//   slot  [B][Me + 2 Ms]         exact overwrite flag (i32), summary count
//                                (f32, rounded), summary flags (i32: 1 active,
//                                2 fresh = active and previously unused)
struct BlockGeom {
  int blk, ring_head, ring_filled, n_ev, Kmax, Te, Ts;
  int64_t pos0;
  int64_t b_sb, b_sh, b_sl, g_sb;
};

__host__ __device__ __forceinline__ size_t ws_dot_s(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return (size_t)B * Hkv * Te * Me;
}
__host__ __device__ __forceinline__ size_t ws_dec(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return ws_dot_s(B, Hkv, Me, Ms, Te, Ts) + (size_t)B * Hkv * Ts * Ms;
}
__host__ __device__ __forceinline__ size_t ws_wtok(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return ws_dec(B, Hkv, Me, Ms, Te, Ts) + (size_t)B * 3 * (Te > Ts ? Te : Ts);
}
__host__ __device__ __forceinline__ size_t ws_slot(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return ws_wtok(B, Hkv, Me, Ms, Te, Ts) + (size_t)B * Ts;
}
__host__ __device__ __forceinline__ size_t ws_total(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return ws_slot(B, Hkv, Me, Ms, Te, Ts) + (size_t)B * (Me + 2 * Ms);
}
#define CODA_WS(fn, s, g) fn((s).B, (s).Hkv, (s).Me, (s).Ms, (g).Te, (g).Ts)

// Source row of evicted candidate e (index into the chunk's time-ordered
// [ring | block] sequence) for KV head h: ring slot or block token.
template <typename T, int DH>
__device__ __forceinline__ const T* cand_row(const coda_bank_desc& s, const BlockGeom& g, const T* kbk, int b,
                                             int h, int e, bool value) {
  const int Lbuf = s.W + s.Me + s.Ms;
  if (e < g.ring_filled) {
    const int slot = (g.ring_filled == s.W) ? (g.ring_head + e) % s.W : e;
    const T* buf = (const T*)(value ? s.v_buf : s.k_buf);
    return buf + (((int64_t)b * s.Hkv + h) * Lbuf + slot) * DH;
  }
  return kbk + b * g.b_sb + h * g.b_sh + (int64_t)(e - g.ring_filled) * g.b_sl;
}

__device__ __forceinline__ float cand_gate(const coda_bank_desc& s, const BlockGeom& g, const float* gb, int b,
                                           int e) {
  if (e < g.ring_filled) {
    const int slot = (g.ring_filled == s.W) ? (g.ring_head + e) % s.W : e;
    return s.g_recent[(int64_t)b * s.W + slot];
  }
  return gb[(int64_t)b * g.g_sb + (e - g.ring_filled)];
}

// K1: per (b, h): unit() of the candidate rows and their per-head cosine
// dots against the exact V-norm and summary LF-K-norm caches
// (memory_banks.py:492-500, :640-644, :866-868).
template <typename T, int DH>
__global__ __launch_bounds__(256) void block_route_kernel(const coda_bank_desc s, BlockGeom g, const T* kbk,
                                                          const T* vbk, const int32_t* __restrict__ plan_c,
                                                          float* __restrict__ ws) {
  constexpr int NV = (DH + 63) / 64, NWV = 4;
  extern __shared__ __attribute__((aligned(16))) float rsm[];
  const int h = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int LF = DH - s.lf;
  float* vn = rsm;                 // [Te][DH]
  float* kn = vn + g.Te * DH;      // [Ts][LF]
  const int32_t* pc = plan_c + (int64_t)b * g.Kmax;
  for (int r = wv; r < g.Te + g.Ts; r += NWV) {
    const bool is_v = r < g.Te;
    const int tt = is_v ? r : r - g.Te;
    const int e = pc[tt];
    const T* src = is_v ? cand_row<T, DH>(s, g, vbk, b, h, e, true) : cand_row<T, DH>(s, g, kbk, b, h, e, false);
    const int len = is_v ? DH : LF;
    const int off = is_v ? 0 : s.lf;
    float x[NV];
    bool act[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = d < len;
      x[i] = act[i] ? Elt<T>::ld(src[off + d]) : 0.f;
    }
    wave_unit<T, NV>(x, act);
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (act[i]) (is_v ? vn[tt * DH + lane + 64 * i] : kn[tt * LF + lane + 64 * i]) = x[i];
  }
  __syncthreads();
  if (g.Te > 0) {
    const T* en = (const T*)s.exact_v_norm + ((int64_t)b * s.Hkv + h) * s.Me * DH;
    float* out = ws + (((int64_t)b * s.Hkv + h) * g.Te) * s.Me;
    const int Me = s.Me;
    wave_dots<T>(
        g.Te * Me, DH, wv, NWV, lane, [&](int it) { return en + (int64_t)(it % Me) * DH; },
        [&](int it) { return (const float*)(vn + (it / Me) * DH); }, [&](int it, float v) { out[it] = v; });
  }
  if (g.Ts > 0) {
    const T* sn = (const T*)s.sum_lf_k_norm + ((int64_t)b * s.Hkv + h) * s.Ms * LF;
    float* out = ws + CODA_WS(ws_dot_s, s, g) + (((int64_t)b * s.Hkv + h) * g.Ts) * s.Ms;
    const int Ms = s.Ms;
    wave_dots<T>(
        g.Ts * Ms, LF, wv, NWV, lane, [&](int it) { return sn + (int64_t)(it % Ms) * LF; },
        [&](int it) { return (const float*)(kn + (it / Ms) * LF); }, [&](int it, float v) { out[it] = v; });
  }
}

// K2: per b: head means, exact decisions (novelty, LRU topk, cumsum rank,
// touch / overwrite, LRU stamps, used), summary routing, weights, counts.
// Reference: memory_banks.py:635-697 + :721-727 (exact), :513-528 +
// :866-918 (summary).  Per-slot results go to the workspace; `allowed` is
// updated here, after every read of the pre-update bits.
template <typename T, int DH>
__global__ __launch_bounds__(256) void block_decide_kernel(const coda_bank_desc s, BlockGeom g, const float* gb,
                                                           const int32_t* __restrict__ plan_c,
                                                           float* __restrict__ ws) {
  using E = Elt<T>;
  extern __shared__ __attribute__((aligned(16))) char dsm[];
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int W = s.W, Me = s.Me, Ms = s.Ms, Hkv = s.Hkv, Te = g.Te, Ts = g.Ts;
  const int Lbuf = W + Me + Ms;
  uint8_t* al = s.allowed + (int64_t)b * Lbuf;
  const int32_t* pc = plan_c + (int64_t)b * g.Kmax;
  const int TT = max(Te, Ts);
  int32_t* dec = reinterpret_cast<int32_t*>(ws + CODA_WS(ws_dec, s, g)) + (int64_t)b * 3 * TT;
  float* wtok = ws + CODA_WS(ws_wtok, s, g) + (int64_t)b * Ts;
  int32_t* eflag = reinterpret_cast<int32_t*>(ws + CODA_WS(ws_slot, s, g)) + (int64_t)b * (Me + 2 * Ms);
  float* cnt = reinterpret_cast<float*>(eflag + Me);
  int32_t* sflag = eflag + Me + Ms;

  if (Te > 0) {
    // LDS: rk [Me] items (16 B each) | sc [Te][Me] f32 | best [Te] f32 | best_i [Te] i32
    sel::Item<int64_t>* rk = reinterpret_cast<sel::Item<int64_t>*>(dsm);
    float* sc = reinterpret_cast<float*>(rk + Me);
    float* best = sc + Te * Me;
    int* best_i = reinterpret_cast<int*>(best + Te);
    const float* de = ws + (int64_t)b * Hkv * Te * Me;
    for (int i = t; i < Te * Me; i += 256) {
      float acc = 0.f;
      for (int h = 0; h < Hkv; ++h) acc += de[(int64_t)h * Te * Me + i];
      float v = E::rnd(acc / (float)Hkv);
      const int m = i % Me;
      if (m >= s.active_exact || al[W + m] == 0) v = neg_fill<T>();
      sc[i] = v;
    }
    for (int m = t; m < Me; m += 256) {
      const bool u = al[W + m] != 0 && m < s.active_exact;
      rk[m] = sel::Item<int64_t>{u ? s.mem_last[(int64_t)b * Me + m] : kNegBig, (int64_t)m};
    }
    __syncthreads();
    for (int tt = wv; tt < Te; tt += 4) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int m = lane; m < Me; m += 64) {
        const float v = sc[tt * Me + m];
        if (v > bv || (v == bv && m < bi)) { bv = v; bi = m; }
      }
      wave_argmax(bv, bi);
      if (lane == 0) { best[tt] = bv; best_i[tt] = bi; }
    }
    __syncthreads();
    if (t == 0) {
      const int Ae = s.active_exact;
      int any_used = 0;
      for (int m = 0; m < Me; ++m) any_used |= al[W + m] != 0;
      const int n_lru = min(Te, Ae);
      sel::topk_order<int64_t>(rk, Me, n_lru, false, true);
      int64_t* last = s.mem_last + (int64_t)b * Me;
      int rank = -1;
      int64_t cnt_ow = 0, cnt_cap = 0, cnt_hit = 0, cnt_gated = 0, cnt_fr = 0;
      for (int tt = 0; tt < Te; ++tt) {
        const float gate = cand_gate(s, g, gb, b, pc[tt]);
        const bool keep = s.gated ? (gate >= s.tau_exact) : true;
        const float bv = best[tt];
        const bool novel = !any_used || bv < E::rnd(s.tau_novel);
        const bool hit = any_used && bv >= E::rnd(s.tau_match);
        const bool nk = novel && keep;
        if (nk) ++rank;                       // rank = cumsum(nk) - 1 at tt
        const bool cap = nk && rank < Ae;
        int idx = best_i[tt];
        if (cap) {
          int r = rank < 0 ? 0 : rank;
          if (r > n_lru - 1) r = n_lru - 1;
          idx = (int)rk[r].i;
        }
        const bool touch = keep && (!novel || cap);
        const bool ow = s.refresh_on_hit ? (keep && (cap || hit)) : cap;
        dec[tt] = idx;
        dec[TT + tt] = (ow ? 1 : 0) | (touch ? 2 : 0);
        cnt_ow += ow;
        cnt_cap += cap;
        cnt_hit += (hit && keep);
        cnt_gated += !keep;
        cnt_fr += (nk && !cap);
      }
      // LRU stamps: last[m] = max pos of the tokens touching m
      for (int m = 0; m < Me; ++m) {
        int64_t pv = kNegBig;
        bool tm = false;
        int f = 0;
        for (int tt = 0; tt < Te; ++tt) {
          if (dec[tt] != m) continue;
          if (dec[TT + tt] & 2) {
            tm = true;
            const int64_t p = g.pos0 - g.ring_filled + pc[tt];
            if (p > pv) pv = p;
          }
          f |= dec[TT + tt] & 1;
        }
        if (tm) last[m] = pv;
        eflag[m] = f;
      }
      if (s.metrics) {
        atomic_add_i64(s.metrics + CODA_CNT_EXACT_OVERWRITES, cnt_ow);
        atomic_add_i64(s.metrics + CODA_CNT_EXACT_FRUSTRATED, cnt_fr);
        atomic_add_i64(s.metrics + CODA_CNT_EXACT_INSERTS, cnt_cap);
        atomic_add_i64(s.metrics + CODA_CNT_EXACT_HITS, cnt_hit);
        if (s.gated) atomic_add_i64(s.metrics + CODA_CNT_TOKENS_GATED_OUT, cnt_gated);
      }
      if (s.frustrated) atomic_add_i64(s.frustrated + 0, cnt_fr);
    }
    __syncthreads();
  } else {
    for (int m = t; m < Me; m += 256) eflag[m] = 0;
  }
  if (Ts > 0) {
    float* sc = reinterpret_cast<float*>(dsm);  // [Ts][Ms]; the exact scratch is dead
    const float* dsd = ws + CODA_WS(ws_dot_s, s, g) + (int64_t)b * Hkv * Ts * Ms;
    for (int i = t; i < Ts * Ms; i += 256) {
      float acc = 0.f;
      for (int h = 0; h < Hkv; ++h) acc += dsd[(int64_t)h * Ts * Ms + i];
      float v = E::rnd(acc / (float)Hkv);
      if (i % Ms >= s.active_summary) v = neg_fill<T>();
      sc[i] = v;
    }
    __syncthreads();
    for (int tt = wv; tt < Ts; tt += 4) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int m = lane; m < Ms; m += 64) {
        const float v = sc[tt * Ms + m];
        if (v > bv || (v == bv && m < bi)) { bv = v; bi = m; }
      }
      wave_argmax(bv, bi);
      if (lane == 0) {
        dec[2 * TT + tt] = bi;
        const float gate = cand_gate(s, g, gb, b, pc[tt]);
        wtok[tt] = (!s.gated || gate >= s.tau_summary) ? E::rnd(gate) : 0.f;
      }
    }
    __syncthreads();
    for (int m = t; m < Ms; m += 256) {
      float c = 0.f;
      for (int tt = 0; tt < Ts; ++tt)
        if (dec[2 * TT + tt] == m) c += wtok[tt];
      cnt[m] = E::rnd(c);
      const bool active = cnt[m] > 0.f;
      const bool fresh = active && al[W + Me + m] == 0;
      sflag[m] = (active ? 1 : 0) | (fresh ? 2 : 0);
    }
  } else {
    for (int m = t; m < Ms; m += 256) { cnt[m] = 0.f; sflag[m] = 0; }
  }
  __syncthreads();
  if (t == 0) {
    int64_t upd = 0, ins = 0;
    int all_used = 1, any_cnt = 0;
    for (int m = 0; m < Ms; ++m) {
      const int f = sflag[m];
      upd += f & 1;
      ins += (f >> 1) & 1;
      if (m < s.active_summary) {
        if (!(al[W + Me + m] != 0 || (f & 1))) all_used = 0;
        if (f & 1) any_cnt = 1;
      }
    }
    if (Ts > 0) {
      if (s.metrics) {
        atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_UPDATES, upd);
        if (s.overwrite_on_insert) atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_INSERTS, ins);
      }
      if (s.frustrated) {
        if (!all_used) atomic_add_i64(s.frustrated + 1, 1);
        if (any_cnt) atomic_add_i64(s.frustrated + 2, 1);
      }
    }
    for (int m = 0; m < Me; ++m)
      if (eflag[m]) al[W + m] = 1;
    for (int m = 0; m < Ms; ++m)
      if (sflag[m] & 1) al[W + Me + m] = 1;
  }
}

// K3: per (b, h): exact delta writeback + V-norm cache, summary
// accumulation + EMA + LF-K-norm cache (memory_banks.py:707-742,
// :880-932), then the ring write of this chunk's surviving block tokens for
// head h (every candidate row of head h is read before it).
template <typename T, int DH>
__global__ __launch_bounds__(256) void block_apply_kernel(const coda_bank_desc s, BlockGeom g, const T* kbk,
                                                          const T* vbk, const float* gb,
                                                          const int32_t* __restrict__ plan_c,
                                                          const float* __restrict__ ws) {
  using E = Elt<T>;
  constexpr int NV = (DH + 63) / 64, NWV = 4;
  const int h = blockIdx.x, b = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int W = s.W, Me = s.Me, Ms = s.Ms, Hkv = s.Hkv, Te = g.Te, Ts = g.Ts, lf = s.lf, LF = DH - lf;
  const int Lbuf = W + Me + Ms;
  const int TT = max(Te, Ts);
  const int32_t* dec = reinterpret_cast<const int32_t*>(ws + CODA_WS(ws_dec, s, g)) + (int64_t)b * 3 * TT;
  const float* wtok = ws + CODA_WS(ws_wtok, s, g) + (int64_t)b * Ts;
  const int32_t* eflag = reinterpret_cast<const int32_t*>(ws + CODA_WS(ws_slot, s, g)) + (int64_t)b * (Me + 2 * Ms);
  const float* cnt = reinterpret_cast<const float*>(eflag + Me);
  const int32_t* sflag = eflag + Me + Ms;
  const int32_t* pc = plan_c + (int64_t)b * g.Kmax;
  T* kb = (T*)s.k_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;
  T* vb = (T*)s.v_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;

  if (g.n_ev > 0 && Te > 0) {
    for (int m = wv; m < Me; m += NWV) {
      if (!eflag[m]) continue;
      float nv[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lane + 64 * i;
        act[i] = d < DH;
        nv[i] = 0.f;
        if (!act[i]) continue;
        T* kr = kb + (int64_t)(W + m) * DH;
        T* vr = vb + (int64_t)(W + m) * DH;
        const float mk = E::ld(kr[d]), mv = E::ld(vr[d]);
        float ak = 0.f, av = 0.f;
        for (int tt = 0; tt < Te; ++tt) {
          if (dec[tt] != m || !(dec[TT + tt] & 1)) continue;
          const int e = pc[tt];
          ak += E::rnd(E::ld(cand_row<T, DH>(s, g, kbk, b, h, e, false)[d]) - mk);
          av += E::rnd(E::ld(cand_row<T, DH>(s, g, vbk, b, h, e, true)[d]) - mv);
        }
        kr[d] = E::st(mk + E::rnd(ak));
        nv[i] = E::rnd(mv + E::rnd(av));
        vr[d] = E::st(nv[i]);
      }
      wave_unit<T, NV>(nv, act);
      T* nr = (T*)s.exact_v_norm + (((int64_t)b * Hkv + h) * Me + m) * DH;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) nr[lane + 64 * i] = E::st(nv[i]);
    }
  }
  if (g.n_ev > 0 && Ts > 0) {
    const float eta_h = E::rnd(1.f / (1.f + expf(-s.eta_logit[h])));
    for (int m = wv; m < Ms; m += NWV) {
      const int f = sflag[m];
      if (!(f & 1)) continue;
      const float eta = (s.overwrite_on_insert && (f & 2)) ? 1.f : eta_h;
      const float den = fmaxf(cnt[m], eps_r<T>());
      T* kr = kb + (int64_t)(W + Me + m) * DH;
      T* vr = vb + (int64_t)(W + Me + m) * DH;
      float nk[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lane + 64 * i;
        act[i] = d < LF;
        nk[i] = 0.f;
        if (d >= DH) continue;
        float sv = 0.f;
        for (int tt = 0; tt < Ts; ++tt) {
          if (dec[2 * TT + tt] != m) continue;
          sv += E::rnd(E::ld(cand_row<T, DH>(s, g, vbk, b, h, pc[tt], true)[d]) * wtok[tt]);
        }
        const float mv = E::ld(vr[d]);
        const float avg_v = E::rnd(E::rnd(sv) / den);
        vr[d] = E::st(mv + E::rnd(eta * E::rnd(avg_v - mv)));
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lf + lane + 64 * i;
        if (!act[i]) continue;
        float sk = 0.f;
        for (int tt = 0; tt < Ts; ++tt) {
          if (dec[2 * TT + tt] != m) continue;
          sk += E::rnd(E::ld(cand_row<T, DH>(s, g, kbk, b, h, pc[tt], false)[d]) * wtok[tt]);
        }
        const float mk = E::ld(kr[d]);
        const float avg_k = E::rnd(E::rnd(sk) / den);
        const float dk = E::rnd(E::rnd(avg_k * s.energy_scale) - mk);
        nk[i] = E::rnd(mk + E::rnd(eta * dk));
        kr[d] = E::st(nk[i]);
      }
      wave_unit<T, NV>(nk, act);
      T* nr = (T*)s.sum_lf_k_norm + (((int64_t)b * Hkv + h) * Ms + m) * LF;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) nr[lane + 64 * i] = E::st(nk[i]);
    }
  }
  __syncthreads();
  // ring write of the surviving block tokens (combined index i >= Lr)
  uint8_t* al = s.allowed + (int64_t)b * Lbuf;
  const int Lr = g.ring_filled;
  const int first = max(Lr, g.n_ev);
  const int total = Lr + g.blk;
  const int head = (Lr == W) ? g.ring_head : 0;
  for (int i = first + wv; i < total; i += NWV) {
    const int slot = (head + i) % W;
    const int jb = i - Lr;
    const T* ks = kbk + b * g.b_sb + h * g.b_sh + (int64_t)jb * g.b_sl;
    const T* vs = vbk + b * g.b_sb + h * g.b_sh + (int64_t)jb * g.b_sl;
    for (int d = lane; d < DH; d += 64) {
      kb[(int64_t)slot * DH + d] = ks[d];
      vb[(int64_t)slot * DH + d] = vs[d];
    }
    if (h == 0 && lane == 0) {
      s.g_recent[(int64_t)b * W + slot] = gb[(int64_t)b * g.g_sb + jb];
      al[slot] = 1;
    }
  }
}

// Rotate a full ring into time order: slot s <- slot (head + s) % W.
template <typename T, int DH>
__global__ __launch_bounds__(256) void ring_rotate_kernel(const coda_bank_desc s, int head, T* tmp, float* gtmp) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int W = s.W, Lbuf = s.W + s.Me + s.Ms;
  T* kb = (T*)s.k_buf + ((int64_t)b * s.Hkv + h) * Lbuf * DH;
  T* vb = (T*)s.v_buf + ((int64_t)b * s.Hkv + h) * Lbuf * DH;
  T* tk = tmp + ((int64_t)b * s.Hkv + h) * 2 * W * DH;
  T* tv = tk + (int64_t)W * DH;
  for (int i = threadIdx.x; i < W * DH; i += 256) {
    tk[i] = kb[i];
    tv[i] = vb[i];
  }
  if (h == 0)
    for (int i = threadIdx.x; i < W; i += 256) gtmp[(int64_t)b * W + i] = s.g_recent[(int64_t)b * W + i];
  __syncthreads();
  for (int i = threadIdx.x; i < W * DH; i += 256) {
    const int slot = i / DH, d = i % DH;
    const int src = (head + slot) % W;
    kb[i] = tk[(int64_t)src * DH + d];
    vb[i] = tv[(int64_t)src * DH + d];
  }
  if (h == 0)
    for (int i = threadIdx.x; i < W; i += 256)
      s.g_recent[(int64_t)b * W + i] = gtmp[(int64_t)b * W + (head + i) % W];
}

// F.normalize of rows: x rows (o, i) at x + o*x_so + i*x_si, len channels.
template <typename T, int NV>
__global__ __launch_bounds__(256) void unit_rows_kernel(T* out, int64_t o_so, int64_t o_si, const T* x,
                                                        int64_t x_so, int64_t x_si, int64_t outer, int inner,
                                                        int len) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= outer * inner) return;
  const int64_t o = r / inner, i = r % inner;
  const T* xr = x + o * x_so + i * x_si;
  T* orow = out + o * o_so + i * o_si;
  float v[NV];
  bool act[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int d = lane + 64 * k;
    act[k] = d < len;
    v[k] = act[k] ? Elt<T>::ld(xr[d]) : 0.f;
  }
  wave_unit<T, NV>(v, act);
#pragma unroll
  for (int k = 0; k < NV; ++k)
    if (act[k]) orow[lane + 64 * k] = Elt<T>::st(v[k]);
}

// ------------------------------------------------------------ validation
// Sizes and constants only (entry points that never touch the bank data).
static int validate_sizes(const coda_bank_desc* s, const char* who) {
  CODA_REQUIRE(s != nullptr, "%s: null state descriptor", who);
  CODA_REQUIRE(s->dtype == CODA_F32 || s->dtype == CODA_BF16, "%s: dtype must be CODA_F32 or CODA_BF16", who);
  CODA_REQUIRE(s->Dh == 32 || s->Dh == 64 || s->Dh == 128, "%s: head_dim %d unsupported (32, 64, 128)", who,
               s->Dh);
  CODA_REQUIRE(s->B >= 0 && s->Hkv > 0 && s->W > 0 && s->Me >= 0 && s->Ms >= 0,
               "%s: bad sizes B=%d Hkv=%d W=%d Me=%d Ms=%d", who, s->B, s->Hkv, s->W, s->Me, s->Ms);
  CODA_REQUIRE(s->lf == s->Dh / 2, "%s: lf must be Dh/2 (got %d)", who, s->lf);
  CODA_REQUIRE(s->active_exact >= 0 && s->active_exact <= s->Me, "%s: active_exact %d outside [0, %d]", who,
               s->active_exact, s->Me);
  CODA_REQUIRE(s->active_summary >= 0 && s->active_summary <= s->Ms, "%s: active_summary %d outside [0, %d]",
               who, s->active_summary, s->Ms);
  CODA_REQUIRE(s->Me <= 1024 && s->Ms <= 1024, "%s: bank sizes above 1024 unsupported", who);
  return CODA_OK;
}

static int validate_bank(const coda_bank_desc* s, const char* who) {
  int rc = validate_sizes(s, who);
  if (rc) return rc;
  CODA_REQUIRE(s->k_buf && s->v_buf && s->allowed && s->g_recent, "%s: state buffers missing", who);
  CODA_REQUIRE(s->Me == 0 || (s->mem_last && s->exact_v_norm), "%s: exact bank buffers missing", who);
  CODA_REQUIRE(s->Ms == 0 || (s->sum_lf_k_norm && s->eta_logit), "%s: summary bank buffers missing", who);
  return CODA_OK;
}

static size_t decode_lds(const coda_bank_desc* s) {
  const int LF = s->Dh - s->lf;
  return sizeof(float) * ((size_t)s->Hkv * s->Dh * 3 + (size_t)s->Hkv * LF + (size_t)s->Hkv * (s->Me + s->Ms));
}

template <typename T, int DH>
static int launch_decode(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb,
                         int64_t nb_sh, const float* g_new, int ring_idx, int ring_filled, int64_t pos,
                         hipStream_t st) {
  const size_t lds = decode_lds(s);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)decode_write_kernel<T, DH>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(CODA_EHIP, "coda_decode_write: LDS attribute: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL((decode_write_kernel<T, DH>), dim3(s->B), dim3(512), lds, st, *s, (const T*)k_new,
                     (const T*)v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos);
  return check_launch("decode_write");
}

}  // namespace coda

using namespace coda;

extern "C" int coda_decode_write(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb,
                                 int64_t nb_sh, const float* g_new, int ring_idx, int ring_filled, int64_t pos,
                                 void* stream) {
  int rc = validate_bank(s, "coda_decode_write");
  if (rc) return rc;
  CODA_REQUIRE(k_new && v_new && g_new, "coda_decode_write: new token pointers missing");
  CODA_REQUIRE(ring_filled >= 0 && ring_filled <= s->W, "coda_decode_write: ring_filled %d outside [0, %d]",
               ring_filled, s->W);
  CODA_REQUIRE(ring_filled < s->W || (ring_idx >= 0 && ring_idx < s->W),
               "coda_decode_write: ring_idx %d outside [0, %d)", ring_idx, s->W);
  CODA_REQUIRE(decode_lds(s) <= 160 * 1024, "coda_decode_write: Hkv=%d too large for one workgroup", s->Hkv);
  if (s->B == 0) return CODA_OK;
  hipStream_t st = (hipStream_t)stream;
  const bool bf = s->dtype == CODA_BF16;
  switch (s->Dh) {
    case 32:
      return bf ? launch_decode<bf16_t, 32>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st)
                : launch_decode<float, 32>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st);
    case 64:
      return bf ? launch_decode<bf16_t, 64>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st)
                : launch_decode<float, 64>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st);
    default:
      return bf ? launch_decode<bf16_t, 128>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st)
                : launch_decode<float, 128>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st);
  }
}

extern "C" int coda_block_plan(const float* g_ring, int ring_head, int ring_filled, int W, const float* g_seq,
                               int64_t g_sb, int B, int L, int block_size, int k_exact, int k_summary, int do_exact,
                               int do_summary, int32_t* plan, int Kmax, void* stream) {
  CODA_REQUIRE(W > 0 && B >= 0 && L >= 0 && block_size > 0, "coda_block_plan: bad sizes");
  CODA_REQUIRE(ring_filled >= 0 && ring_filled <= W, "coda_block_plan: ring_filled outside [0, W]");
  CODA_REQUIRE(ring_head >= 0 && ring_head < W, "coda_block_plan: ring_head outside [0, W)");
  CODA_REQUIRE(ring_filled == W || ring_head == 0, "coda_block_plan: a partial ring must start at slot 0");
  CODA_REQUIRE(g_ring && g_seq && plan, "coda_block_plan: null pointer");
  CODA_REQUIRE(Kmax >= 1, "coda_block_plan: Kmax must be positive");
  const int K = (do_exact && do_summary) ? (k_exact > k_summary ? k_exact : k_summary)
                                         : (do_exact ? k_exact : (do_summary ? k_summary : 0));
  const int K_eff = K < block_size ? K : block_size;  // a chunk evicts at most block_size tokens
  CODA_REQUIRE(K_eff <= Kmax, "coda_block_plan: Kmax %d below candidate count %d", Kmax, K_eff);
  const int n_chunks = (L + block_size - 1) / block_size;
  if (B == 0 || n_chunks == 0 || (!do_exact && !do_summary)) return CODA_OK;
  const size_t lds = sizeof(sel::Item<float>) * (size_t)block_size;
  CODA_REQUIRE(lds <= 64 * 1024, "coda_block_plan: block_size %d too large (max 4096)", block_size);
  PlanGeom p{W, L, block_size, ring_filled, ring_head, k_exact, k_summary, do_exact, do_summary, Kmax, B};
  hipLaunchKernelGGL(block_plan_kernel, dim3(n_chunks, B), dim3(64), lds, (hipStream_t)stream, g_ring, g_seq,
                     g_sb, p, plan);
  return check_launch("block_plan");
}

static size_t block_ws_bytes(const coda_bank_desc* s, int Te, int Ts) {
  return sizeof(float) * ws_total(s->B, s->Hkv, s->Me, s->Ms, Te, Ts);
}

extern "C" int coda_block_workspace_bytes(const coda_bank_desc* s, int Kmax, size_t* bytes) {
  int rc = validate_sizes(s, "coda_block_workspace_bytes");
  if (rc) return rc;
  CODA_REQUIRE(bytes != nullptr, "coda_block_workspace_bytes: null out pointer");
  *bytes = block_ws_bytes(s, Kmax, Kmax);
  return CODA_OK;
}

template <typename T, int DH>
static int launch_block(const coda_bank_desc* s, const void* kb, const void* vb, const float* gb, BlockGeom g,
                        const int32_t* plan_c, float* ws, hipStream_t st) {
  const int LF = DH - s->lf;
  if (g.n_ev > 0 && (g.Te > 0 || g.Ts > 0)) {
    const size_t lds1 = sizeof(float) * ((size_t)g.Te * DH + (size_t)g.Ts * LF);
    const size_t lds2 = std::max(sizeof(sel::Item<int64_t>) * (size_t)s->Me +
                                     sizeof(float) * ((size_t)g.Te * s->Me + 2 * (size_t)g.Te),
                                 sizeof(float) * (size_t)g.Ts * s->Ms);
    if (lds1 > 64 * 1024 || lds2 > 64 * 1024)
      return fail(CODA_EUNSUP, "coda_block_write: candidate counts Te=%d Ts=%d too large", g.Te, g.Ts);
    hipLaunchKernelGGL((block_route_kernel<T, DH>), dim3(s->Hkv, s->B), dim3(256), lds1, st, *s, g, (const T*)kb,
                       (const T*)vb, plan_c, ws);
    int rc = check_launch("block_route");
    if (rc) return rc;
    hipLaunchKernelGGL((block_decide_kernel<T, DH>), dim3(s->B), dim3(256), lds2, st, *s, g, gb, plan_c, ws);
    rc = check_launch("block_decide");
    if (rc) return rc;
  }
  hipLaunchKernelGGL((block_apply_kernel<T, DH>), dim3(s->Hkv, s->B), dim3(256), 0, st, *s, g, (const T*)kb,
                     (const T*)vb, gb, plan_c, ws);
  return check_launch("block_apply");
}

extern "C" int coda_block_write(const coda_bank_desc* s, const void* kb, const void* vb, int64_t b_sb, int64_t b_sh,
                                int64_t b_sl, const float* gb, int64_t g_sb, int blk, int ring_head, int ring_filled,
                                int64_t pos0, const int32_t* plan_c, int Kmax, int Te, int Ts, void* workspace,
                                size_t workspace_bytes, void* stream) {
  int rc = validate_bank(s, "coda_block_write");
  if (rc) return rc;
  CODA_REQUIRE(kb && vb && gb, "coda_block_write: block pointers missing");
  CODA_REQUIRE(blk > 0, "coda_block_write: empty block");
  CODA_REQUIRE(ring_filled >= 0 && ring_filled <= s->W, "coda_block_write: ring_filled outside [0, W]");
  CODA_REQUIRE(ring_head >= 0 && ring_head < s->W && (ring_filled == s->W || ring_head == 0),
               "coda_block_write: bad ring head %d", ring_head);
  const int total = ring_filled + blk;
  const int keep_len = total < s->W ? total : s->W;
  const int n_ev = total - keep_len;
  CODA_REQUIRE(Te >= 0 && Ts >= 0 && Te <= n_ev && Ts <= n_ev, "coda_block_write: Te=%d Ts=%d exceed n_ev=%d", Te,
               Ts, n_ev);
  CODA_REQUIRE((Te == 0 || s->Me > 0) && (Ts == 0 || s->Ms > 0), "coda_block_write: candidates for an empty bank");
  CODA_REQUIRE(n_ev == 0 || (Te == 0 && Ts == 0) || (plan_c && Kmax >= (Te > Ts ? Te : Ts)),
               "coda_block_write: candidate plan missing or Kmax too small");
  const size_t need = block_ws_bytes(s, Te, Ts);
  CODA_REQUIRE(n_ev == 0 || (Te == 0 && Ts == 0) || (workspace && workspace_bytes >= need),
               "coda_block_write: workspace %zu < %zu bytes", workspace_bytes, need);
  if (s->B == 0) return CODA_OK;
  BlockGeom g{blk, ring_head, ring_filled, n_ev, Kmax, Te, Ts, pos0, b_sb, b_sh, b_sl, g_sb};
  hipStream_t st = (hipStream_t)stream;
  const bool bf = s->dtype == CODA_BF16;
  float* ws = (float*)workspace;
  switch (s->Dh) {
    case 32:
      return bf ? launch_block<bf16_t, 32>(s, kb, vb, gb, g, plan_c, ws, st)
                : launch_block<float, 32>(s, kb, vb, gb, g, plan_c, ws, st);
    case 64:
      return bf ? launch_block<bf16_t, 64>(s, kb, vb, gb, g, plan_c, ws, st)
                : launch_block<float, 64>(s, kb, vb, gb, g, plan_c, ws, st);
    default:
      return bf ? launch_block<bf16_t, 128>(s, kb, vb, gb, g, plan_c, ws, st)
                : launch_block<float, 128>(s, kb, vb, gb, g, plan_c, ws, st);
  }
}

extern "C" int coda_ring_rotate(const coda_bank_desc* s, int ring_head, void* workspace, size_t workspace_bytes,
                                void* stream) {
  int rc = validate_sizes(s, "coda_ring_rotate");
  if (rc) return rc;
  CODA_REQUIRE(s->k_buf && s->v_buf && s->g_recent, "coda_ring_rotate: state buffers missing");
  CODA_REQUIRE(ring_head >= 0 && ring_head < s->W, "coda_ring_rotate: ring_head outside [0, W)");
  const size_t esz = s->dtype == CODA_BF16 ? 2 : 4;
  const size_t need = (size_t)s->B * s->Hkv * s->W * s->Dh * 2 * esz + (size_t)s->B * s->W * sizeof(float);
  CODA_REQUIRE(workspace && workspace_bytes >= need, "coda_ring_rotate: workspace %zu < %zu bytes",
               workspace_bytes, need);
  if (s->B == 0 || ring_head == 0) return CODA_OK;
  hipStream_t st = (hipStream_t)stream;
  const size_t tmp_bytes = (size_t)s->B * s->Hkv * s->W * s->Dh * 2 * esz;
  float* gtmp = (float*)((char*)workspace + tmp_bytes);
  const dim3 grid(s->Hkv, s->B);
  const bool bf = s->dtype == CODA_BF16;
#define CODA_ROT(DH)                                                                                      \
  if (bf) hipLaunchKernelGGL((ring_rotate_kernel<bf16_t, DH>), grid, dim3(256), 0, st, *s, ring_head,   \
                             (bf16_t*)workspace, gtmp);                                                 \
  else hipLaunchKernelGGL((ring_rotate_kernel<float, DH>), grid, dim3(256), 0, st, *s, ring_head,       \
                          (float*)workspace, gtmp);
  switch (s->Dh) {
    case 32: CODA_ROT(32) break;
    case 64: CODA_ROT(64) break;
    default: CODA_ROT(128) break;
  }
#undef CODA_ROT
  return check_launch("ring_rotate");
}

// Host-side restatement check: the selection order of torch's CPU topk
// (same code the device kernels run), exported so it can be compared with
// torch.topk on a machine without a GPU.
extern "C" int coda_topk_order_host(const float* vals, int n, int k, int largest, int sorted, int64_t* out_idx) {
  CODA_REQUIRE(vals && out_idx && n >= 0 && k >= 0 && k <= n, "coda_topk_order_host: bad arguments");
  std::vector<sel::Item<float>> a((size_t)n);
  for (int i = 0; i < n; ++i) a[i] = sel::Item<float>{vals[i], (int64_t)i};
  sel::topk_order<float>(a.data(), n, k, largest != 0, sorted != 0);
  for (int i = 0; i < k; ++i) out_idx[i] = a[i].i;
  return CODA_OK;
}

extern "C" int coda_topk_order_host_i64(const int64_t* vals, int n, int k, int largest, int sorted,
                                        int64_t* out_idx) {
  CODA_REQUIRE(vals && out_idx && n >= 0 && k >= 0 && k <= n, "coda_topk_order_host_i64: bad arguments");
  std::vector<sel::Item<int64_t>> a((size_t)n);
  for (int i = 0; i < n; ++i) a[i] = sel::Item<int64_t>{vals[i], (int64_t)i};
  sel::topk_order<int64_t>(a.data(), n, k, largest != 0, sorted != 0);
  for (int i = 0; i < k; ++i) out_idx[i] = a[i].i;
  return CODA_OK;
}

extern "C" int coda_unit_rows(int dtype, void* out, int64_t o_so, int64_t o_si, const void* x, int64_t x_so,
                              int64_t x_si, int64_t outer, int inner, int len, void* stream) {
  CODA_REQUIRE(dtype == CODA_F32 || dtype == CODA_BF16, "coda_unit_rows: unsupported dtype %d", dtype);
  CODA_REQUIRE(outer >= 0 && inner >= 0 && len > 0 && len <= 128, "coda_unit_rows: bad sizes");
  CODA_REQUIRE(out && x, "coda_unit_rows: null pointer");
  const int64_t rows = outer * inner;
  if (rows == 0) return CODA_OK;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == CODA_F32)
    hipLaunchKernelGGL((unit_rows_kernel<float, 2>), grid, block, 0, st, (float*)out, o_so, o_si, (const float*)x,
                       x_so, x_si, outer, inner, len);
  else
    hipLaunchKernelGGL((unit_rows_kernel<bf16_t, 2>), grid, block, 0, st, (bf16_t*)out, o_so, o_si,
                       (const bf16_t*)x, x_so, x_si, outer, inner, len);
  return check_launch("unit_rows");
}
