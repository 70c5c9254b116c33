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
#include "bank_ops.h"
#include "common.h"
#include "select.h"

#include <math.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <mutex>
#include <vector>

namespace coda {


// ------------------------------------------------------------ decode
// One workgroup (512 threads) per sequence b: the whole update of one
// evicted token (memory_banks.py:183-432).  The two-kernel decode step
// (decode_route_kernel + the attention kernel's apply prologue) spreads
// the same work over (sequence, head) workgroups.
template <typename T, int DH>
__global__ __launch_bounds__(512) void decode_write_kernel(const coda_bank_desc s, const T* __restrict__ k_new,
                                                           const T* __restrict__ v_new, int64_t nb_sb,
                                                           int64_t nb_sh, const float* __restrict__ g_new,
                                                           int j, int filled, int64_t pos, RopeK rk) {
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
      const T* kr = kn_src + h * nb_sh;
      T kv = kr[d];
      if (rk.mode) {
        const int pi = rope_k_partner(d, DH, rk.mode), ti = rope_k_table(d, DH, rk.mode);
        kv = E::st(rope_k_elem<T>(E::ld(kv), E::ld(kr[pi]), E::ld(((const T*)rk.cs)[ti]),
                                  E::ld(((const T*)rk.sn)[ti]), d, DH, rk.mode));
      }
      kb[((int64_t)h * Lbuf + filled) * DH + d] = kv;
      vb[((int64_t)h * Lbuf + filled) * DH + d] = vn_src[h * nb_sh + d];
    }
    if (t == 0) {
      s.g_recent[(int64_t)b * W + filled] = g_new[b];
      al[filled] = 1;
    }
    return;
  }

  // LDS: ke, ve, vn [Hkv][DH]; kn [Hkv][LF]; de [Hkv][Me]; ds [Hkv][Ms];
  //      used [Me + Ms] i32; last [Me] i64
  float* ke = smem;
  float* ve = ke + Hkv * DH;
  float* vnrm = ve + Hkv * DH;
  float* knrm = vnrm + Hkv * DH;
  float* de = knrm + Hkv * LF;
  float* dsum = de + Hkv * Me;
  // int64 stamps need 8-byte alignment: both offsets are rounded to even words
  int* used = reinterpret_cast<int*>(smem + ((3 * Hkv * DH + Hkv * LF + Hkv * (Me + Ms) + 1) & ~1));
  int64_t* last = reinterpret_cast<int64_t*>(used + ((Me + Ms + 1) & ~1));
  for (int i = t; i < Hkv * DH; i += NT) {
    const int h = i / DH, d = i % DH;
    ke[i] = E::ld(kb[((int64_t)h * Lbuf + j) * DH + d]);
    ve[i] = E::ld(vb[((int64_t)h * Lbuf + j) * DH + d]);
  }
  for (int m = t; m < Me + Ms; m += NT) used[m] = al[W + m];
  for (int m = t; m < Me; m += NT) last[m] = s.mem_last[(int64_t)b * Me + m];
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
  if (wv == 0 && Me > 0) decide_exact<T>(s, de, used, last, g_e, dec, true, lane);
  if (wv == 1 && Ms > 0) decide_summary<T>(s, dsum, used + Me, g_e, dec, true, lane);
  __syncthreads();
  for (int h = wv; h < Hkv; h += NWV)
    apply_head<T, DH>(s, b, h, dec, ke + h * DH, ve + h * DH, kn_src + h * nb_sh, vn_src + h * nb_sh, j, g_e,
                      lane, nullptr, nullptr, nullptr, rk);
  if (t == 0) commit_decode_meta(s, b, dec, j, pos_e, g_new[b]);
}

// Routing kernel of the decode step: one workgroup per (head h, sequence
// b) takes head h's routing dots for evicting ring slot j; the h == 0
// workgroup also snapshots the sequence's bank metadata before any update.
template <typename T, int DH>
__global__ __launch_bounds__(256) void decode_route_kernel(const coda_bank_desc s, int j, float* ws) {
  __shared__ __attribute__((aligned(16))) float ke[DH], ve[DH], vnrm[DH], knrm[DH];
  const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int Hkv = s.Hkv, W = s.W, Me = s.Me, Ms = s.Ms;
  DStepWs w = dstep_ws(ws, b, Hkv, Me, Ms);
  if (h == 0) {
    const uint8_t* al = s.allowed + (int64_t)b * (W + Me + Ms);
    for (int m = t; m < Me + Ms; m += 256) w.used[m] = al[W + m];
    for (int m = t; m < Me; m += 256) w.last[m] = s.mem_last[(int64_t)b * Me + m];
    if (t == 0) *w.g_e = s.g_recent[(int64_t)b * W + j];
  }
  // dots layout: exact [Hkv][Me] then summary [Hkv][Ms]
  route_head_dots<T, DH>(s, b, h, j, ke, ve, vnrm, knrm, w.dots + (int64_t)h * Me,
                         w.dots + (int64_t)Hkv * Me + (int64_t)h * Ms);
}

// Bank update of one decode token from its routing record, spread over
// (head hk, sequence b) workgroups of 4 waves, followed by the routing
// record of the next token (which evicts ring slot jn = (j + 1) % W):
//   1. every load the workgroup needs is issued at once: the record of
//      sequence b, head hk's norm caches (staged in LDS), the evicted row j,
//      and the row evicted next (the new token itself when W == 1);
//   2. wave 0 takes the exact decision, wave 1 the summary decision (each
//      workgroup of a sequence recomputes the same decision from the same
//      record, so no cross-workgroup barrier is needed); waves 2-3 form the
//      unit vectors of the next evicted row;
//   3. wave 0 writes head hk's rows (exact slot, summary slot, ring slot j)
//      and patches the staged norm rows it rewrote; workgroup hk == 0 also
//      writes the sequence metadata;
//   4. all waves take the next record's dots against the staged (updated)
//      norm rows, with the per-row arithmetic of the routing kernel.
// LDS: record [words] f32 | norm stage [Me*DH + Ms*LF] T | ke, ve, vnrm, knrm [DH] f32.

// Copy nbytes (a multiple of 16) global -> LDS with direct global->LDS
// loads, spread over the waves of the workgroup: one wave instruction moves
// 1 KiB (lane l the bytes [16 l, 16 l + 16) of it).  The loads are
// asynchronous; they count in vmcnt and land before `s_waitcnt vmcnt(0)`.
__device__ __forceinline__ void wg_copy_lds(void* dst, const void* src, int nbytes) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int c = wv * 1024; c < nbytes; c += nw * 1024)
    if (c + 16 * lane < nbytes)
      __builtin_amdgcn_global_load_lds((const char*)src + c + 16 * lane,
                                       (__attribute__((address_space(3))) void*)((char*)dst + c), 16, 0, 0);
}

template <typename T, int DH>
__global__ __launch_bounds__(256) void decode_bank_kernel(const coda_bank_desc s, const T* __restrict__ k_new,
                                                          const T* __restrict__ v_new, int64_t nb_sb, int64_t nb_sh,
                                                          const float* __restrict__ g_new, int j, int64_t pos,
                                                          const float* __restrict__ rec_in,
                                                          float* __restrict__ rec_out, RopeK rk) {
  using E = Elt<T>;
  constexpr int NV = (DH + 63) / 64;
  extern __shared__ __attribute__((aligned(16))) float dsm[];
  __shared__ DecodeDecision dec;
  const int hk = blockIdx.x, b = blockIdx.y, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int Hkv = s.Hkv, W = s.W, Me = s.Me, Ms = s.Ms, lf = s.lf, LF = DH - lf;
  const int Lbuf = W + Me + Ms;
  const int words = dstep_words(Hkv, Me, Ms);
  const int jn = j + 1 == W ? 0 : j + 1;
  float* rec = dsm;
  T* stage = reinterpret_cast<T*>(rec + words);
  float* ke = reinterpret_cast<float*>(stage + dbank_stage_elems(DH, Me, Ms, lf));
  float* ve = ke + DH;
  float* vnrm = ve + DH;
  float* knrm = vnrm + DH;
  const DStepWs L = dstep_ws(rec, 0, Hkv, Me, Ms);
  const int64_t plane = ((int64_t)b * Hkv + hk) * Lbuf;
  const T* kn_row = k_new + b * nb_sb + hk * nb_sh;
  const T* vn_row = v_new + b * nb_sb + hk * nb_sh;

  // ---- 1. loads
  wg_copy_lds(rec, rec_in + (int64_t)b * words, words * 4);
  if (Me > 0)
    wg_copy_lds(stage, (const T*)s.exact_v_norm + ((int64_t)b * Hkv + hk) * Me * DH, Me * DH * (int)sizeof(T));
  if (Ms > 0)
    wg_copy_lds(stage + Me * DH, (const T*)s.sum_lf_k_norm + ((int64_t)b * Hkv + hk) * Ms * LF,
                Ms * LF * (int)sizeof(T));
  const T* kr = (const T*)s.k_buf + (plane + j) * DH;
  const T* vr = (const T*)s.v_buf + (plane + j) * DH;
  for (int d = t; d < DH; d += 256) {
    ke[d] = E::ld(kr[d]);
    ve[d] = E::ld(vr[d]);
  }
  // the row evicted next: waves 2 (V, full) and 3 (K, LF band) hold it in registers
  const T* kx = jn == j ? kn_row : (const T*)s.k_buf + (plane + jn) * DH;
  const T* vx = jn == j ? vn_row : (const T*)s.v_buf + (plane + jn) * DH;
  float xn[NV];
  bool an[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = lane + 64 * i;
    an[i] = wv == 2 ? d < DH : d < LF;
    const int dc = an[i] ? d : 0;
    xn[i] = (wv >= 2 && an[i]) ? E::ld(wv == 2 ? vx[dc] : kx[lf + dc]) : 0.f;
    if (wv == 3 && an[i] && jn == j && rk.mode) {
      // a one-slot ring: the token evicted next is this raw new K, roped
      const int dd = lf + dc, pi = rope_k_partner(dd, DH, rk.mode), ti = rope_k_table(dd, DH, rk.mode);
      xn[i] = rope_k_elem<T>(xn[i], E::ld(kx[pi]), E::ld(((const T*)rk.cs)[ti]), E::ld(((const T*)rk.sn)[ti]), dd,
                             DH, rk.mode);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the direct LDS loads have landed
  __syncthreads();
  // ---- 2. decisions / next unit vectors
  const float g_e = *L.g_e;
  if (wv == 0 && Me > 0) decide_exact<T>(s, L.dots, L.used, L.last, g_e, dec, hk == 0, lane);
  if (wv == 1 && Ms > 0) decide_summary<T>(s, L.dots + Hkv * Me, L.used + Me, g_e, dec, hk == 0, lane);
  if ((wv == 2 && Me > 0) || (wv == 3 && Ms > 0)) {
    wave_unit<T, NV>(xn, an);
    float* dst = wv == 2 ? vnrm : knrm;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (an[i]) dst[lane + 64 * i] = xn[i];
  }
  __syncthreads();
  // ---- 3. row writes of head hk, metadata
  if (wv == 0)
    apply_head<T, DH>(s, b, hk, dec, ke, ve, kn_row, vn_row, j, g_e, lane, Me > 0 ? stage + dec.idx_e * DH : nullptr,
                      Ms > 0 ? stage + Me * DH + dec.idx_s * LF : nullptr, nullptr, rk);
  if (wv == 1 && hk == 0) {
    // metadata of the sequence, and the next record's snapshot of it
    const DStepWs wn = dstep_ws(rec_out, b, Hkv, Me, Ms);
    const bool ow_e = Me > 0 && dec.ow_e, keep_e = Me > 0 && dec.keep_e, keep_s = Ms > 0 && dec.keep_s;
    const int ie = Me > 0 ? dec.idx_e : -1, is = Ms > 0 ? dec.idx_s : -1;
    for (int m = lane; m < Me + Ms; m += 64)
      wn.used[m] = L.used[m] | ((ow_e && m == ie) || (keep_s && m == Me + is) ? 1 : 0);
    for (int m = lane; m < Me; m += 64) wn.last[m] = (keep_e && m == ie) ? pos - W : L.last[m];
    if (lane == 0) {
      *wn.g_e = jn == j ? g_new[b] : s.g_recent[(int64_t)b * W + jn];
      commit_decode_meta(s, b, dec, j, pos - W, g_new[b]);
    }
  }
  __syncthreads();
  // ---- 4. next record: head hk's dots against the updated norm rows
  float* out_e = rec_out + (int64_t)b * words + (int64_t)hk * Me;
  float* out_s = rec_out + (int64_t)b * words + (int64_t)Hkv * Me + (int64_t)hk * Ms;
  // (one lane per dot: exact rows on waves 0-1, summary rows on waves 2-3)
  if (Me > 0 && wv < 2)
    wave_dots<T>(
        Me, DH, wv, 2, lane, [&](int it) { return (const T*)stage + it * DH; }, [&](int) { return (const float*)vnrm; },
        [&](int it, float v) { out_e[it] = v; });
  if (Ms > 0 && wv >= 2)
    wave_dots<T>(
        Ms, LF, wv - 2, 2, lane, [&](int it) { return (const T*)stage + Me * DH + it * LF; },
        [&](int) { return (const float*)knrm; }, [&](int it, float v) { out_s[it] = v; });
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
// A chunk is one launch of block_fused_kernel (below) when its working set
// fits in LDS; otherwise four launches:
//   route  grid (Hkv + 1, B, nz): workgroups h < Hkv normalise a share of
//          head h's candidate rows and take their cosine dots with the
//          head's norm caches (staged in LDS); workgroup Hkv snapshots the
//          pre-update bank metadata of sequence b (used bits, LRU stamps,
//          candidate gates) and computes the LRU victim order.
//   decide grid (1 + ceil(Ts / kDecideChunk), B): workgroup 0 takes the
//          exact decisions of sequence b (and commits its LRU stamps), the
//          others route kDecideChunk summary candidates each (head-mean
//          scores, first-occurrence argmax, token weights).
//   apply  grid (Hkv, B, nz): workgroup (h, b, z) applies the decisions to
//          its share of head h's slots (exact delta write-back, summary
//          accumulate + EMA, norm caches); (0, b, 0) also writes the
//          per-sequence metadata.
//   ring   grid (Hkv, B, nzr): the chunk's surviving tokens into the ring,
//          after the bank writes have read the evicted ring rows.
// Workspace (4-byte words), TT = max(Te, Ts):
//   dot_e [B][Hkv][Te][Me] f32, dot_s [B][Hkv][Ts][Ms] f32,
//   snap  [B][SNAP]: used (Me+Ms) i32 | last (Me) i64 | gate (TT) f32 | lru (Me) i32,
//   dec   [B][DEC]: decisions (block_decide_kernel; the fused kernel's
//         per-token routing),
//   sync  [B][64] u64: the fused kernel's sync flags.
struct BlockGeom {
  int blk, ring_head, ring_filled, n_ev, Kmax, Te, Ts;
  int64_t pos0;
  int64_t b_sb, b_sh, b_sl, g_sb;
};
// Where the one-launch update copies the bank slots it stages (the state
// before the chunk's update): K / V (B, Hkv, Me + Ms, Dh), visibility
// bytes (B, Me + Ms); k == nullptr: no copy.
struct BankSnap {
  void* k;
  void* v;
  uint8_t* allowed;
};

__host__ __device__ __forceinline__ int even_up(int x) { return (x + 1) & ~1; }
__host__ __device__ __forceinline__ int snap_words(int Me, int Ms, int TT) {
  return even_up(even_up(Me + Ms) + 2 * Me + TT + Me);
}
__host__ __device__ __forceinline__ size_t ws_dot_s(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return (size_t)B * Hkv * Te * Me;
}
__host__ __device__ __forceinline__ size_t ws_snap(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return (ws_dot_s(B, Hkv, Me, Ms, Te, Ts) + (size_t)B * Hkv * Ts * Ms + 1) & ~(size_t)1;  // 8-byte aligned
}
__host__ __device__ __forceinline__ int dec_words(int Me, int Te, int Ts);
// sync flags of the fused kernel: 64 64-bit words per sequence, 8-byte aligned
__host__ __device__ __forceinline__ size_t ws_sync(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return (ws_snap(B, Hkv, Me, Ms, Te, Ts) + (size_t)B * snap_words(Me, Ms, Te > Ts ? Te : Ts) +
          (size_t)B * dec_words(Me, Te, Ts) + 1) & ~(size_t)1;
}
__host__ __device__ __forceinline__ size_t ws_total(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return ws_sync(B, Hkv, Me, Ms, Te, Ts) + 128 * (size_t)B + 2;
}
#define CODA_WS(fn, s, g) fn((s).B, (s).Hkv, (s).Me, (s).Ms, (g).Te, (g).Ts)

struct Snap {
  int32_t* used;
  int64_t* last;
  float* gate;
  int32_t* lru;
};
__device__ __forceinline__ Snap snap_of(const coda_bank_desc& s, const BlockGeom& g, float* ws, int b) {
  const int TT = max(g.Te, g.Ts);
  int32_t* base = reinterpret_cast<int32_t*>(ws + CODA_WS(ws_snap, s, g)) + (int64_t)b * snap_words(s.Me, s.Ms, TT);
  Snap sn;
  sn.used = base;
  // int64 stamps at an 8-byte aligned word offset: the snap area starts at
  // an even word and (Me + Ms) may be odd, so stamps follow a pad word
  sn.last = reinterpret_cast<int64_t*>(base + even_up(s.Me + s.Ms));
  sn.gate = reinterpret_cast<float*>(base + even_up(s.Me + s.Ms) + 2 * s.Me);
  sn.lru = base + even_up(s.Me + s.Ms) + 2 * s.Me + TT;
  return sn;
}

// Source row of evicted candidate e (index into the chunk's time-ordered
// [ring | block] sequence) for KV head h: ring slot or block token.
template <typename T, int DH>
__device__ __forceinline__ const T* cand_row(const coda_bank_desc& s, const BlockGeom& g, const T* kbk, int b,
                                             int h, int e, bool value) {
  const int Lbuf = s.W + s.Me + s.Ms;
  if (e < g.ring_filled) {
    int slot = e;
    if (g.ring_filled == s.W) {  // circular ring: e < W and ring_head < W, one wrap at most
      slot = g.ring_head + e;
      slot -= slot >= s.W ? s.W : 0;
    }
    const T* buf = (const T*)(value ? s.v_buf : s.k_buf);
    return buf + (((int64_t)b * s.Hkv + h) * Lbuf + slot) * DH;
  }
  return kbk + b * g.b_sb + h * g.b_sh + (int64_t)(e - g.ring_filled) * g.b_sl;
}

// Where candidate e's gate is (ring slot or block token), without a load.
__device__ __forceinline__ const float* cand_gate_ptr(const coda_bank_desc& s, const BlockGeom& g, const float* gb,
                                                      int b, int e) {
  int slot = e;
  if (g.ring_filled == s.W) {
    slot = g.ring_head + e;
    slot -= slot >= s.W ? s.W : 0;
  }
  return e < g.ring_filled ? s.g_recent + (int64_t)b * s.W + slot : gb + (int64_t)b * g.g_sb + (e - g.ring_filled);
}
__device__ __forceinline__ float cand_gate(const coda_bank_desc& s, const BlockGeom& g, const float* gb, int b,
                                           int e) {
  if (e < g.ring_filled) {
    int slot = e;
    if (g.ring_filled == s.W) {
      slot = g.ring_head + e;
      slot -= slot >= s.W ? s.W : 0;
    }
    return s.g_recent[(int64_t)b * s.W + slot];
  }
  return gb[(int64_t)b * g.g_sb + (e - g.ring_filled)];
}

// Rows x cands dots from LDS, 4 x 4 register blocks, each a chain of fused
// multiply-adds in the CPU matmul order (dot_pair: channel pairs in
// increasing order, odd channel first); result rounded to the element type
// (the matmul output dtype).
template <typename T, int RB, int CB, bool SC = false>
__device__ __forceinline__ void lds_dots_blk(const float* rows, int n_rows, const float* cands, int n_c, int len,
                                             int stride, float* out /* [n_c][n_rows] */) {
  const int nbr = (n_rows + RB - 1) / RB, nbc = (n_c + CB - 1) / CB;
  for (int blk = threadIdx.x; blk < nbr * nbc; blk += blockDim.x) {
    const int r0 = RB * (blk % nbr), c0 = CB * (blk / nbr);
    float acc[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) acc[i][j] = 0.f;
#pragma unroll 2
    for (int d = 0; d < len; d += 4) {
      float4 rv[RB], cv[CB];
#pragma unroll
      for (int i = 0; i < RB; ++i) rv[i] = *reinterpret_cast<const float4*>(rows + min(r0 + i, n_rows - 1) * stride + d);
#pragma unroll
      for (int j = 0; j < CB; ++j) cv[j] = *reinterpret_cast<const float4*>(cands + min(c0 + j, n_c - 1) * stride + d);
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) {
          acc[i][j] = dot_pair(acc[i][j], cv[j].x, rv[i].x, cv[j].y, rv[i].y);
          acc[i][j] = dot_pair(acc[i][j], cv[j].z, rv[i].z, cv[j].w, rv[i].w);
        }
    }
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j)
        if (r0 + i < n_rows && c0 + j < n_c) {
          if constexpr (SC)  // coherent at agent scope: read by workgroups on other XCDs in this launch
            __hip_atomic_store(out + (c0 + j) * n_rows + r0 + i, Elt<T>::rnd(acc[i][j]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          else
            out[(c0 + j) * n_rows + r0 + i] = Elt<T>::rnd(acc[i][j]);
        }
  }
}
// out[c][r] = rnd(dot(cands[c], rows[r])), each an fma chain over the
// channel pairs in order (the same value whatever the blocking); blocks of
// 4 x 4 dots per thread when there are enough of them, else 2 x 1
template <typename T, bool SC = false>
__device__ __forceinline__ void lds_dots(const float* rows, int n_rows, const float* cands, int n_c, int len,
                                         int stride, float* out /* [n_c][n_rows] */) {
  if (((n_rows + 3) / 4) * ((n_c + 3) / 4) >= (int)blockDim.x)
    lds_dots_blk<T, 4, 4, SC>(rows, n_rows, cands, n_c, len, stride, out);
  else
    lds_dots_blk<T, 2, 1, SC>(rows, n_rows, cands, n_c, len, stride, out);
}

// Stage `n` rows of `len` elements (row stride `rs` elements) into LDS fp32
// with row stride `ls` floats; 16-byte loads, 8 per thread in flight
// before their stores.
template <typename T>
__device__ __forceinline__ void stage_rows(float* dst, int ls, const T* src, int64_t rs, int n, int len) {
  const int chunks = len >> 3, nt = blockDim.x, total = n * chunks;
  for (int base = threadIdx.x; base < total; base += 8 * nt) {
    float x[8][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = min(base + u * nt, total - 1);
      load8f<T>(src + (i / chunks) * rs + 8 * (i % chunks), x[u]);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * nt;
      if (i < total) {
        float4* d = reinterpret_cast<float4*>(dst + (i / chunks) * ls + 8 * (i % chunks));
        d[0] = make_float4(x[u][0], x[u][1], x[u][2], x[u][3]);
        d[1] = make_float4(x[u][4], x[u][5], x[u][6], x[u][7]);
      }
    }
  }
}

// Normalised candidate rows into LDS: each wave takes 8 rows at a time,
// loads all of them, then normalises them one by one.
template <typename T, int DH>
__device__ __forceinline__ void stage_cands(float* dst, int ls, const coda_bank_desc& s, const BlockGeom& g,
                                            const T* src_blk, const int32_t* pc, int b, int h, int n, int off,
                                            int len, bool value) {
  constexpr int NV = (DH + 63) / 64, RB = 8;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  bool act[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) act[i] = lane + 64 * i < len;
  for (int r0 = wv * RB; r0 < n; r0 += nw * RB) {
    float x[RB][NV];
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const int r = min(r0 + u, n - 1);
      const T* row = cand_row<T, DH>(s, g, src_blk, b, h, pc[r], value);
#pragma unroll
      for (int i = 0; i < NV; ++i) x[u][i] = act[i] ? Elt<T>::ld(row[off + lane + 64 * i]) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      if (r0 + u >= n) break;
      wave_unit<T, NV>(x[u], act);
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) dst[(r0 + u) * ls + lane + 64 * i] = x[u][i];
    }
  }
}

// The chunk's candidates of head h, normalised (F.normalize, rounded as the
// reference) into LDS, rows [r_lo, r_hi) of the concatenated list (the Te
// exact candidates, then the Ts summary candidates): exact candidates as V
// rows (all DH channels) into dst_e from candidate e_lo = min(r_lo, Te) on,
// summary candidates as LF-K bands (channels lf ..) into dst_s from
// candidate max(r_lo - Te, 0) on.  Every wave takes rows r_lo + wv + nw u;
// all plan indices of a pass load first, then all candidate rows, then the
// normalisation.
template <typename T, int DH>
__device__ __forceinline__ void stage_cands_both(float* dst_e, int le, float* dst_s, int lsum, const coda_bank_desc& s,
                                                 const BlockGeom& g, const T* vbk, const T* kbk, const int32_t* pc,
                                                 int b, int h, int r_lo, int r_hi) {
  constexpr int NV = (DH + 63) / 64, RB = 12;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int Te = g.Te, n = r_hi, lf = s.lf, LF = DH - lf;
  const int e_lo = min(r_lo, Te), s_lo = max(r_lo - Te, 0);
  for (int r0 = r_lo; r0 < n; r0 += nw * RB) {
    int idx[RB];
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const int r = min(r0 + wv + nw * u, n - 1);
      idx[u] = pc[r < Te ? r : r - Te];
    }
    float x[RB][NV];
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const int r = min(r0 + wv + nw * u, n - 1);
      const bool ex = r < Te;
      const T* row = cand_row<T, DH>(s, g, ex ? vbk : kbk, b, h, idx[u], ex) + (ex ? 0 : lf);
      const int len = ex ? DH : LF;
#pragma unroll
      for (int i = 0; i < NV; ++i) x[u][i] = lane + 64 * i < len ? Elt<T>::ld(row[lane + 64 * i]) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const int r = r0 + wv + nw * u;
      if (r >= n) break;
      const bool ex = r < Te;
      const int len = ex ? DH : LF;
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) act[i] = lane + 64 * i < len;
      wave_unit<T, NV>(x[u], act);
      float* dst = ex ? dst_e + (r - e_lo) * le : dst_s + (r - Te - s_lo) * lsum;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) dst[lane + 64 * i] = x[u][i];
    }
  }
}

template <typename T, int DH>
__global__ __launch_bounds__(256) void block_route_kernel(const coda_bank_desc s, BlockGeom g, const T* kbk,
                                                          const T* vbk, const float* gb,
                                                          const int32_t* __restrict__ plan_c, float* ws) {
  extern __shared__ __attribute__((aligned(16))) float rsm[];
  const int h = blockIdx.x, b = blockIdx.y, z = blockIdx.z, t = threadIdx.x;
  const int Me = s.Me, Ms = s.Ms, W = s.W, LF = DH - s.lf;
  const int32_t* pc = plan_c + (int64_t)b * g.Kmax;
  if (h == s.Hkv) {
    if (z != 0) return;
    Snap sn = snap_of(s, g, ws, b);
    const uint8_t* al = s.allowed + (int64_t)b * (W + Me + Ms);
    for (int m = t; m < Me + Ms; m += blockDim.x) sn.used[m] = al[W + m];
    for (int m = t; m < Me; m += blockDim.x) sn.last[m] = s.mem_last[(int64_t)b * Me + m];
    const int TT = max(g.Te, g.Ts);
    for (int i = t; i < TT; i += blockDim.x) sn.gate[i] = cand_gate(s, g, gb, b, pc[i]);
    if (g.Te > 0) {
      sel::Item<int64_t>* rk = reinterpret_cast<sel::Item<int64_t>*>(rsm);
      const int Ae = act_exact(s);
      for (int m = t; m < Me; m += blockDim.x) {
        const bool u = al[W + m] != 0 && m < Ae;
        rk[m] = sel::Item<int64_t>{u ? s.mem_last[(int64_t)b * Me + m] : kNegBig, (int64_t)m};
      }
      __shared__ int ties;
      if (t == 0) ties = 0;
      __syncthreads();
      const int n_lru = min(g.Te, Ae);
      // Keys that reach the first n_lru places with no equal key: the
      // sorted topk order is their rank order, whatever the algorithm
      // (the usual case once the bank is full: LRU stamps are distinct).
      for (int m = t; m < Me; m += blockDim.x) {
        const int64_t km = rk[m].v;
        int lt = 0, eq = 0;
        for (int j = 0; j < Me; ++j) {
          const int64_t kj = rk[j].v;
          lt += kj < km;
          eq += (kj == km) & (j != m);
        }
        if (lt < n_lru) {
          if (eq) atomicOr(&ties, 1);
          else sn.lru[lt] = m;
        }
      }
      __syncthreads();
      // ties among the leading keys: their order is libstdc++'s
      if (ties) {
        if (t == 0) sel::topk_order<int64_t>(rk, Me, n_lru, false, true);
        __syncthreads();
        for (int r = t; r < n_lru; r += blockDim.x) sn.lru[r] = (int32_t)rk[r].i;
      }
    }
    return;
  }
  // workgroup z takes rows [r_lo, r_hi) of the concatenated candidate list
  // (exact then summary), so the dots of one (sequence, head) spread over
  // gridDim.z workgroups; each dot is formed as with one workgroup
  const int n = g.Te + g.Ts, per = (n + (int)gridDim.z - 1) / (int)gridDim.z;
  const int r_lo = z * per, r_hi = min(n, r_lo + per);
  if (r_lo >= r_hi) return;
  const int e_lo = min(r_lo, g.Te), ne = min(r_hi, g.Te) - e_lo;
  const int s_lo = max(r_lo - g.Te, 0), ns = max(r_hi - g.Te, 0) - s_lo;
  // LDS: exact norm rows [Me][DH+4] | exact candidates [ne][DH+4] |
  //      summary norm rows [Ms][LF+4] | summary candidates [ns][LF+4]
  const int le = DH + 4, lsum = LF + 4;
  float* nrm_e = rsm;
  float* cnd_e = nrm_e + (ne > 0 ? Me * le : 0);
  float* nrm_s = cnd_e + ne * le;
  float* cnd_s = nrm_s + (ns > 0 ? Ms * lsum : 0);
  if (ne > 0) stage_rows<T>(nrm_e, le, (const T*)s.exact_v_norm + ((int64_t)b * s.Hkv + h) * Me * DH, DH, Me, DH);
  if (ns > 0)
    stage_rows<T>(nrm_s, lsum, (const T*)s.sum_lf_k_norm + ((int64_t)b * s.Hkv + h) * Ms * LF, LF, Ms, LF);
  stage_cands_both<T, DH>(cnd_e, le, cnd_s, lsum, s, g, vbk, kbk, pc, b, h, r_lo, r_hi);
  __syncthreads();
  if (ne > 0)
    lds_dots<T>(nrm_e, Me, cnd_e, ne, DH, le, ws + (((int64_t)b * s.Hkv + h) * g.Te + e_lo) * Me);
  if (ns > 0)
    lds_dots<T>(nrm_s, Ms, cnd_s, ns, LF, lsum,
                ws + CODA_WS(ws_dot_s, s, g) + (((int64_t)b * s.Hkv + h) * g.Ts + s_lo) * Ms);
}

// Decision record of a chunk, per sequence (4-byte words), written by
// block_decide_kernel and read by block_apply_kernel:
//   idx_e [Te] i32 | fl_e [Te] i32 (1 overwrite, 2 touch) | eflag [Me] i32 |
//   idx_s [Ts] i32 | wtok [Ts] f32
__host__ __device__ __forceinline__ int dec_words(int Me, int Te, int Ts) { return even_up(2 * Te + Me + 2 * Ts); }
__host__ __device__ __forceinline__ size_t ws_dec(int B, int Hkv, int Me, int Ms, int Te, int Ts) {
  return ws_snap(B, Hkv, Me, Ms, Te, Ts) + (size_t)B * snap_words(Me, Ms, Te > Ts ? Te : Ts);
}
struct Dec {
  int32_t* idx_e;
  int32_t* fl_e;
  int32_t* eflag;
  int32_t* idx_s;
  float* wtok;
};
__device__ __forceinline__ Dec dec_of(const coda_bank_desc& s, const BlockGeom& g, float* ws, int b) {
  int32_t* base = reinterpret_cast<int32_t*>(ws + CODA_WS(ws_dec, s, g)) + (int64_t)b * dec_words(s.Me, g.Te, g.Ts);
  Dec d;
  d.idx_e = base;
  d.fl_e = base + g.Te;
  d.eflag = base + 2 * g.Te;
  d.idx_s = base + 2 * g.Te + s.Me;
  d.wtok = reinterpret_cast<float*>(base + 2 * g.Te + s.Me + g.Ts);
  return d;
}

// Summary candidates per decide workgroup.
static constexpr int kDecideChunk = 8;

// Decisions of one chunk (memory_banks.py:640-697 exact, :866-878 summary).
// Workgroup x == 0: exact decisions of sequence b from the per-head dots
// and the metadata snapshot (LRU stamps are committed here, the only
// writer); x >= 1: summary routing of candidates [8 (x-1), 8 x).
template <typename T>
__global__ __launch_bounds__(256) void block_decide_kernel(const coda_bank_desc s, BlockGeom g,
                                                           const int32_t* __restrict__ plan_c, float* ws) {
  using E = Elt<T>;
  extern __shared__ __attribute__((aligned(16))) float dsm2[];
  __shared__ float best[kDecideChunk > 64 ? kDecideChunk : 64];
  __shared__ int best_i[kDecideChunk > 64 ? kDecideChunk : 64];
  const int x = blockIdx.x, b = blockIdx.y, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int Me = s.Me, Ms = s.Ms, Hkv = s.Hkv, Te = g.Te, Ts = g.Ts, W = s.W;
  const Snap sn = snap_of(s, g, ws, b);
  const Dec dc = dec_of(s, g, ws, b);
  if (x == 0) {
    if (Te == 0) return;
    // the per-head dots stay in global memory (read once each, coalesced
    // over slots), so LDS does not grow with the number of heads
    const float* dg = ws + (int64_t)b * Hkv * Te * Me;  // [Hkv][Te][Me]
    int* used = reinterpret_cast<int*>(dsm2);           // [Me]
    int* idx_l = used + Me;                             // [Te]
    int* fl_l = idx_l + Te;                             // [Te]
    for (int m = t; m < Me; m += blockDim.x) used[m] = sn.used[m];
    __syncthreads();
    __shared__ int any_used_s;
    if (wv == 0) {
      int u = 0;
      for (int m = lane; m < Me; m += 64) u |= used[m] != 0;
      u = wave_or(u);
      if (lane == 0) any_used_s = u;
    }
    // candidates 64 at a time: the best slot of each (one wave per
    // candidate), then thread 0 walks them in token order, its rank and
    // counters carried from chunk to chunk
    const int Ae = act_exact(s);
    const int n_lru = min(Te, Ae);
    int rank = -1;
    int64_t cnt_ow = 0, cnt_cap = 0, cnt_hit = 0, cnt_gated = 0, cnt_fr = 0;
    for (int c0 = 0; c0 < Te; c0 += 64) {
      const int cn = min(64, Te - c0);
      for (int k = wv; k < cn; k += blockDim.x >> 6) {
        const int tt = c0 + k;
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int m = lane; m < Me; m += 64) {
          // head mean in head order (the reference's mean over heads)
          float acc = 0.f;
          for (int hh = 0; hh < Hkv; ++hh) acc += dg[((int64_t)hh * Te + tt) * Me + m];
          float v = E::rnd(acc / (float)Hkv);
          if (m >= Ae || used[m] == 0) v = neg_fill<T>();
          if (v > bv || (v == bv && m < bi)) { bv = v; bi = m; }
        }
        wave_argmax(bv, bi);
        if (lane == 0) { best[k] = bv; best_i[k] = bi; }
      }
      __syncthreads();
      if (t == 0) {
        const int any_used = any_used_s;
        for (int k = 0; k < cn; ++k) {
          const int tt = c0 + k;
          const bool keep = s.gated ? (sn.gate[tt] >= s.tau_exact) : true;
          const float bv = best[k];
          const bool novel = !any_used || bv < E::rnd(s.tau_novel);
          const bool hit = any_used && bv >= E::rnd(s.tau_match);
          const bool nk = novel && keep;
          if (nk) ++rank;  // cumsum(novel & keep) - 1 at tt
          const bool cap = nk && rank < Ae;
          int idx = best_i[k];
          if (cap) {
            int r = rank < 0 ? 0 : rank;
            if (r > n_lru - 1) r = n_lru - 1;
            idx = sn.lru[r];
          }
          const bool touch = keep && (!novel || cap);
          const bool ow = s.refresh_on_hit ? (keep && (cap || hit)) : cap;
          idx_l[tt] = idx;
          fl_l[tt] = (ow ? 1 : 0) | (touch ? 2 : 0);
          cnt_ow += ow;
          cnt_cap += cap;
          cnt_hit += (hit && keep);
          cnt_gated += !keep;
          cnt_fr += (nk && !cap);
        }
      }
      __syncthreads();
    }
    if (t == 0) {
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
    int32_t* tr = s.trace ? s.trace + (int64_t)b * (2 * Te + Ts) : nullptr;
    for (int tt = t; tt < Te; tt += blockDim.x) {
      dc.idx_e[tt] = idx_l[tt];
      dc.fl_e[tt] = fl_l[tt];
      if (tr) {
        tr[tt] = idx_l[tt];
        tr[Te + tt] = fl_l[tt];
      }
    }
    const int32_t* pc = plan_c + (int64_t)b * g.Kmax;
    for (int m = t; m < Me; m += blockDim.x) {
      int f = 0;
      bool tm = false;
      int64_t pv = kNegBig;
      for (int tt = 0; tt < Te; ++tt) {
        if (idx_l[tt] != m) continue;
        f |= fl_l[tt] & 1;
        if (fl_l[tt] & 2) {
          tm = true;
          const int64_t p = g.pos0 - g.ring_filled + pc[tt];
          if (p > pv) pv = p;
        }
      }
      dc.eflag[m] = f;
      if (tm) s.mem_last[(int64_t)b * Me + m] = pv;  // LRU: max pos of the touching tokens
    }
    return;
  }
  // ---- summary routing of candidates [t0, t0 + nt)
  const int t0 = (x - 1) * kDecideChunk;
  const int nt = min(kDecideChunk, Ts - t0);
  if (nt <= 0) return;
  // per-head dots read from global memory (coalesced over slots)
  const float* dsd = ws + CODA_WS(ws_dot_s, s, g) + (int64_t)b * Hkv * Ts * Ms;  // [Hkv][Ts][Ms]
  for (int tt = wv; tt < nt; tt += blockDim.x >> 6) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    const int As = act_summary(s);
    for (int m = lane; m < Ms; m += 64) {
      float acc = 0.f;
      for (int hh = 0; hh < Hkv; ++hh) acc += dsd[((int64_t)hh * Ts + t0 + tt) * Ms + m];
      float v = E::rnd(acc / (float)Hkv);
      if (m >= As) v = neg_fill<T>();
      if (v > bv || (v == bv && m < bi)) { bv = v; bi = m; }
    }
    wave_argmax(bv, bi);
    if (lane == 0) {
      dc.idx_s[t0 + tt] = bi;
      if (s.trace) s.trace[(int64_t)b * (2 * Te + Ts) + 2 * Te + t0 + tt] = bi;
      const float gate = sn.gate[t0 + tt];
      dc.wtok[t0 + tt] = (!s.gated || gate >= s.tau_summary) ? E::rnd(gate) : 0.f;
    }
  }
}

// Bank writes of one chunk from the decisions (memory_banks.py:707-742
// exact write-back, :880-932 summary accumulate + EMA).  Workgroup (h, b, z)
// owns the exact slots [z pe, (z + 1) pe) and the summary slots [z PS,
// (z + 1) PS) of head h, so one (sequence, head) spreads over gridDim.z
// workgroups; candidate values are read where they lie (ring slots or block
// rows, not yet overwritten: the ring write is block_ring_kernel, launched
// after this one).  Each summary slot keeps the list of its tokens in token
// order, so one thread per (active slot, channel) sums the slot's weighted
// tokens in registers (fp32, token order: the scatter_add order) and
// applies the EMA in the same pass.  Workgroup (0, b, 0) also writes the
// per-sequence metadata (visibility bytes of written slots, counters).
// LDS (4-byte words): idx_e, fl_e [Te] | idx_s, wtok [Ts] | token lists
//      [PS][Ts] | nlist, cnt, sflag, act_list [PS] | new LF keys [PS][LF] |
//      summary flags of every slot [Ms] | misc [8].
static constexpr int kApplyThreads = 512;
static constexpr int kRingPre = 8;   // 16-byte ring-write chunks per thread loaded up front

__host__ __device__ __forceinline__ size_t apply_lds_bytes(int Ms, int Te, int Ts, int PS, int LF) {
  return 4 * ((size_t)2 * Te + 2 * Ts + (size_t)PS * Ts + 4 * PS + (size_t)PS * LF + Ms + 8);
}

// Eight consecutive elements moved as raw bits: PW 16-byte words.
template <typename T>
struct Piece8 {
  static constexpr int PW = sizeof(T) / 2;
  uint4 w[PW];
};
template <typename T>
__device__ __forceinline__ Piece8<T> ld8(const T* p) {
  Piece8<T> x;
#pragma unroll
  for (int i = 0; i < Piece8<T>::PW; ++i) x.w[i] = reinterpret_cast<const uint4*>(p)[i];
  return x;
}
template <typename T>
__device__ __forceinline__ void st8(T* p, const Piece8<T> x) {
#pragma unroll
  for (int i = 0; i < Piece8<T>::PW; ++i) reinterpret_cast<uint4*>(p)[i] = x.w[i];
}
// A piece into an LDS row of the fused update's norm caches (bf16 rows are
// only 8-byte aligned there), and four values of such a row widened to fp32.
template <typename T>
__device__ __forceinline__ void st8_row(T* p, const Piece8<T> x) {
  if constexpr (sizeof(T) == 2) {
    reinterpret_cast<uint2*>(p)[0] = make_uint2(x.w[0].x, x.w[0].y);
    reinterpret_cast<uint2*>(p)[1] = make_uint2(x.w[0].z, x.w[0].w);
  } else {
    st8<T>(p, x);
  }
}
template <typename T>
__device__ __forceinline__ float4 ld4_row(const T* p) {
  if constexpr (sizeof(T) == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(bf2f((bf16_t)(u.x & 0xffffu)), bf2f((bf16_t)(u.x >> 16)), bf2f((bf16_t)(u.y & 0xffffu)),
                       bf2f((bf16_t)(u.y >> 16)));
  } else {
    return *reinterpret_cast<const float4*>(p);
  }
}
// The eight values of a piece as floats.
template <typename T>
__device__ __forceinline__ void piece8_f(const Piece8<T>& x, float f[8]) {
#pragma unroll
  for (int q = 0; q < Piece8<T>::PW; ++q) {
    const uint32_t w[4] = {x.w[q].x, x.w[q].y, x.w[q].z, x.w[q].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (sizeof(T) == 2) {
        f[2 * i] = bf2f((bf16_t)(w[i] & 0xffffu));
        f[2 * i + 1] = bf2f((bf16_t)(w[i] >> 16));
      } else {
        f[4 * q + i] = __builtin_bit_cast(float, w[i]);
      }
    }
  }
}

template <typename T, int DH>
__global__ __launch_bounds__(kApplyThreads) void block_apply_kernel(const coda_bank_desc s, BlockGeom g, const T* kbk,
                                                                    const T* vbk, const int32_t* __restrict__ plan_c,
                                                                    float* ws) {
  using E = Elt<T>;
  constexpr int NV = (DH + 63) / 64, LF = DH / 2, NCOL = DH + LF;
  extern __shared__ __attribute__((aligned(16))) float asm_[];
  const int h = blockIdx.x, b = blockIdx.y, z = blockIdx.z, nz = gridDim.z;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, NT = blockDim.x, NW = NT >> 6;
  const int W = s.W, Me = s.Me, Ms = s.Ms, Hkv = s.Hkv, Te = g.Te, Ts = g.Ts, lf = s.lf;
  const int Lbuf = W + Me + Ms;
  T* kb = (T*)s.k_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;
  T* vb = (T*)s.v_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;
  uint8_t* al = s.allowed + (int64_t)b * Lbuf;
  const int32_t* pc = plan_c + (int64_t)b * g.Kmax;
  const int pe = (Me + nz - 1) / nz, e0 = min(Me, z * pe), e1 = min(Me, e0 + pe);
  const int PS = (Ms + nz - 1) / nz, s0 = min(Ms, z * PS), s1 = min(Ms, s0 + PS), nsl = s1 - s0;
  int32_t* idx_e = reinterpret_cast<int32_t*>(asm_);
  int32_t* fl_e = idx_e + Te;
  int32_t* idx_s = fl_e + Te;
  float* wtok = reinterpret_cast<float*>(idx_s + Ts);
  int32_t* list = reinterpret_cast<int32_t*>(wtok + Ts);  // [PS][Ts]
  int32_t* nlist = list + (size_t)PS * Ts;
  float* cnt = reinterpret_cast<float*>(nlist + PS);
  int32_t* sflag = reinterpret_cast<int32_t*>(cnt + PS);
  int32_t* act_list = sflag + PS;
  float* knew = reinterpret_cast<float*>(act_list + PS);  // [PS][LF]
  int32_t* fl_all = reinterpret_cast<int32_t*>(knew + (size_t)PS * LF);
  int32_t* misc = fl_all + Ms;
  const Snap sn = snap_of(s, g, ws, b);
  const Dec dc = dec_of(s, g, ws, b);
  for (int i = t; i < Te; i += NT) { idx_e[i] = dc.idx_e[i]; fl_e[i] = dc.fl_e[i]; }
  for (int i = t; i < Ts; i += NT) { idx_s[i] = dc.idx_s[i]; wtok[i] = dc.wtok[i]; }
  __syncthreads();
  // tokens of summary slot m in order (into lst when given), their count
  // k and weight sum (fp32 in token order; adding 0 for other slots'
  // tokens leaves the sum unchanged); tokens read 16 at a time
  auto slot_scan = [&](int m, int32_t* lst, int& k) {
    float c = 0.f;
    k = 0;
    for (int t0 = 0; t0 < Ts; t0 += 16) {
      int iv[16];
      float w16[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int tt = min(t0 + u, Ts - 1);
        iv[u] = t0 + u < Ts ? idx_s[tt] : -1;
        w16[u] = wtok[tt];
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const bool on = iv[u] == m;
        c += on ? w16[u] : 0.f;
        if (on && lst) lst[k] = t0 + u;
        k += on ? 1 : 0;
      }
    }
    return E::rnd(c);
  };
  if (Ts > 0) {
    for (int j = t; j < nsl; j += NT) {
      const int m = s0 + j;
      int k;
      const float c = slot_scan(m, list + (size_t)j * Ts, k);
      nlist[j] = k;
      cnt[j] = c;
      const bool active = c > 0.f;
      sflag[j] = (active ? 1 : 0) | ((active && sn.used[Me + m] == 0) ? 2 : 0);
    }
  }
  // ---- exact write-back of this workgroup's slots (memory_banks.py:707-742):
  // one wave per written slot, deltas summed in token order
  if (Te > 0) {
    for (int m = e0 + wv; m < e1; m += NW) {
      if (!dc.eflag[m]) continue;
      T* kr = kb + (int64_t)(W + m) * DH;
      T* vr = vb + (int64_t)(W + m) * DH;
      float mk[NV], mv[NV], ak[NV], av[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = min(lane + 64 * i, DH - 1);
        mk[i] = E::ld(kr[d]);
        mv[i] = E::ld(vr[d]);
        ak[i] = 0.f;
        av[i] = 0.f;
      }
      for (int tt = 0; tt < Te; ++tt) {
        if (idx_e[tt] != m || !(fl_e[tt] & 1)) continue;
        const T* ck = cand_row<T, DH>(s, g, kbk, b, h, pc[tt], false);
        const T* cv = cand_row<T, DH>(s, g, vbk, b, h, pc[tt], true);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int d = min(lane + 64 * i, DH - 1);
          ak[i] += E::rnd(E::ld(ck[d]) - mk[i]);
          av[i] += E::rnd(E::ld(cv[d]) - mv[i]);
        }
      }
      float nv[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lane + 64 * i;
        act[i] = d < DH;
        nv[i] = 0.f;
        if (act[i]) {
          kr[d] = E::st(mk[i] + E::rnd(ak[i]));
          nv[i] = E::rnd(mv[i] + E::rnd(av[i]));
          vr[d] = E::st(nv[i]);
        }
      }
      wave_unit<T, NV>(nv, act);
      T* nr = (T*)s.exact_v_norm + (((int64_t)b * Hkv + h) * Me + m) * DH;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) nr[lane + 64 * i] = E::st(nv[i]);
    }
  }
  if (Ts > 0) {
    __syncthreads();
    // active slots, compacted in slot order by wave 0 (ballot prefix counts)
    if (wv == 0) {
      int na = 0;
      for (int j0 = 0; j0 < nsl; j0 += 64) {
        const int j = j0 + lane;
        const bool on = j < nsl && (sflag[j] & 1);
        const uint64_t bal = __ballot(on);
        if (on) act_list[na + __popcll(bal & ((1ull << lane) - 1ull))] = j;
        na += __popcll(bal);
      }
      if (lane == 0) misc[0] = na;
    }
    __syncthreads();
    // ---- accumulate + EMA: thread (group q, channel col) takes the active
    // slots q, q + NG, ...; 8 slots at a time, their metadata and the
    // values of their first token read before any arithmetic; further
    // tokens of a slot (rare) follow in token order (fp32 sum)
    const int n_act = misc[0];
    const float eta_h = s.eta[h];
    constexpr int NG = kApplyThreads / NCOL, SB = 8;
    const int q = t / NCOL, col = t % NCOL;
    if (q < NG) {
      const bool is_v = col < DH;
      const int d = is_v ? col : lf + (col - DH);
      T* rbase = (is_v ? vb : kb) + (int64_t)(W + Me) * DH + d;
      // token tt's value at this channel: V (channel col) or K (channel lf + col - DH)
      auto tok = [&](int tt) { return E::ld(cand_row<T, DH>(s, g, is_v ? vbk : kbk, b, h, pc[tt], is_v)[d]); };
      for (int a0 = q; a0 < n_act; a0 += NG * SB) {
        int jj[SB], nk[SB], fl[SB], t0[SB];
        float cn[SB];
#pragma unroll
        for (int j = 0; j < SB; ++j) jj[j] = act_list[min(a0 + NG * j, n_act - 1)];
#pragma unroll
        for (int j = 0; j < SB; ++j) {
          nk[j] = nlist[jj[j]];
          fl[j] = sflag[jj[j]];
          cn[j] = cnt[jj[j]];
          t0[j] = list[(size_t)jj[j] * Ts];
        }
        float x0[SB], w0[SB], mem[SB];
#pragma unroll
        for (int j = 0; j < SB; ++j) {
          x0[j] = tok(t0[j]);
          w0[j] = wtok[t0[j]];
          mem[j] = E::ld(rbase[(int64_t)(s0 + jj[j]) * DH]);
        }
#pragma unroll
        for (int j = 0; j < SB; ++j) {
          if (a0 + NG * j >= n_act) break;
          const int jl = jj[j], m = s0 + jl;
          float a = E::rnd(x0[j] * w0[j]);
          for (int k = 1; k < nk[j]; ++k) {
            const int tt = list[(size_t)jl * Ts + k];
            a += E::rnd(tok(tt) * wtok[tt]);
          }
          const float eta = (s.overwrite_on_insert && (fl[j] & 2)) ? 1.f : eta_h;
          const float avg = E::rnd(E::rnd(a) / fmaxf(cn[j], eps_r<T>()));
          if (is_v) {
            rbase[(int64_t)m * DH] = E::st(mem[j] + E::rnd(eta * E::rnd(avg - mem[j])));
          } else {
            const float dk = E::rnd(E::rnd(avg * s.energy_scale) - mem[j]);
            const float nkv = E::rnd(mem[j] + E::rnd(eta * dk));
            rbase[(int64_t)m * DH] = E::st(nkv);
            knew[jl * LF + (col - DH)] = nkv;  // new LF key for the norm cache
          }
        }
      }
    }
    __syncthreads();
    for (int ai = wv; ai < n_act; ai += NW) {
      const int jl = act_list[ai], m = s0 + jl;
      float x[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int dd = lane + 64 * i;
        act[i] = dd < LF;
        x[i] = act[i] ? knew[jl * LF + dd] : 0.f;
      }
      wave_unit<T, NV>(x, act);
      T* nr = (T*)s.sum_lf_k_norm + (((int64_t)b * Hkv + h) * Ms + m) * LF;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) nr[lane + 64 * i] = E::st(x[i]);
    }
  }
  // ---- per-sequence metadata (one workgroup per sequence)
  if (h == 0 && z == 0) {
    for (int m = t; m < Me; m += NT)
      if (Te > 0 && dc.eflag[m]) al[W + m] = 1;
    if (Ts > 0) {
      for (int m = t; m < Ms; m += NT) {
        int k;
        const bool active = slot_scan(m, nullptr, k) > 0.f;
        fl_all[m] = (active ? 1 : 0) | ((active && sn.used[Me + m] == 0) ? 2 : 0);
        if (active) al[W + Me + m] = 1;
      }
      __syncthreads();
      if (wv == 0) {
        int64_t upd = 0, ins = 0;
        int all_used = 1, any_cnt = 0;
        const int As = act_summary(s);
        for (int m = lane; m < Ms; m += 64) {
          const int f = fl_all[m];
          upd += f & 1;
          ins += (f >> 1) & 1;
          if (m < As) {
            if (!(sn.used[Me + m] != 0 || (f & 1))) all_used = 0;
            if (f & 1) any_cnt = 1;
          }
        }
        for (int o = 32; o > 0; o >>= 1) {
          upd += __shfl_xor(upd, o, 64);
          ins += __shfl_xor(ins, o, 64);
        }
        all_used = wave_and(all_used);
        any_cnt = wave_or(any_cnt);
        if (lane == 0) {
          if (s.metrics) {
            atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_UPDATES, upd);
            if (s.overwrite_on_insert) atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_INSERTS, ins);
          }
          if (s.frustrated) {
            if (!all_used) atomic_add_i64(s.frustrated + 1, 1);
            if (any_cnt) atomic_add_i64(s.frustrated + 2, 1);
          }
        }
      }
    }
  }
}

// Ring write of the chunk's surviving block tokens (memory_banks.py:135-177)
// for head h of sequence b, after the bank writes have read the evicted
// ring rows; the lead head also writes the ring gates and visibility bytes.
// Workgroup z takes the 16-byte pieces [z per, (z + 1) per) of the copy.
template <typename T, int DH>
__global__ __launch_bounds__(kApplyThreads) void block_ring_kernel(const coda_bank_desc s, BlockGeom g, const T* kbk,
                                                                   const T* vbk, const float* gb) {
  constexpr int CH = DH / 8;
  const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x, NT = blockDim.x;
  const int W = s.W, Lbuf = W + s.Me + s.Ms;
  const bool lead = h == 0;
  T* kb = (T*)s.k_buf + ((int64_t)b * s.Hkv + h) * Lbuf * DH;
  T* vb = (T*)s.v_buf + ((int64_t)b * s.Hkv + h) * Lbuf * DH;
  uint8_t* al = s.allowed + (int64_t)b * Lbuf;
  auto blk_row = [&](const T* base, int jb) { return base + b * g.b_sb + h * g.b_sh + (int64_t)jb * g.b_sl; };
  const int Lr = g.ring_filled;
  const int first = max(Lr, g.n_ev);
  const int total = Lr + g.blk;
  const int rhead = (Lr == W) ? g.ring_head : 0;
  const int n_all = (total - first) * CH;  // pieces of 8 elements per plane (K and V each)
  const int per = (n_all + (int)gridDim.z - 1) / (int)gridDim.z;
  const int p0 = min(n_all, (int)blockIdx.z * per), n_ring = min(n_all, p0 + per);
  auto ring_store = [&](int i, Piece8<T> xk, Piece8<T> xv) {
    const int r = first + i / CH, c = i % CH;
    const int slot = (rhead + r) % W;
    st8<T>(kb + (int64_t)slot * DH + 8 * c, xk);
    st8<T>(vb + (int64_t)slot * DH + 8 * c, xv);
    if (lead && c == 0) {
      s.g_recent[(int64_t)b * W + slot] = gb[(int64_t)b * g.g_sb + (r - Lr)];
      al[slot] = 1;
    }
  };
  for (int base = p0 + t; base < n_ring; base += kRingPre * NT) {
    Piece8<T> rk[kRingPre], rv[kRingPre];
#pragma unroll
    for (int u = 0; u < kRingPre; ++u) {
      const int i = base + u * NT;
      if (i < n_ring) {
        const int jb = first + i / CH - Lr, c = i % CH;
        rk[u] = ld8<T>(blk_row(kbk, jb) + 8 * c);
        rv[u] = ld8<T>(blk_row(vbk, jb) + 8 * c);
      }
    }
#pragma unroll
    for (int u = 0; u < kRingPre; ++u)
      if (base + u * NT < n_ring) ring_store(base + u * NT, rk[u], rv[u]);
  }
}

// ------------------------------------------------------------ fused block write
// The chunk's whole bank update in one launch when its working set fits in
// LDS: NZ workgroups per (sequence b, head h), with the routing rows, bank
// slots and ring pieces of head h split over them.  Workgroup (h, z, b):
//   1. stages the raw K and V rows of the chunk's candidates for head h
//      (the plan's first max(Te, Ts) tokens: the exact candidates are the
//      first Te, the summary candidates the first Ts), its own bank slots,
//      the norm caches its routing rows need, and the sequence's bank
//      metadata (used bits, LRU stamps, candidate gates, LRU victim order);
//   2. normalises its share of the routing rows (exact candidates z, z +
//      NZ, ... as V rows, summary candidates z, z + NZ, ... as LF-K
//      bands) and forms their dots with head h's norm caches (the CPU
//      matmul order) into the workspace;
//   -- sync 1 of the Hkv * NZ workgroups of b (meanwhile: the LRU order) --
//   3. routes the tokens it is assigned (token i of [Te | Ts] goes to
//      workgroup i mod (Hkv * NZ)): head-mean of the dots, first-occurrence
//      argmax, published to the workspace;
//   -- sync 2 (meanwhile: its share of head h's ring) --
//   4. reads every token's routing, takes the exact decisions (the same
//      serial walk, from the same values, in every workgroup) and applies
//      them and the summary routing to its own slots of head h (exact delta
//      write-back, summary accumulate + EMA, norm caches).
// Workgroup (0, 0, b) (the lead) commits what the sequence shares: LRU stamps,
// visibility bytes, ring gates, counters and the decision trace, after
// sync 1 (every workgroup has read them by then).
// Sync: every workgroup of b stores (2 epoch + k) at sync k in its own
// 64-bit flag word of the workspace and waits until all flags of b reach
// it; the epoch is unique per launch, so no word needs clearing.  The epoch
// of sequence b mixes the host's per-call value with a generation word of
// b kept in the workspace's tail, which the lead workgroup advances once
// every workgroup of b has passed sync 2 (so all of them read the same
// value first): a launch replayed from a captured graph, whose host value
// is fixed, still meets its own sync words and never a stale one.  What
// crosses a sync (dots, routing) is written and read with agent-scope
// atomic accesses (coherent across the XCDs' L2s, no cache write-back or
// invalidation), and a workgroup's flag is stored only after all its
// waves' such stores have completed.  A workgroup waits on workgroups of b
// only; they lie in one contiguous range of launch order (with whole other
// sequences at most, at most 64 workgroups), dispatched after every earlier
// range: one that waits never holds back one it waits for.  Waits are
// bounded (spin_limit sleeps, about 0.1 s by default); a workgroup that
// gives up counts itself in g_block_sync_timeouts and in the workspace's
// status word, and exits without writing any more state (the chunk's
// update is then incomplete: the caller reads the status word and must
// treat the state as lost).
static constexpr int kFusedThreads = 512;
static constexpr int kFusedMaxGroup = 64;  // Hkv * NZ: one wave polls every flag of a sequence
static constexpr int kSyncSpinLimit = 1 << 20;
static __device__ unsigned int g_block_sync_timeouts;

// Sync of the K workgroups of one sequence (see above).  While wave 0
// polls, waves 1 .. hold `busy`: work that needs nothing from the other
// workgroups (it sees thread ids from 0 and a stride of blockDim - 64).
// Returns true, in every thread, when the wait gave up (spin_limit < 0:
// at once, without polling: the host's way to take the failure path).
template <typename F>
__device__ __forceinline__ bool group_sync(unsigned long long* flags, int K, int me, unsigned long long val,
                                           unsigned long long alt, int spin_limit, unsigned long long* status,
                                           int* gave_up, F&& busy) {
  // this wave's coherent stores complete, then the workgroup's
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(flags + me, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    for (int n = 0;; ++n) {
      if (n > spin_limit) {
        if (lane == 0) {
          atomicAdd(&g_block_sync_timeouts, 1u);
          __hip_atomic_fetch_add(status, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          *gave_up = 1;
        }
        break;
      }
      bool ok = true;
      if (lane < K) {
        const unsigned long long v = __hip_atomic_load(flags + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = v == val || v == alt;
      }
      if (__all(ok)) break;
      __builtin_amdgcn_s_sleep(2);
    }
  } else {
    busy((int)threadIdx.x - 64, (int)blockDim.x - 64);
  }
  __syncthreads();
  return *gave_up != 0;
}

struct FusedLds {
  int raw_k, raw_v, own_ek, own_ev, own_sv, own_sk, gate, used, last, rk, lru, pc, idx_e, fl_e, bv_e, bi_e, idx_s,
      wtok, eflag, smask, scnt, sflag, knew, ov, total;
};
__host__ __device__ __forceinline__ int al16(int x) { return (x + 15) & ~15; }
__host__ __device__ __forceinline__ FusedLds fused_lds(int DH, int esz, int Me, int Ms, int Te, int Ts, int NZ) {
  const int TT = Te > Ts ? Te : Ts, LF = DH / 2;
  const int PE = (Me + NZ - 1) / NZ, PS = (Ms + NZ - 1) / NZ;
  const int ne = (Te + NZ - 1) / NZ, ns = (Ts + NZ - 1) / NZ;
  FusedLds L;
  int o = 0;
  L.raw_k = o; o += al16(TT * DH * esz);
  L.raw_v = o; o += al16(TT * DH * esz);
  L.own_ek = o; o += al16(PE * DH * esz);
  L.own_ev = o; o += al16(PE * DH * esz);
  L.own_sv = o; o += al16(PS * DH * esz);
  L.own_sk = o; o += al16(PS * DH * esz);
  L.gate = o; o += al16(4 * TT);
  L.used = o; o += al16(4 * (Me + Ms));
  L.last = o; o += al16(8 * Me);
  L.rk = o; o += al16(16 * Me);
  L.lru = o; o += al16(4 * Me);
  L.pc = o; o += al16(4 * TT);
  L.idx_e = o; o += al16(4 * Te);
  L.fl_e = o; o += al16(4 * Te);
  L.bv_e = o; o += al16(4 * Te);
  L.bi_e = o; o += al16(4 * Te);
  L.idx_s = o; o += al16(4 * Ts);
  L.wtok = o; o += al16(4 * Ts);
  L.eflag = o; o += al16(4 * Me);
  L.smask = o; o += al16(8 * Ms);
  L.scnt = o; o += al16(4 * Ms);
  L.sflag = o; o += al16(4 * Ms);
  L.knew = o; o += al16(4 * PS * LF);
  L.ov = o;
  // routing rows: head h's norm caches in the element type (widened as the
  // dots read them) and this workgroup's normalised rows in fp32
  L.total = o + al16(Me * (DH + 4) * esz) + al16(4 * ne * (DH + 4)) + al16(Ms * (LF + 4) * esz) +
            al16(4 * ns * (LF + 4));
  return L;
}

template <typename T, int DH>
__global__ __launch_bounds__(kFusedThreads) void block_fused_kernel(const coda_bank_desc s, BlockGeom g, int NZ,
                                                                    const T* kbk, const T* vbk, const float* gb,
                                                                    const int32_t* __restrict__ plan_c, float* ws,
                                                                    unsigned long long* flags_all,
                                                                    unsigned long long host_epoch,
                                                                    unsigned long long* tail, int spin_limit,
                                                                    BankSnap snap) {
  using E = Elt<T>;
  constexpr int NV = (DH + 63) / 64, LF = DH / 2, NCOL = DH + LF, CH = DH / 8;
  extern __shared__ __attribute__((aligned(16))) char fsm[];
  __shared__ int ties, sync_gave_up;
  // workgroup -> (sequence, head, z): workgroups are dealt round robin to
  // the 8 XCDs, so the NZ workgroups of one (sequence, head) pair take
  // consecutive turns of one XCD (they share its L2); the workgroups of a
  // sequence still fill one contiguous range of launch order
  const int xcd = blockIdx.x & 7, turn = blockIdx.x >> 3;
  const int pair = (turn / NZ) * 8 + xcd, z = turn % NZ;
  const int b = pair / s.Hkv, h = pair % s.Hkv;
  if (b >= s.B) return;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, NT = blockDim.x, NW = NT >> 6;
  const int W = s.W, Me = s.Me, Ms = s.Ms, Hkv = s.Hkv, Te = g.Te, Ts = g.Ts;
  const int TT = max(Te, Ts), Lbuf = W + Me + Ms, K = Hkv * NZ, me = h * NZ + z;
  const bool lead = me == 0;
  const int Ae = act_exact(s), As = act_summary(s), n_lru = min(Te, Ae);
  const FusedLds L = fused_lds(DH, (int)sizeof(T), Me, Ms, Te, Ts, NZ);
  T* raw_k = reinterpret_cast<T*>(fsm + L.raw_k);    // [TT][DH] candidate K rows of head h
  T* raw_v = reinterpret_cast<T*>(fsm + L.raw_v);    // [TT][DH] candidate V rows
  T* own_ek = reinterpret_cast<T*>(fsm + L.own_ek);  // [PE][DH] own exact slots: K
  T* own_ev = reinterpret_cast<T*>(fsm + L.own_ev);  // V
  T* own_sv = reinterpret_cast<T*>(fsm + L.own_sv);  // [PS][DH] own summary slots: V
  T* own_sk = reinterpret_cast<T*>(fsm + L.own_sk);  // [PS][DH] own summary slots: K
  float* gate = reinterpret_cast<float*>(fsm + L.gate);
  int32_t* used = reinterpret_cast<int32_t*>(fsm + L.used);
  int64_t* last = reinterpret_cast<int64_t*>(fsm + L.last);
  sel::Item<int64_t>* rk = reinterpret_cast<sel::Item<int64_t>*>(fsm + L.rk);
  int32_t* lru = reinterpret_cast<int32_t*>(fsm + L.lru);
  int32_t* pcl = reinterpret_cast<int32_t*>(fsm + L.pc);
  int32_t* idx_e = reinterpret_cast<int32_t*>(fsm + L.idx_e);
  int32_t* fl_e = reinterpret_cast<int32_t*>(fsm + L.fl_e);
  float* bv_e = reinterpret_cast<float*>(fsm + L.bv_e);
  int32_t* bi_e = reinterpret_cast<int32_t*>(fsm + L.bi_e);
  int32_t* idx_s = reinterpret_cast<int32_t*>(fsm + L.idx_s);
  float* wtok = reinterpret_cast<float*>(fsm + L.wtok);
  int32_t* eflag = reinterpret_cast<int32_t*>(fsm + L.eflag);
  uint64_t* smask = reinterpret_cast<uint64_t*>(fsm + L.smask);
  float* scnt = reinterpret_cast<float*>(fsm + L.scnt);
  int32_t* sflag = reinterpret_cast<int32_t*>(fsm + L.sflag);
  float* knew = reinterpret_cast<float*>(fsm + L.knew);  // [PS][LF]
  const int le = DH + 4, lsum = LF + 4;
  // this workgroup's routing rows: exact candidates e = z, z + NZ, ... and
  // summary candidates z, z + NZ, ... (every workgroup forms both kinds)
  const int ne = z < Te ? (Te - z + NZ - 1) / NZ : 0, ns = z < Ts ? (Ts - z + NZ - 1) / NZ : 0;
  // (rows of le / lsum elements: 8-byte aligned in bf16, 16-byte in fp32,
  // and 2 (bf16) or 4 (fp32) banks apart from row to row)
  constexpr int ES = (int)sizeof(T);
  char* ovp = fsm + L.ov;
  T* nrm_e = reinterpret_cast<T*>(ovp);                                               // [Me][le]
  ovp += ne > 0 ? al16(Me * le * ES) : 0;
  float* cnd_e = reinterpret_cast<float*>(ovp);                                       // [ne][le]
  ovp += al16(4 * ne * le);
  T* nrm_s = reinterpret_cast<T*>(ovp);                                               // [Ms][lsum]
  ovp += ns > 0 ? al16(Ms * lsum * ES) : 0;
  float* cnd_s = reinterpret_cast<float*>(ovp);                                       // [ns][lsum]
  // this workgroup's bank slots of head h
  const int PE = (Me + NZ - 1) / NZ, e0 = min(Me, z * PE), e1 = min(Me, e0 + PE);
  const int PS = (Ms + NZ - 1) / NZ, s0 = min(Ms, z * PS), s1 = min(Ms, s0 + PS);
  T* kb = (T*)s.k_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;
  T* vb = (T*)s.v_buf + ((int64_t)b * Hkv + h) * Lbuf * DH;
  uint8_t* al = s.allowed + (int64_t)b * Lbuf;
  const int32_t* pc = plan_c + (int64_t)b * g.Kmax;
  unsigned long long* flags = flags_all + (int64_t)b * K;
  // epoch of this launch for sequence b: the host value mixed with b's
  // generation word (tail[b]); tail[B] is the status word
  unsigned long long* status = tail + s.B;
  if (t == 0) sync_gave_up = 0;
  const Dec dx = dec_of(s, g, ws, b);  // exchange: idx_s [Ts], best value / slot of the exact tokens
  const int Lr = g.ring_filled, first = max(Lr, g.n_ev), rhead = (Lr == W) ? g.ring_head : 0;

  // ---- 1. staging in one batch of loads: the plan entries behind this
  // thread's candidate pieces first, then plan, metadata, own bank slots
  // and norm caches, then the candidate rows and gates through those plan
  // entries (their wait covers only the entries), then every LDS store
  {
    constexpr int UR = 2;  // pieces of each kind per thread and round
    constexpr int CHL = LF / 8;
    const int n_raw = TT * CH, n_us = Me + Ms, n_ee = (e1 - e0) * CH, n_ss = (s1 - s0) * CH;
    const int n_ne = ne > 0 ? Me * CH : 0, n_ns = ns > 0 ? Ms * CHL : 0;
    const int n_rnd = max(max(max(n_raw, TT), max(n_us, n_ee)), max(max(n_ss, n_ne), n_ns));
    const T* nre = (const T*)s.exact_v_norm + ((int64_t)b * Hkv + h) * Me * DH;
    const T* nrs = (const T*)s.sum_lf_k_norm + ((int64_t)b * Hkv + h) * Ms * LF;
    for (int base = t; base < n_rnd; base += UR * NT) {
      int32_t rr[UR], vpc[UR];
      uint32_t vus[UR];
      int64_t vla[UR];
      Piece8<T> vek[UR], vev[UR], vsv[UR], vsk[UR], vne[UR], vns[UR], vrk[UR], vrv[UR];
      float vg[UR];
      // every load unconditional, from a clamped index or (an empty array)
      // the workspace: the compiler then counts the loads in flight and
      // waits for the plan entries alone before the candidate rows, where a
      // load under a branch makes it wait for everything
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int i = base + u * NT;
        rr[u] = pc[min(i, n_raw - 1) / CH];
      }
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int i = base + u * NT;
        vpc[u] = pc[min(i, TT - 1)];
        vus[u] = al[W + min(i, n_us - 1)];
        vla[u] = *(Me > 0 ? s.mem_last + (int64_t)b * Me + min(i, Me - 1) : reinterpret_cast<const int64_t*>(ws));
        {
          const int ic = min(i, max(n_ee, 1) - 1), r = ic / CH, c = ic % CH;
          const int64_t o = (int64_t)(W + e0 + r) * DH + 8 * c;
          vek[u] = ld8<T>(n_ee > 0 ? kb + o : reinterpret_cast<const T*>(ws));
          vev[u] = ld8<T>(n_ee > 0 ? vb + o : reinterpret_cast<const T*>(ws));
        }
        {
          const int ic = min(i, max(n_ss, 1) - 1), r = ic / CH, c = ic % CH;
          const int64_t o = (int64_t)(W + Me + s0 + r) * DH + 8 * c;
          vsv[u] = ld8<T>(n_ss > 0 ? vb + o : reinterpret_cast<const T*>(ws));
          vsk[u] = ld8<T>(n_ss > 0 ? kb + o : reinterpret_cast<const T*>(ws));
        }
        vne[u] = ld8<T>(n_ne > 0 ? nre + 8 * (int64_t)min(i, n_ne - 1) : reinterpret_cast<const T*>(ws));
        vns[u] = ld8<T>(n_ns > 0 ? nrs + 8 * (int64_t)min(i, n_ns - 1) : reinterpret_cast<const T*>(ws));
      }
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int i = base + u * NT;
        const int c = min(i, n_raw - 1) % CH;
        vrk[u] = ld8<T>(cand_row<T, DH>(s, g, kbk, b, h, rr[u], false) + 8 * c);
        vrv[u] = ld8<T>(cand_row<T, DH>(s, g, vbk, b, h, rr[u], true) + 8 * c);
        vg[u] = *cand_gate_ptr(s, g, gb, b, rr[u]);
      }
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int i = base + u * NT;
        if (i < TT) pcl[i] = vpc[u];
        if (i < n_us) used[i] = (int32_t)(vus[u] & 0xffu);
        if (i < Me) last[i] = vla[u];
        if (i < n_ee) {
          const int r = i / CH, c = i % CH;
          st8<T>(own_ek + r * DH + 8 * c, vek[u]);
          st8<T>(own_ev + r * DH + 8 * c, vev[u]);
        }
        if (i < n_ss) {
          const int r = i / CH, c = i % CH;
          st8<T>(own_sv + r * DH + 8 * c, vsv[u]);
          st8<T>(own_sk + r * DH + 8 * c, vsk[u]);
        }
        if (i < n_ne) st8_row<T>(nrm_e + (i / CH) * le + 8 * (i % CH), vne[u]);
        if (i < n_ns) st8_row<T>(nrm_s + (i / CHL) * lsum + 8 * (i % CHL), vns[u]);
        if (i < n_raw) {
          st8<T>(raw_k + 8 * i, vrk[u]);
          st8<T>(raw_v + 8 * i, vrv[u]);
          if (i % CH == 0) gate[i / CH] = vg[u];
        }
      }
    }
  }
  // b's generation word, first used at sync 1: loaded after the staging
  // loop (a load pending at a loop's head is waited for there), through a
  // lane-varying zero in the address, which keeps it in a vector register (a
  // uniform load is copied to a scalar register, and waited for, at once)
  const int lane0 = (int)__builtin_amdgcn_mbcnt_lo(0u, 0u);
  const unsigned long long gen_b =
      __hip_atomic_load(tail + b + lane0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  // LRU keys over the pre-update stamps (memory_banks.py:640-660):
  // ascending stamps of used active slots, unused ones first
  if (Te > 0)
    for (int m = t; m < Me; m += NT) {
      const bool u = used[m] != 0 && m < Ae;
      rk[m] = sel::Item<int64_t>{u ? last[m] : kNegBig, (int64_t)m};
    }
  if (t == 0) ties = 0;
  __syncthreads();
  // ---- 2. this workgroup's routing rows, normalised (exact: V, all DH
  // channels; summary: K channels [DH/2, DH)), then their dots with head
  // h's norm caches, one dot per thread (lanes over bank slots)
  for (int r = wv; r < ne + ns; r += NW) {
    const bool ex = r < ne;
    const int k = ex ? r : r - ne, c = z + k * NZ;
    float x[NV];
    bool act[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      act[i] = ex ? d < DH : (d >= LF && d < DH);
      x[i] = E::ld((ex ? raw_v : raw_k)[c * DH + min(d, DH - 1)]);
    }
    if (ex) {
      wave_unit<T, NV>(x, act);
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) cnd_e[k * le + lane + 64 * i] = x[i];
    } else {
      wave_unit<T, NV, LF>(x, act);
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) cnd_s[k * lsum + lane + 64 * i - LF] = x[i];
    }
  }
  __syncthreads();
  {
    float* dot_e = ws + ((int64_t)b * Hkv + h) * Te * Me;
    float* dot_s = ws + CODA_WS(ws_dot_s, s, g) + ((int64_t)b * Hkv + h) * Ts * Ms;
    const int n_e = ne * Me, n_s = ns * Ms, n_all = n_e + n_s;
    // each dot is one serial chain (DH or DH/2 steps): the exact dots take
    // the last n_e threads alone, the summary dots the others, so that no
    // thread chains an exact dot after a summary one (when n_e <= NT / 2)
    const bool split = n_e > 0 && 2 * n_e <= NT;
    const int ns_thr = split ? NT - n_e : NT;
    const int it0 = split ? (t >= ns_thr ? n_s + (t - ns_thr) : t) : t;
    const int step = split ? (t >= ns_thr ? n_all : ns_thr) : NT;
    for (int it1 = it0; it1 < (split && t < ns_thr ? n_s : n_all); it1 += step) {
      // item order: [exact | summary] in the unsplit case, [summary | exact] in the split one
      const int it = split ? (it1 < n_s ? n_e + it1 : it1 - n_s) : it1;
      const bool ex = it < n_e;
      const int k = ex ? it / Me : (it - n_e) / Ms, m = ex ? it % Me : (it - n_e) % Ms;
      const T* rw = ex ? nrm_e + m * le : nrm_s + m * lsum;
      const float* cd = ex ? cnd_e + k * le : cnd_s + k * lsum;
      const int len = ex ? DH : LF;
      float acc = 0.f;
#pragma unroll 4
      for (int d = 0; d < len; d += 4) {
        const float4 rv = ld4_row<T>(rw + d);
        const float4 cv = *reinterpret_cast<const float4*>(cd + d);
        acc = dot_pair(acc, cv.x, rv.x, cv.y, rv.y);
        acc = dot_pair(acc, cv.z, rv.z, cv.w, rv.w);
      }
      // coherent at agent scope: read by workgroups on other XCDs
      float* o = ex ? dot_e + (int64_t)(z + k * NZ) * Me + m : dot_s + (int64_t)(z + k * NZ) * Ms + m;
      __hip_atomic_store(o, E::rnd(acc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // sync 1; meanwhile the LRU victim order (rank of each key among all:
  // one key per wave and pass, counted by ballots over the others)
  const unsigned long long epoch = (host_epoch + gen_b * 0x9E3779B97F4A7C15ull) & ((1ull << 62) - 1);
  const bool gave_up1 = group_sync(flags, K, me, 2 * epoch, 2 * epoch + 1, spin_limit, status, &sync_gave_up,
                                   [&](int t1, int nt1) {
    if (Te > 0) {
      const int wb = t1 >> 6, nwb = nt1 >> 6, ln = t1 & 63;
      for (int m = wb; m < Me; m += nwb) {
        const int64_t km = rk[m].v;
        int lt = 0, eq = 0;
        for (int j0 = 0; j0 < Me; j0 += 64) {
          const int j = j0 + ln;
          const bool in = j < Me;
          const int64_t kj = rk[in ? j : 0].v;
          lt += __popcll(__ballot(in && kj < km));
          eq += __popcll(__ballot(in && kj == km && j != m));
        }
        if (ln == 0 && lt < n_lru) {
          if (eq) atomicOr(&ties, 1);
          else lru[lt] = m;
        }
      }
    }
    if (snap.k) {
      // the bank slots as staged, before this chunk's update, copied out of
      // LDS while the sync waits (a loop of stores only: inside the staging
      // loop, with its loads, every store would be waited for)
      const int64_t sb = ((int64_t)b * Hkv + h) * (Me + Ms) * DH;
      const int n_ee = (e1 - e0) * CH, n_ss = (s1 - s0) * CH;
      for (int i = t1; i < n_ee + n_ss; i += nt1) {
        const bool ex = i < n_ee;
        const int j = ex ? i : i - n_ee, r = j / CH, c = j % CH;
        const int64_t row = ex ? e0 + r : Me + s0 + r;
        st8<T>((T*)snap.k + sb + row * DH + 8 * c, ld8<T>((ex ? own_ek : own_sk) + r * DH + 8 * c));
        st8<T>((T*)snap.v + sb + row * DH + 8 * c, ld8<T>((ex ? own_ev : own_sv) + r * DH + 8 * c));
      }
      if (lead)
        for (int i = t1; i < Me + Ms; i += nt1) snap.allowed[(int64_t)b * (Me + Ms) + i] = (uint8_t)used[i];
    }
  });
  if (gave_up1) return;
  // ---- 3. routing of this workgroup's tokens (token i of [Te | Ts] goes
  // to workgroup i mod K): one wave per token
  {
    const float* dall_e = ws + (int64_t)b * Hkv * Te * Me;
    const float* dall_s = ws + CODA_WS(ws_dot_s, s, g) + (int64_t)b * Hkv * Ts * Ms;
    for (int i = me + K * wv; i < Te + Ts; i += K * NW) {
      const bool ex = i < Te;
      const int tt = ex ? i : i - Te, M = ex ? Me : Ms;
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int m = lane; m < M; m += 64) {
        // the heads' dots 8 at a time, all in flight before the sum (kept
        // in head order: the reference's mean over heads)
        const float* src = ex ? dall_e + (int64_t)tt * Me + m : dall_s + (int64_t)tt * Ms + m;
        const int64_t hstride = ex ? (int64_t)Te * Me : (int64_t)Ts * Ms;
        float acc = 0.f;
        for (int h0 = 0; h0 < Hkv; h0 += 8) {
          float hv[8];
#pragma unroll
          for (int u = 0; u < 8; ++u)
            hv[u] = h0 + u < Hkv ? __hip_atomic_load(src + (h0 + u) * hstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                 : 0.f;
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (h0 + u < Hkv) acc += hv[u];
        }
        float v = E::rnd(acc / (float)Hkv);
        if (ex ? (m >= Ae || used[m] == 0) : m >= As) v = neg_fill<T>();
        if (v > bv || (v == bv && m < bi)) { bv = v; bi = m; }
      }
      wave_argmax(bv, bi);
      if (lane == 0) {
        if (ex) {
          __hip_atomic_store(dx.fl_e + tt, __builtin_bit_cast(int32_t, bv), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(dx.idx_e + tt, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          __hip_atomic_store(dx.idx_s + tt, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
  if (Te > 0 && ties) {
    // ties among the leading LRU keys: libstdc++'s order
    if (t == 0) sel::topk_order<int64_t>(rk, Me, n_lru, false, true);
    __syncthreads();
    for (int r = t; r < n_lru; r += NT) lru[r] = (int32_t)rk[r].i;
  }
  // sync 2; meanwhile this workgroup's share of head h's ring (every
  // workgroup of head h has read its candidate rows before sync 1)
  const bool gave_up2 = group_sync(flags, K, me, 2 * epoch + 1, 2 * epoch + 1, spin_limit, status, &sync_gave_up,
                                   [&](int t1, int nt1) {
    const int n_all = (Lr + g.blk - first) * CH;
    const int pz = (n_all + NZ - 1) / NZ, p0 = min(n_all, z * pz), p1 = min(n_all, p0 + pz);
    for (int base = p0 + t1; base < p1; base += kRingPre * nt1) {
      Piece8<T> pk[kRingPre], pv[kRingPre];
#pragma unroll
      for (int u = 0; u < kRingPre; ++u) {
        const int i = min(base + u * nt1, p1 - 1);
        const int jb = first + i / CH - Lr, c = i % CH;
        pk[u] = ld8<T>(kbk + b * g.b_sb + h * g.b_sh + (int64_t)jb * g.b_sl + 8 * c);
        pv[u] = ld8<T>(vbk + b * g.b_sb + h * g.b_sh + (int64_t)jb * g.b_sl + 8 * c);
      }
#pragma unroll
      for (int u = 0; u < kRingPre; ++u) {
        const int i = base + u * nt1;
        if (i < p1) {
          const int slot = (rhead + first + i / CH) % W, c = i % CH;
          st8<T>(kb + (int64_t)slot * DH + 8 * c, pk[u]);
          st8<T>(vb + (int64_t)slot * DH + 8 * c, pv[u]);
        }
      }
    }
    // ring gates and visibility bytes of the chunk's surviving tokens
    // (per sequence: head 0's workgroups share them)
    if (h == 0) {
      const int n_tok = Lr + g.blk - first;
      const int pt = (n_tok + NZ - 1) / NZ, q0 = min(n_tok, z * pt), q1 = min(n_tok, q0 + pt);
      for (int i = q0 + t1; i < q1; i += nt1) {
        const int r = first + i, slot = (rhead + r) % W;
        s.g_recent[(int64_t)b * W + slot] = gb[(int64_t)b * g.g_sb + (r - Lr)];
        al[slot] = 1;
      }
    }
  });
  if (gave_up2) return;
  // every workgroup of b has read gen_b (before its sync-1 flag): the next
  // launch on this workspace takes the next generation
  if (lead && t == 0) __hip_atomic_store(tail + b, gen_b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // ---- 4a. every token's routing (all three loads in flight together);
  // exact decisions (memory_banks.py:640-697)
  for (int i = t; i < TT; i += NT) {
    const int ie = min(i, max(Te, 1) - 1), is = min(i, max(Ts, 1) - 1);
    const int32_t fe = Te > 0 ? __hip_atomic_load(dx.fl_e + ie, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    const int32_t xe = Te > 0 ? __hip_atomic_load(dx.idx_e + ie, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    const int32_t xs = Ts > 0 ? __hip_atomic_load(dx.idx_s + is, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    if (i < Te) {
      bv_e[i] = __builtin_bit_cast(float, fe);
      bi_e[i] = xe;
    }
    if (i < Ts) {
      idx_s[i] = xs;
      const float gt = gate[i];
      wtok[i] = (!s.gated || gt >= s.tau_summary) ? E::rnd(gt) : 0.f;
    }
  }
  __syncthreads();
  // exact decisions on wave 0 (at most 64 tokens: lane tt takes token tt),
  // the summary slots' token masks on the other waves, side by side
  const int sum_w0 = Te > 0 ? 1 : 0;  // first wave of the summary masks
  if (Te > 0 && wv == 0) {
    // (exact flags and touch stamps start cleared; the staged stamps are no
    // longer read)
    int u = 0;
    for (int m = lane; m < Me; m += 64) {
      u |= used[m] != 0;
      eflag[m] = 0;
      last[m] = kNegBig;
    }
    const int any_used = wave_or(u);
    // the rank of a novel kept token (the reference's cumsum(novel & keep)
    // - 1) from the ballot of the lanes before it
    const uint64_t lt_mask = lane ? (~0ull >> (64 - lane)) : 0ull;
    const int tt = lane;
    const bool in = tt < Te;
    const int ti = in ? tt : Te - 1;
    const bool keep = s.gated ? (gate[ti] >= s.tau_exact) : true;
    const float bv = bv_e[ti];
    const bool novel = !any_used || bv < E::rnd(s.tau_novel);
    const bool hit = any_used && bv >= E::rnd(s.tau_match);
    const bool nk = in && novel && keep;
    const uint64_t bal = __ballot(nk);
    const int rank = __popcll(bal & lt_mask) + (nk ? 1 : 0) - 1;
    const bool cap = nk && rank < Ae;
    int idx = bi_e[ti];
    if (cap) idx = lru[min(max(rank, 0), n_lru - 1)];
    const bool touch = keep && (!novel || cap);
    const bool ow = s.refresh_on_hit ? (keep && (cap || hit)) : cap;
    if (in) {
      idx_e[tt] = idx;
      fl_e[tt] = (ow ? 1 : 0) | (touch ? 2 : 0);
      // the slot's flags through LDS atomics (after this wave's clears, in
      // its LDS order): written (an overwriting token) and touched (max
      // position of the touching tokens)
      if (ow) atomicOr(&eflag[idx], 1);
      if (touch) atomicMax(reinterpret_cast<long long*>(&last[idx]), (long long)(g.pos0 - g.ring_filled + pcl[tt]));
    }
    if (lead && (s.metrics || s.frustrated)) {
      const int c_ow = __popcll(__ballot(in && ow)), c_cap = __popcll(__ballot(in && cap));
      const int c_hit = __popcll(__ballot(in && hit && keep)), c_gated = __popcll(__ballot(in && !keep));
      const int c_fr = __popcll(__ballot(nk && !cap));
      if (lane == 0) {
        if (s.metrics) {
          atomic_add_i64(s.metrics + CODA_CNT_EXACT_OVERWRITES, c_ow);
          atomic_add_i64(s.metrics + CODA_CNT_EXACT_FRUSTRATED, c_fr);
          atomic_add_i64(s.metrics + CODA_CNT_EXACT_INSERTS, c_cap);
          atomic_add_i64(s.metrics + CODA_CNT_EXACT_HITS, c_hit);
          if (s.gated) atomic_add_i64(s.metrics + CODA_CNT_TOKENS_GATED_OUT, c_gated);
        }
        if (s.frustrated) atomic_add_i64(s.frustrated + 0, c_fr);
      }
    }
  }
  if (wv >= sum_w0) {
    // summary slots, 8 per wave and pass: token masks (ballots over the
    // tokens), then lane u sums slot u's weights in token order (fp32: the
    // scatter_add order) and sets its active / newly used flags
    for (int m0 = 8 * (wv - sum_w0); m0 < Ms; m0 += 8 * (NW - sum_w0)) {
      uint64_t mine = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint64_t mk = __ballot(lane < Ts && idx_s[min(lane, max(Ts, 1) - 1)] == m0 + u);
        if (lane == u) mine = mk;
      }
      const int m = m0 + lane;
      if (lane < 8 && m < Ms) {
        float c = 0.f;
        for (uint64_t r = mine; r; r &= r - 1) c += wtok[__builtin_ctzll(r)];
        c = E::rnd(c);
        smask[m] = mine;
        scnt[m] = c;
        const bool active = c > 0.f;
        sflag[m] = (active ? 1 : 0) | ((active && used[Me + m] == 0) ? 2 : 0);
      }
    }
  }
  __syncthreads();
  if (lead) {
    if (Te > 0)
      for (int m = t; m < Me; m += NT) {
        if (last[m] != kNegBig) s.mem_last[(int64_t)b * Me + m] = last[m];  // LRU: max pos of the touching tokens
        if (eflag[m]) al[W + m] = 1;
      }
    int32_t* tr = s.trace ? s.trace + (int64_t)b * (2 * Te + Ts) : nullptr;
    if (tr) {
      for (int tt = t; tt < Te; tt += NT) {
        tr[tt] = idx_e[tt];
        tr[Te + tt] = fl_e[tt];
      }
      for (int tt = t; tt < Ts; tt += NT) tr[2 * Te + tt] = idx_s[tt];
    }
    for (int m = t; m < Ms; m += NT)
      if (sflag[m] & 1) al[W + Me + m] = 1;
    if (Ts > 0 && wv == 0) {
      // counts and flags by ballots (no shuffle chain on the lead's path)
      int64_t upd = 0, ins = 0;
      bool all_used = true, any_cnt = false;
      for (int m0 = 0; m0 < Ms; m0 += 64) {
        const int m = m0 + lane;
        const int f = m < Ms ? sflag[m] : 0;
        const bool act = m < Ms && m < As;
        upd += __popcll(__ballot(f & 1));
        ins += __popcll(__ballot((f >> 1) & 1));
        all_used = all_used && __ballot(act && !(used[Me + min(m, Ms - 1)] != 0 || (f & 1))) == 0;
        any_cnt = any_cnt || __ballot(act && (f & 1)) != 0;
      }
      if (lane == 0) {
        if (s.metrics) {
          atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_UPDATES, upd);
          if (s.overwrite_on_insert) atomic_add_i64(s.metrics + CODA_CNT_SUMMARY_INSERTS, ins);
        }
        if (s.frustrated) {
          if (!all_used) atomic_add_i64(s.frustrated + 1, 1);
          if (any_cnt) atomic_add_i64(s.frustrated + 2, 1);
        }
      }
    }
  }
  __syncthreads();
  // ---- 4b. exact write-back of this workgroup's slots (memory_banks.py:
  // 707-742): one wave per written slot, deltas summed in token order
  if (Te > 0) {
    for (int m = e0 + wv; m < e1; m += NW) {
      if (!eflag[m]) continue;
      const int r = m - e0;
      float mk[NV], mv[NV], ak[NV], av[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = min(lane + 64 * i, DH - 1);
        mk[i] = E::ld(own_ek[r * DH + d]);
        mv[i] = E::ld(own_ev[r * DH + d]);
        ak[i] = 0.f;
        av[i] = 0.f;
      }
      for (int tt = 0; tt < Te; ++tt) {
        if (idx_e[tt] != m || !(fl_e[tt] & 1)) continue;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int d = min(lane + 64 * i, DH - 1);
          ak[i] += E::rnd(E::ld(raw_k[tt * DH + d]) - mk[i]);
          av[i] += E::rnd(E::ld(raw_v[tt * DH + d]) - mv[i]);
        }
      }
      T* kr = kb + (int64_t)(W + m) * DH;
      T* vr = vb + (int64_t)(W + m) * DH;
      float nv[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = lane + 64 * i;
        act[i] = d < DH;
        nv[i] = 0.f;
        if (act[i]) {
          kr[d] = E::st(mk[i] + E::rnd(ak[i]));
          nv[i] = E::rnd(mv[i] + E::rnd(av[i]));
          vr[d] = E::st(nv[i]);
        }
      }
      wave_unit<T, NV>(nv, act);
      T* nr = (T*)s.exact_v_norm + (((int64_t)b * Hkv + h) * Me + m) * DH;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) nr[lane + 64 * i] = E::st(nv[i]);
    }
  }
  // ---- 4c. summary accumulate + EMA of this workgroup's slots
  // (memory_banks.py:880-932): one wave per slot, lane l taking columns l,
  // l + 64, ... (column col < DH is V channel col, else K channel
  // DH/2 + col - DH), all of them over the slot's tokens in token order (the
  // fp32 scatter_add order); then the slot's new LF key row through LDS and
  // its norm-cache row, within the wave
  if (Ts > 0) {
    const float eta_h = s.eta[h];
    constexpr int NCW = (NCOL + 63) / 64;
    for (int m = s0 + wv; m < s1; m += NW) {
      if (!(sflag[m] & 1)) continue;
      const uint64_t msk = smask[m];
      const float eta = (s.overwrite_on_insert && (sflag[m] & 2)) ? 1.f : eta_h;
      const float cnt = fmaxf(scnt[m], eps_r<T>());
      const int rl = m - s0;
      const T* tokv[NCW];
      float a[NCW];
#pragma unroll
      for (int jc = 0; jc < NCW; ++jc) {
        const int col = min(lane + 64 * jc, NCOL - 1);
        tokv[jc] = (col < DH ? raw_v : raw_k) + (col < DH ? col : LF + (col - DH));
      }
      {
        uint64_t r = msk;
        int tt = __builtin_ctzll(r);
        float wt = wtok[tt];
#pragma unroll
        for (int jc = 0; jc < NCW; ++jc) a[jc] = E::rnd(E::ld(tokv[jc][tt * DH]) * wt);
        for (r &= r - 1; r; r &= r - 1) {
          tt = __builtin_ctzll(r);
          wt = wtok[tt];
#pragma unroll
          for (int jc = 0; jc < NCW; ++jc) a[jc] += E::rnd(E::ld(tokv[jc][tt * DH]) * wt);
        }
      }
#pragma unroll
      for (int jc = 0; jc < NCW; ++jc) {
        const int col = lane + 64 * jc;
        if (col >= NCOL) continue;
        const float avg = E::rnd(E::rnd(a[jc]) / cnt);
        if (col < DH) {
          const float mem = E::ld(own_sv[rl * DH + col]);
          vb[(int64_t)(W + Me + m) * DH + col] = E::st(mem + E::rnd(eta * E::rnd(avg - mem)));
        } else {
          const int d = LF + (col - DH);
          const float mem = E::ld(own_sk[rl * DH + d]);
          const float dk = E::rnd(E::rnd(avg * s.energy_scale) - mem);
          const float nkv = E::rnd(mem + E::rnd(eta * dk));
          kb[(int64_t)(W + Me + m) * DH + d] = E::st(nkv);
          knew[rl * LF + (col - DH)] = nkv;  // new LF key for the norm cache
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LF keys are in LDS
      __builtin_amdgcn_wave_barrier();
      float x[NV];
      bool act[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int dd = lane + 64 * i;
        act[i] = dd < LF;
        x[i] = act[i] ? knew[rl * LF + dd] : 0.f;
      }
      wave_unit<T, NV>(x, act);
      T* nr = (T*)s.sum_lf_k_norm + (((int64_t)b * Hkv + h) * Ms + m) * LF;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (act[i]) nr[lane + 64 * i] = E::st(x[i]);
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
  CODA_REQUIRE(s->Ms == 0 || (s->sum_lf_k_norm && s->eta), "%s: summary bank buffers missing", who);
  return CODA_OK;
}

int launch_decode_route(const coda_bank_desc* s, int j, float* ws, hipStream_t st) {
  const dim3 grid(s->Hkv, s->B), block(256);
  const bool bf = s->dtype == CODA_BF16;
  switch (s->Dh) {
    case 32:
      if (bf) hipLaunchKernelGGL((decode_route_kernel<bf16_t, 32>), grid, block, 0, st, *s, j, ws);
      else hipLaunchKernelGGL((decode_route_kernel<float, 32>), grid, block, 0, st, *s, j, ws);
      break;
    case 64:
      if (bf) hipLaunchKernelGGL((decode_route_kernel<bf16_t, 64>), grid, block, 0, st, *s, j, ws);
      else hipLaunchKernelGGL((decode_route_kernel<float, 64>), grid, block, 0, st, *s, j, ws);
      break;
    default:
      if (bf) hipLaunchKernelGGL((decode_route_kernel<bf16_t, 128>), grid, block, 0, st, *s, j, ws);
      else hipLaunchKernelGGL((decode_route_kernel<float, 128>), grid, block, 0, st, *s, j, ws);
  }
  return check_launch("decode_route");
}

template <typename T, int DH>
static int launch_dbank(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb, int64_t nb_sh,
                        const float* g_new, int j, int64_t pos, const float* rec_in, float* rec_out, hipStream_t st,
                        RopeK rk) {
  const size_t lds = dbank_lds(*s);
  const int rc = lds_limit<decode_bank_kernel<T, DH>>(lds, "coda_decode_step");
  if (rc) return rc;
  hipLaunchKernelGGL((decode_bank_kernel<T, DH>), dim3(s->Hkv, s->B), dim3(256), lds, st, *s, (const T*)k_new,
                     (const T*)v_new, nb_sb, nb_sh, g_new, j, pos, rec_in, rec_out, rk);
  return check_launch("decode_bank");
}

int launch_decode_bank(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb, int64_t nb_sh,
                       const float* g_new, int j, int64_t pos, const float* rec_in, float* rec_out, hipStream_t st,
                       RopeK rk) {
  if (dbank_lds(*s) > 160 * 1024)
    return fail(CODA_EUNSUP, "coda_decode_step: bank of %d + %d rows does not fit one workgroup", s->Me, s->Ms);
  const bool bf = s->dtype == CODA_BF16;
#define CODA_DBANK(D)                                                                                         \
  return bf ? launch_dbank<bf16_t, D>(s, k_new, v_new, nb_sb, nb_sh, g_new, j, pos, rec_in, rec_out, st, rk) \
            : launch_dbank<float, D>(s, k_new, v_new, nb_sb, nb_sh, g_new, j, pos, rec_in, rec_out, st, rk)
  switch (s->Dh) {
    case 32: CODA_DBANK(32);
    case 64: CODA_DBANK(64);
    default: CODA_DBANK(128);
  }
#undef CODA_DBANK
}

static size_t decode_lds(const coda_bank_desc* s) {
  const int LF = s->Dh - s->lf;
  return sizeof(float) * ((size_t)s->Hkv * s->Dh * 3 + (size_t)s->Hkv * LF + (size_t)s->Hkv * (s->Me + s->Ms) + 1 +
                          (size_t)((s->Me + s->Ms + 1) & ~1) + 2 * (size_t)s->Me);
}

template <typename T, int DH>
static int launch_decode(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb,
                         int64_t nb_sh, const float* g_new, int ring_idx, int ring_filled, int64_t pos,
                         hipStream_t st, RopeK rk) {
  const size_t lds = decode_lds(s);
  const int rc = lds_limit<decode_write_kernel<T, DH>>(lds, "coda_decode_write");
  if (rc) return rc;
  hipLaunchKernelGGL((decode_write_kernel<T, DH>), dim3(s->B), dim3(512), lds, st, *s, (const T*)k_new,
                     (const T*)v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, rk);
  return check_launch("decode_write");
}

int decode_write_impl(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb, int64_t nb_sh,
                      const float* g_new, int ring_idx, int ring_filled, int64_t pos, hipStream_t st, RopeK rk,
                      const char* who) {
  int rc = validate_bank(s, who);
  if (rc) return rc;
  CODA_REQUIRE(k_new && v_new && g_new, "%s: new token pointers missing", who);
  CODA_REQUIRE(ring_filled >= 0 && ring_filled <= s->W, "%s: ring_filled %d outside [0, %d]", who, ring_filled, s->W);
  CODA_REQUIRE(ring_filled < s->W || (ring_idx >= 0 && ring_idx < s->W), "%s: ring_idx %d outside [0, %d)", who,
               ring_idx, s->W);
  CODA_REQUIRE(decode_lds(s) <= 160 * 1024, "%s: Hkv=%d too large for one workgroup", who, s->Hkv);
  if (s->B == 0) return CODA_OK;
  const bool bf = s->dtype == CODA_BF16;
#define CODA_DWRITE(D)                                                                                             \
  return bf ? launch_decode<bf16_t, D>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st, rk) \
            : launch_decode<float, D>(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, st, rk)
  switch (s->Dh) {
    case 32: CODA_DWRITE(32);
    case 64: CODA_DWRITE(64);
    default: CODA_DWRITE(128);
  }
#undef CODA_DWRITE
}

}  // namespace coda

using namespace coda;

extern "C" int coda_decode_write(const coda_bank_desc* s, const void* k_new, const void* v_new, int64_t nb_sb,
                                 int64_t nb_sh, const float* g_new, int ring_idx, int ring_filled, int64_t pos,
                                 void* stream) {
  return decode_write_impl(s, k_new, v_new, nb_sb, nb_sh, g_new, ring_idx, ring_filled, pos, (hipStream_t)stream,
                           RopeK{nullptr, nullptr, 0}, "coda_decode_write");
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

// The workspace's tail: the last B + 1 8-byte words of the caller's buffer
// (at a place that depends only on its size and B, so every chunk of a call
// finds them): a generation word per sequence, then the status word (give-
// ups of the one-launch update's waits, added by the kernel, never cleared
// by it).
static size_t block_tail_bytes(const coda_bank_desc* s) { return 8 * ((size_t)s->B + 1) + 8; }
static unsigned long long* block_tail(const coda_bank_desc* s, void* workspace, size_t workspace_bytes) {
  return reinterpret_cast<unsigned long long*>((char*)workspace + (workspace_bytes / 8) * 8) - (s->B + 1);
}
static size_t block_ws_bytes(const coda_bank_desc* s, int Te, int Ts) {
  return sizeof(float) * ws_total(s->B, s->Hkv, s->Me, s->Ms, Te, Ts) + block_tail_bytes(s);
}

extern "C" int coda_block_workspace_bytes(const coda_bank_desc* s, int Kmax, size_t* bytes) {
  int rc = validate_sizes(s, "coda_block_workspace_bytes");
  if (rc) return rc;
  CODA_REQUIRE(bytes != nullptr, "coda_block_workspace_bytes: null out pointer");
  *bytes = block_ws_bytes(s, Kmax, Kmax);
  return CODA_OK;
}

// Host part of the fused block write's launch epochs: unique per launch in
// the process (48 bits), started from a clock-derived value so that a sync
// word left in a reused workspace never carries the epoch of a later
// launch (the kernel mixes in the sequence's generation word).
static unsigned long long next_epoch() {
  static std::atomic<unsigned long long> ep{
      (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count() * 0x9E3779B97F4A7C15ull};
  return ep.fetch_add(1, std::memory_order_relaxed) & ((1ull << 48) - 1);
}

// The fused kernel runs when its LDS fits and CODA_BLOCK_FUSED is not "0"
// (read at every call, so that one process can compare the two paths).
static bool fused_enabled() {
  const char* e = getenv("CODA_BLOCK_FUSED");
  return !(e && e[0] == '0');
}

// Launch shapes and dynamic LDS of a chunk's bank update with Te / Ts
// candidates over `pairs` (sequence, head) pairs, shared by the launcher and
// coda_block_write_check.  The one-launch kernel: each head over NZ
// workgroups, about 256 in all (more where one workgroup's LDS would not
// fit), at most 8 per head and 64 per sequence; nz = 0 when it cannot run.
struct FusedShape {
  int nz;
  size_t lds;
};
static FusedShape fused_shape(const coda_bank_desc* s, int esz, int Te, int Ts, int pairs) {
  FusedShape f{0, 0};
  if (!(Te <= 64 && Ts <= 64 && Te + Ts > 0 && s->Hkv <= kFusedMaxGroup)) return f;
  const int nz_max = std::max(1, std::min({kFusedMaxGroup / s->Hkv, 8, Te + Ts}));
  int NZ = std::max(1, std::min((256 + pairs - 1) / pairs, nz_max));
  size_t lds = fused_lds(s->Dh, esz, s->Me, s->Ms, Te, Ts, NZ).total;
  while (lds + 1024 > kLdsMax && NZ < nz_max) lds = fused_lds(s->Dh, esz, s->Me, s->Ms, Te, Ts, ++NZ).total;
  if (lds + 1024 <= kLdsMax) f = FusedShape{NZ, lds};  // the kernel's own static LDS is under 1 KiB
  return f;
}
// The four-kernel path: candidate rows split over nz_r route workgroups per
// (sequence, head) (about 512 in all, at least 8 rows each); bank slots over
// nz_a apply workgroups (about 512 in all), PS summary slots each.
struct SplitShape {
  int nz_r, nz_a, PS;
  size_t lds_route, lds_decide, lds_apply;
};
static SplitShape split_shape(const coda_bank_desc* s, int Te, int Ts, int pairs) {
  const int DH = s->Dh, LF = DH - s->lf, n = Te + Ts;
  const size_t room = kLdsMax - 1024;  // each kernel's static LDS is under 1 KiB
  SplitShape p;
  auto route_lds = [&](int nz) {
    const int per = (n + nz - 1) / nz;
    const size_t ne = (size_t)std::min(per, Te), ns = (size_t)std::min(per, Ts);
    return std::max(sizeof(float) * ((ne > 0 ? (s->Me + ne) * (DH + 4) : 0) + (ns > 0 ? (s->Ms + ns) * (LF + 4) : 0)),
                    sizeof(sel::Item<int64_t>) * (size_t)s->Me);
  };
  // more route workgroups where one's candidate rows would not fit
  p.nz_r = std::max(1, std::min((512 + pairs - 1) / pairs, (n + 7) / 8));
  p.lds_route = route_lds(p.nz_r);
  while (p.lds_route > room && p.nz_r < n) p.lds_route = route_lds(++p.nz_r);
  p.lds_decide = sizeof(int) * ((size_t)s->Me + 2 * Te);
  // more apply workgroups where one's summary token lists would not fit
  const int nz_a_max = std::max(1, std::max(s->Me, s->Ms));
  p.nz_a = std::max(1, std::min((512 + pairs - 1) / pairs, nz_a_max));
  p.PS = (s->Ms + p.nz_a - 1) / p.nz_a;
  p.lds_apply = apply_lds_bytes(s->Ms, Te, Ts, p.PS, LF);
  while (p.lds_apply > room && p.nz_a < nz_a_max) {
    ++p.nz_a;
    p.PS = (s->Ms + p.nz_a - 1) / p.nz_a;
    p.lds_apply = apply_lds_bytes(s->Ms, Te, Ts, p.PS, LF);
  }
  return p;
}

// Spin limit of the fused kernel's bounded waits (coda_block_sync_spin_limit)
static std::atomic<int> g_spin_limit{kSyncSpinLimit};

template <typename T, int DH>
static int launch_block(const coda_bank_desc* s, const void* kb, const void* vb, const float* gb, BlockGeom g,
                        const int32_t* plan_c, float* ws, unsigned long long* tail, hipStream_t st,
                        BankSnap snap) {
  const int TT = g.Te > g.Ts ? g.Te : g.Ts;
  const int pairs = s->B * s->Hkv;
  if (g.n_ev > 0 && TT > 0 && fused_enabled()) {
    const FusedShape fs = fused_shape(s, (int)sizeof(T), g.Te, g.Ts, pairs);
    const int NZ = fs.nz;
    const size_t lds = fs.lds;
    if (NZ > 0) {
      int rc = lds_limit<block_fused_kernel<T, DH>>(lds, "coda_block_write");
      if (rc) return rc;
      unsigned long long* flags = reinterpret_cast<unsigned long long*>(ws + CODA_WS(ws_sync, *s, g));
      // (sequence, head) pairs in blocks of 8, one pair per XCD (a pair
      // beyond B * Hkv exits at once)
      const int nwg = ((pairs + 7) / 8) * 8 * NZ;
      hipLaunchKernelGGL((block_fused_kernel<T, DH>), dim3(nwg), dim3(kFusedThreads), lds, st, *s, g, NZ,
                         (const T*)kb, (const T*)vb, gb, plan_c, ws, flags, next_epoch(), tail,
                         g_spin_limit.load(std::memory_order_relaxed), snap);
      return check_launch("block_fused");
    }
  }
  if (snap.k)
    return fail(CODA_EUNSUP, "coda_block_write_snapshot: the one-launch update does not run for this chunk "
                             "(Te=%d Ts=%d n_ev=%d)", g.Te, g.Ts, g.n_ev);
  const SplitShape sp = split_shape(s, g.Te, g.Ts, pairs);
  if (g.n_ev > 0 && TT > 0) {
    int rc = lds_limit<block_route_kernel<T, DH>>(sp.lds_route, "coda_block_write");
    if (rc) return rc;
    hipLaunchKernelGGL((block_route_kernel<T, DH>), dim3(s->Hkv + 1, s->B, sp.nz_r), dim3(256), sp.lds_route, st,
                       *s, g, (const T*)kb, (const T*)vb, gb, plan_c, ws);
    rc = check_launch("block_route");
    if (rc) return rc;
  }
  const int nsc = (g.Ts + kDecideChunk - 1) / kDecideChunk;
  if (g.n_ev > 0 && TT > 0) {
    const size_t lds_d = sp.lds_decide;
    int rc = lds_limit<block_decide_kernel<T>>(lds_d, "coda_block_write");
    if (rc) return rc;
    hipLaunchKernelGGL((block_decide_kernel<T>), dim3(1 + nsc, s->B), dim3(256), lds_d, st, *s, g, plan_c, ws);
    rc = check_launch("block_decide");
    if (rc) return rc;
  }
  if (g.n_ev > 0 && TT > 0) {
    int rc = lds_limit<block_apply_kernel<T, DH>>(sp.lds_apply, "coda_block_write");
    if (rc) return rc;
    hipLaunchKernelGGL((block_apply_kernel<T, DH>), dim3(s->Hkv, s->B, sp.nz_a), dim3(kApplyThreads), sp.lds_apply,
                       st, *s, g, (const T*)kb, (const T*)vb, plan_c, ws);
    rc = check_launch("block_apply");
    if (rc) return rc;
  }
  {
    // at most two 16-byte pieces per thread and plane in each workgroup
    const int first = std::max(g.ring_filled, g.n_ev);
    const int n_all = (g.ring_filled + g.blk - first) * (DH / 8);
    const int nzr = std::max(1, (n_all + 2 * kApplyThreads - 1) / (2 * kApplyThreads));
    hipLaunchKernelGGL((block_ring_kernel<T, DH>), dim3(s->Hkv, s->B, nzr), dim3(kApplyThreads), 0, st, *s, g,
                       (const T*)kb, (const T*)vb, gb);
  }
  return check_launch("block_ring");
}

extern "C" int coda_block_write_check(const coda_bank_desc* s, int Te, int Ts) {
  int rc = validate_sizes(s, "coda_block_write_check");
  if (rc) return rc;
  CODA_REQUIRE(Te >= 0 && Ts >= 0, "coda_block_write_check: negative candidate counts");
  if (Te + Ts == 0) return CODA_OK;
  const int esz = s->dtype == CODA_BF16 ? 2 : 4;
  // every batch size: one pair stands for a large batch (one workgroup per
  // (sequence, head) in the four-kernel path), B * Hkv for a given B
  const int pairs = s->B > 0 ? s->B * s->Hkv : (1 << 20);
  if (fused_shape(s, esz, Te, Ts, pairs).nz > 0) return CODA_OK;
  const SplitShape p = split_shape(s, Te, Ts, pairs);
  const size_t room = kLdsMax - 1024;
  CODA_REQUIRE(p.lds_route <= room && p.lds_decide <= room && p.lds_apply <= room,
               "coda_block_write_check: a chunk with %d exact and %d summary candidates at head_dim %d, Me=%d, "
               "Ms=%d needs %zu / %zu / %zu bytes of LDS (routing / decisions / bank writes), above the %zu a "
               "workgroup has on gfx950: the norm caches of one head (Me*(Dh+4) + Ms*(Dh/2+4) floats) and the "
               "summary token lists (Ms*Ts words) must fit",
               Te, Ts, s->Dh, s->Me, s->Ms, p.lds_route, p.lds_decide, p.lds_apply, room);
  return CODA_OK;
}

static int block_write_impl(const coda_bank_desc* s, const void* kb, const void* vb, int64_t b_sb, int64_t b_sh,
                            int64_t b_sl, const float* gb, int64_t g_sb, int blk, int ring_head, int ring_filled,
                            int64_t pos0, const int32_t* plan_c, int Kmax, int Te, int Ts, void* workspace,
                            size_t workspace_bytes, void* stream, BankSnap snap) {
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
  unsigned long long* tail = workspace ? block_tail(s, workspace, workspace_bytes) : nullptr;
  switch (s->Dh) {
    case 32:
      return bf ? launch_block<bf16_t, 32>(s, kb, vb, gb, g, plan_c, ws, tail, st, snap)
                : launch_block<float, 32>(s, kb, vb, gb, g, plan_c, ws, tail, st, snap);
    case 64:
      return bf ? launch_block<bf16_t, 64>(s, kb, vb, gb, g, plan_c, ws, tail, st, snap)
                : launch_block<float, 64>(s, kb, vb, gb, g, plan_c, ws, tail, st, snap);
    default:
      return bf ? launch_block<bf16_t, 128>(s, kb, vb, gb, g, plan_c, ws, tail, st, snap)
                : launch_block<float, 128>(s, kb, vb, gb, g, plan_c, ws, tail, st, snap);
  }
}

extern "C" int coda_block_write(const coda_bank_desc* s, const void* kb, const void* vb, int64_t b_sb, int64_t b_sh,
                                int64_t b_sl, const float* gb, int64_t g_sb, int blk, int ring_head, int ring_filled,
                                int64_t pos0, const int32_t* plan_c, int Kmax, int Te, int Ts, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return block_write_impl(s, kb, vb, b_sb, b_sh, b_sl, gb, g_sb, blk, ring_head, ring_filled, pos0, plan_c, Kmax, Te,
                          Ts, workspace, workspace_bytes, stream, BankSnap{nullptr, nullptr, nullptr});
}

extern "C" int coda_block_write_snapshot(const coda_bank_desc* s, const void* kb, const void* vb, int64_t b_sb,
                                         int64_t b_sh, int64_t b_sl, const float* gb, int64_t g_sb, int blk,
                                         int ring_head, int ring_filled, int64_t pos0, const int32_t* plan_c, int Kmax,
                                         int Te, int Ts, void* workspace, size_t workspace_bytes, void* snap_k,
                                         void* snap_v, uint8_t* snap_allowed, void* stream) {
  CODA_REQUIRE(snap_k && snap_v && snap_allowed, "coda_block_write_snapshot: snapshot pointers missing");
  CODA_REQUIRE(((uintptr_t)snap_k % 16) == 0 && ((uintptr_t)snap_v % 16) == 0,
               "coda_block_write_snapshot: snapshot rows must be 16-byte aligned");
  return block_write_impl(s, kb, vb, b_sb, b_sh, b_sl, gb, g_sb, blk, ring_head, ring_filled, pos0, plan_c, Kmax, Te,
                          Ts, workspace, workspace_bytes, stream, BankSnap{snap_k, snap_v, snap_allowed});
}

extern "C" int coda_block_write_chain(const coda_bank_desc* s, const void* kb, const void* vb, int64_t b_sb,
                                      int64_t b_sh, int64_t b_sl, const float* gb, int64_t g_sb, int L, int blk,
                                      int c_first, int n_chunks, int ring_head, int ring_filled, int64_t pos0,
                                      const int32_t* plan, int Kmax, int k_exact, int k_summary, void* workspace,
                                      size_t workspace_bytes, void* snap_k, void* snap_v, uint8_t* snap_allowed,
                                      int64_t snap_stride, int64_t snap_al_stride, int* ring_out, void* stream) {
  int rc = validate_bank(s, "coda_block_write_chain");
  if (rc) return rc;
  CODA_REQUIRE(kb && vb && gb && plan && ring_out && snap_k && snap_v && snap_allowed,
               "coda_block_write_chain: pointer missing");
  CODA_REQUIRE(blk > 0 && n_chunks > 0 && c_first >= 0 && (int64_t)(c_first + n_chunks - 1) * blk < L,
               "coda_block_write_chain: chunks %d .. %d of %d tokens in blocks of %d", c_first,
               c_first + n_chunks - 1, L, blk);
  CODA_REQUIRE(!s->metrics && !s->frustrated && !s->trace,
               "coda_block_write_chain: metrics, frustration flags and traces need the per-chunk calls");
  CODA_REQUIRE(snap_stride >= 0 && snap_al_stride >= 0, "coda_block_write_chain: negative snapshot stride");
  CODA_REQUIRE(((uintptr_t)snap_k % 16) == 0 && ((uintptr_t)snap_v % 16) == 0 &&
                   (snap_stride * (s->dtype == CODA_BF16 ? 2 : 4)) % 16 == 0,
               "coda_block_write_chain: snapshot rows must be 16-byte aligned");
  // the ring progression first: every chunk must evict and take the
  // one-launch update, else nothing is enqueued
  const size_t esz = s->dtype == CODA_BF16 ? 2 : 4;
  int head = ring_head, filled = ring_filled;
  for (int i = 0; i < n_chunks; ++i) {
    const int t = (c_first + i) * blk, n = blk < L - t ? blk : L - t;
    const int total = filled + n, keep = total < s->W ? total : s->W, n_ev = total - keep;
    const int Te = s->Me > 0 ? (k_exact < n_ev ? k_exact : n_ev) : 0;
    const int Ts = s->Ms > 0 ? (k_summary < n_ev ? k_summary : n_ev) : 0;
    CODA_REQUIRE(n_ev > 0 && (Te > 0 || Ts > 0), "coda_block_write_chain: chunk %d evicts nothing", c_first + i);
    CODA_REQUIRE(Te <= Kmax && Ts <= Kmax, "coda_block_write_chain: Kmax %d < candidates", Kmax);
    if (!(fused_enabled() && fused_shape(s, (int)esz, Te, Ts, s->B * s->Hkv).nz > 0))
      return fail(CODA_EUNSUP, "coda_block_write_chain: chunk %d does not take the one-launch update",
                  c_first + i);
    head = filled == s->W ? head : 0;
    if (keep == s->W) head = (head + n_ev) % s->W;
    filled = keep;
  }
  head = ring_head;
  filled = ring_filled;
  for (int i = 0; i < n_chunks; ++i) {
    const int t = (c_first + i) * blk, n = blk < L - t ? blk : L - t;
    const int total = filled + n, keep = total < s->W ? total : s->W, n_ev = total - keep;
    const int Te = s->Me > 0 ? (k_exact < n_ev ? k_exact : n_ev) : 0;
    const int Ts = s->Ms > 0 ? (k_summary < n_ev ? k_summary : n_ev) : 0;
    const char* kbc = (const char*)kb + (int64_t)t * b_sl * (int64_t)esz;
    const char* vbc = (const char*)vb + (int64_t)t * b_sl * (int64_t)esz;
    rc = block_write_impl(s, kbc, vbc, b_sb, b_sh, b_sl, gb + t, g_sb, n, head, filled, pos0 + (int64_t)i * blk,
                          plan + (int64_t)(c_first + i) * s->B * Kmax, Kmax, Te, Ts, workspace, workspace_bytes,
                          stream,
                          BankSnap{(char*)snap_k + (int64_t)i * snap_stride * (int64_t)esz,
                                   (char*)snap_v + (int64_t)i * snap_stride * (int64_t)esz,
                                   snap_allowed + (int64_t)i * snap_al_stride});
    if (rc) return rc;
    head = filled == s->W ? head : 0;
    if (keep == s->W) head = (head + n_ev) % s->W;
    filled = keep;
  }
  ring_out[0] = head;
  ring_out[1] = filled;
  return CODA_OK;
}

// ------------------------------------------------------------ no-alloc variant
// Scratch of coda_block_write_noalloc: one array per GPU, resident until the
// process ends.  In host code the symbol names a host-side stand-in, never
// device memory: host code uses only the device address hipGetSymbolAddress
// returns for the current device, looked up once per device and kept.
static constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static constexpr int kNoAllocMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static int noalloc_scratch(void** out) {
  static std::mutex mu;
  static void* per_device[kNoAllocMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(CODA_EHIP, "coda_block_write_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return fail(CODA_EUNSUP, "coda_block_write_noalloc: device %d beyond %d devices", dev, kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (per_device[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(CODA_EHIP, "coda_block_write_noalloc: scratch address on device %d: %s", dev,
                  hipGetErrorString(e));
    per_device[dev] = p;
  }
  *out = per_device[dev];
  return CODA_OK;
}

extern "C" int coda_block_sync_timeouts(unsigned int* out) {
  CODA_REQUIRE(out != nullptr, "coda_block_sync_timeouts: null out pointer");
  const hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_block_sync_timeouts), sizeof(unsigned int), 0,
                                           hipMemcpyDeviceToHost);
  if (e != hipSuccess) return fail(CODA_EHIP, "coda_block_sync_timeouts: %s", hipGetErrorString(e));
  return CODA_OK;
}

// Dynamic expansion after a bank update (attention.py:358-390): one thread.
__global__ __launch_bounds__(64) void bank_expand_kernel(int32_t* active, const int64_t* fr, int ce, int cs,
                                                         int count_mode, int ran_e, int ran_s, int64_t* counters) {
  if (threadIdx.x != 0) return;
  const int64_t fe = ran_e ? (count_mode ? fr[0] : (int64_t)(fr[0] > 0)) : 0;
  const int64_t fs = ran_s ? (int64_t)(fr[1] == 0 && fr[2] > 0) : 0;
  int64_t de = 0, ds = 0;
  if (active) {
    const int ae = active[0], as = active[1];
    if (fe > 0 && ae < ce) de = fe < (int64_t)(ce - ae) ? fe : (int64_t)(ce - ae);
    if (fs > 0 && as < cs) ds = fs < (int64_t)(cs - as) ? fs : (int64_t)(cs - as);
    active[0] = ae + (int)de;
    active[1] = as + (int)ds;
  }
  if (counters) {
    counters[0] += fs;
    counters[1] += de;
    counters[2] += ds;
  }
}

extern "C" int coda_bank_expand(int32_t* active, const int64_t* frustrated, int ceil_exact, int ceil_summary,
                                int exact_count_mode, int ran_exact, int ran_summary, int64_t* counters,
                                void* stream) {
  CODA_REQUIRE(frustrated != nullptr, "coda_bank_expand: frustration flags missing");
  CODA_REQUIRE(ceil_exact >= 0 && ceil_summary >= 0, "coda_bank_expand: negative ceiling");
  if (!active && !counters) return CODA_OK;
  hipLaunchKernelGGL(bank_expand_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, active, frustrated, ceil_exact,
                     ceil_summary, exact_count_mode, ran_exact, ran_summary, counters);
  return check_launch("bank_expand");
}

extern "C" int coda_block_sync_spin_limit(int limit) {
  return g_spin_limit.exchange(limit < -1 ? -1 : limit, std::memory_order_relaxed);
}

extern "C" size_t coda_block_write_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int coda_block_write_noalloc(const coda_bank_desc* s, const void* kb, const void* vb, int64_t b_sb,
                                        int64_t b_sh, int64_t b_sl, const float* gb, int64_t g_sb, int blk,
                                        int ring_head, int ring_filled, int64_t pos0, const int32_t* plan_c,
                                        int Kmax, int Te, int Ts, void* stream) {
  int rc = validate_bank(s, "coda_block_write_noalloc");
  if (rc) return rc;
  CODA_REQUIRE(Te >= 0 && Ts >= 0, "coda_block_write_noalloc: negative candidate counts");
  const size_t need = block_ws_bytes(s, Te, Ts);
  CODA_REQUIRE(need <= kNoAllocScratchBytes,
               "coda_block_write_noalloc: this chunk needs %zu bytes of scratch, more than the %zu bytes the "
               "library holds per GPU (B * Hkv * (Te * Me + Ts * Ms) fp32 dots dominate); call coda_block_write "
               "with a workspace instead",
               need, kNoAllocScratchBytes);
  // nothing in the scratch needs to start at zero: every word a chunk reads
  // is written earlier in the same call (dots, metadata snapshot,
  // decisions), except the tail's generation and status words, which the
  // array's zero initialisation starts and every call carries on
  void* ws = nullptr;
  rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return coda_block_write(s, kb, vb, b_sb, b_sh, b_sl, gb, g_sb, blk, ring_head, ring_filled, pos0, plan_c, Kmax,
                          Te, Ts, ws, kNoAllocScratchBytes, stream);
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
