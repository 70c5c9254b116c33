/*
 * coda_mi355x.h - C ABI of the MI355X (gfx950) bounded differential-attention
 * hot path of CoDA-GQA-L.
 *
 * Every entry point:
 *   - takes caller-owned device pointers (plain pointers, element strides,
 *     sizes); the library never allocates device memory except where an
 *     entry point documents a workspace the caller passes in;
 *   - validates its arguments on the host before any HIP call, so a bad
 *     shape / stride / size returns a nonzero code without touching the GPU;
 *   - enqueues its kernels on `stream` (a hipStream_t passed as void*, NULL
 *     = the null stream) and returns without synchronising;
 *   - returns 0 on success, a CODA_E* code otherwise; the message of the
 *     last failure on the calling thread is returned by coda_last_error().
 *
 * Element types: CODA_F32 (float), CODA_BF16 (bfloat16 bits, uint16_t),
 * CODA_F16 (half bits, standalone epilogue only).
 *
 * Bit-exactness contract: every bank decision (candidate order, slot index,
 * overwrite / touch flags, LRU stamps) and every bank write follows the
 * reference's CPU eager path operation by operation, including reduced
 * precision rounding points; attention outputs agree to fp32 1e-4 and
 * bf16 2e-2 (max error over the output, relative to its max magnitude).
 */
#ifndef CODA_MI355X_H
#define CODA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CODA_ABI_VERSION 1

enum { CODA_F32 = 0, CODA_BF16 = 1, CODA_F16 = 2 };

enum {
  CODA_OK = 0,
  CODA_EINVAL = 1,   /* bad argument: shape, stride, pointer, dtype */
  CODA_EUNSUP = 2,   /* valid request this build does not implement */
  CODA_EHIP = 3,     /* HIP runtime error (launch / attribute query) */
  CODA_ESMALL = 4    /* caller workspace too small */
};

/* Library version of this header (CODA_ABI_VERSION). */
int coda_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* coda_last_error(void);

/* Hash of the sources the library was built from (16 hex digits, or
 * "unknown"); the Python loader refuses a library whose hash differs from
 * the sources beside it.  No counterpart in the reference, whose epilogue
 * extension setuptools builds (kernels/coda_diff_epilogue/setup.py). */
const char* coda_source_hash(void);

/* Number of HIP devices visible (0 on a host without a GPU; never fails). */
int coda_device_count(void);

/* ------------------------------------------------------------------------
 * Projection front end of the bounded layer (bf16).
 *
 * For M token rows x (M, D) (row stride x_sm, D a multiple of 64) and the
 * packed weights w (n_feat, D), rows in the order q_proj (H*Dh), k_proj
 * (Hkv*Dh; with rope_interleaved == 0 each head's rows reordered to the
 * pairs (i, i + Dh/2) on adjacent rows), v_proj (Hkv*Dh), lambda_proj (H),
 * write_proj (1, when gate), n_feat their sum, one GEMM with fp32
 * accumulation and per-segment epilogues:
 *   q (M, H*Dh)     bf16(x Wq^T + bq)                    (pre-RoPE)
 *   k (M, Hkv*Dh)   RoPE(bf16(x Wk^T + bk)) with the tables (L, Dh/2) at
 *                   row m % L, one bf16 rounding per op (primitives.py:83-113)
 *   v (M, Hkv*Dh)   bf16(x Wv^T + bv)
 *   lam (M, H)      sigmoid(bf16(x Wl^T + bl)), bf16
 *   g (M) float32   sigmoid(bf16(x Wg^T + bg)) in bf16; 1 when gate == 0
 * bias (n_feat) float32, 16-byte aligned, in the weights' row order (zero
 * for a linear without bias).
 * Replaces: the projections of CoDAGQALandmarkPerf2.step
 *   (src/coda_gqa_l/attention.py:396-410, 516-547): q_proj, k_proj,
 *   v_proj, lambda_proj + sigmoid, write_proj + sigmoid, and the RoPE of k.
 * ---------------------------------------------------------------------- */
typedef struct {
  int dtype;               /* CODA_BF16 */
  int M, D, L;             /* token rows, model width, tokens per sequence (table row = m % L) */
  int H, Hkv, Dh;
  int rope_interleaved;
  int gate;                /* 1: write gate from write_proj; 0: g = 1 */
  int w_layout;            /* 0: w row-major (n_feat, D); 1: fragment tiles (coda_project_pack) */
  const void* x;
  int64_t x_sm;
  const void* w;           /* packed weights, layout w_layout */
  const float* bias;       /* (n_feat) */
  const void* rope_cos;    /* (L, Dh/2) */
  const void* rope_sin;
  void* q;
  int64_t q_sm;
  void* k;
  int64_t k_sm;
  void* v;
  int64_t v_sm;
  void* lam;
  int64_t lam_sm;
  float* g;
  void* workspace;         /* unused (coda_project_workspace_bytes is 0) */
  size_t workspace_bytes;
} coda_proj_desc;

/* Decode-shaped inputs only: M <= 64 token rows (more rows: CODA_EINVAL;
 * the layer's prefill projections are library GEMMs).  D 512 .. 8192 and a
 * power of two times 256: each workgroup owns 32 features over all of K,
 * its 8 waves' K-range partials summed in LDS in wave order
 * (deterministic); the weights row-major or in fragment tiles.  Other D (a
 * multiple of 64): 64 x 64 tiles over K, row-major weights only.  No
 * workspace. */
int coda_project(const coda_proj_desc* d, void* stream);

/* The weights of coda_project in fragment tiles (w_layout 1): for row block
 * fb of 16 rows and k-step ks of 32 columns, a 1 KiB tile at element offset
 * (fb * D/32 + ks) * 512 holding W[16 fb + r][32 ks + 8 q + e] at element
 * 8 (r + 16 q) + e (r < 16, q < 4, e < 8) -- the order one wave's 16 x 32
 * MFMA operand load reads, so that a wave streams each row block's K range
 * as contiguous KiBs.  Rows n_feat .. ceil64(n_feat) - 1 are zero.  w:
 * (n_feat, D) row-major with row stride w_sm elements; out: ceil64(n_feat)
 * * D bf16 (ceil64: rounded up to a multiple of 64).  Only for the D that take coda_project's row kernel (512 ..
 * 8192, a power of two times 256): CODA_EUNSUP otherwise, nothing written.
 * No counterpart in the reference (its projections are nn.Linear). */
int coda_project_pack(const void* w, int n_feat, int D, int64_t w_sm, void* out, void* stream);

/* Workspace bytes coda_project needs for this descriptor (0: the kernels
 * keep their partial sums in LDS; kept for callers that size one). */
int coda_project_workspace_bytes(const coda_proj_desc* d, size_t* bytes);



/* ------------------------------------------------------------------------
 * Fused differential attention + epilogue.
 *
 *   out = Norm( Attn(q, K, V) - lam * Attn(q_noise, K, V) )
 *
 * Keys are the concatenation [prefix | block]:
 *   prefix: kp/vp (B, Hkv, Lp, Dh), slot s visible iff allowed[b, s] != 0
 *           (allowed == NULL: all visible).  This is the bounded cache
 *           (ring window + exact bank + summary bank) of the state.
 *   block : kb/vb (B, Hkv, Lb, Dh); causal == 1: query i sees block key j
 *           iff j <= i + (Lb - Lq) (lower-right alignment); causal == 2:
 *           iff j <= i (upper-left, torch SDPA is_causal); causal == 0: all.
 * q is taken pre-RoPE when rope_cos/rope_sin are given ((Lq, Dh/2) tables
 * of the query positions; interleaved pairs (2i,2i+1) or, with
 * rope_interleaved == 0, half-split pairs (i, i+Dh/2)), else post-RoPE.
 * q_noise == NULL: q_noise = pairwise rotation of (roped) q by per-head
 * angle tables theta_cos/theta_sin (H, Dh/2).
 * Norm: RMSNorm over Dh with weight rms_w (eps), or identity (rms_w NULL).
 * GQA: query head h reads KV head h / (H / Hkv).
 *
 * Replaces: the attention seam CoDAGQALandmarkPerf2._sdpa_stacked_two_stream
 *   (src/coda_gqa_l/attention.py:416-465) together with the prefix / causal
 *   mask policy of prefill_chunked (attention.py:635-693) and attend_step
 *   (attention.py:476-514), and the operator
 *   diff_flash_attn(q, q_noise, k, v, lam, rms_weight, eps, is_causal,
 *   sm_scale) (src/coda_gqa_l/triton_diff_flash/__init__.py:86-146).
 * ---------------------------------------------------------------------- */
typedef struct {
  int dtype;                  /* CODA_F32 or CODA_BF16 */
  int B, H, Hkv, Lq, Dh;
  const void* q;              /* (B,H,Lq,Dh) */
  int64_t q_sb, q_sh, q_sl;   /* element strides; d stride is 1 */
  const void* q_noise;        /* (B,H,Lq,Dh) or NULL */
  int64_t qn_sb, qn_sh, qn_sl;
  const void* theta_cos;      /* (H, Dh/2) contiguous, used iff q_noise == NULL */
  const void* theta_sin;
  const void* rope_cos;       /* (Lq, Dh/2) contiguous or NULL */
  const void* rope_sin;
  int rope_interleaved;
  const void* kp;             /* prefix keys (B,Hkv,Lp,Dh) or NULL when Lp == 0 */
  const void* vp;
  int Lp;
  int64_t p_sb, p_sh, p_sl;
  const uint8_t* allowed;     /* (B, Lp) bool bytes, row stride al_sb, or NULL */
  int64_t al_sb;
  const void* kb;             /* block keys (B,Hkv,Lb,Dh) or NULL when Lb == 0 */
  const void* vb;
  int Lb;
  int64_t b_sb, b_sh, b_sl;
  int causal;                 /* 0 none, 1 lower-right, 2 upper-left */
  const void* lam;            /* (B,H,Lq) */
  int64_t lam_sb, lam_sh, lam_sl;
  const void* rms_w;          /* (Dh) or NULL */
  float eps;
  float sm_scale;             /* <= 0: 1/sqrt(Dh) */
  void* out;                  /* (B,H,Lq,Dh) */
  int64_t o_sb, o_sh, o_sl;
  void* workspace;            /* device scratch, >= coda_attn_workspace_bytes() */
  size_t workspace_bytes;
} coda_attn_desc;

/* Device scratch bytes coda_diff_attn_fwd needs for this descriptor. */
int coda_attn_workspace_bytes(const coda_attn_desc* d, size_t* bytes);

int coda_diff_attn_fwd(const coda_attn_desc* d, void* stream);

/* The attention of chunks c_first .. c_first + n_chunks - 1 of a chunked
 * prefill call in one launch, from bank snapshots instead of the live state.
 * Chunk c covers queries [t0, t0 + Lq) of the call, t0 = c * blk,
 * Lq = min(blk, L - t0); it attends to
 *   prefix: bank snapshot c - c_first: d->kp / d->vp (B, Hkv, Lp, Dh) with
 *           strides p_*, advanced by (c - c_first) * snap_stride elements,
 *           visibility bytes d->allowed (row stride al_sb) advanced by
 *           (c - c_first) * al_stride bytes (the exact and summary slots as
 *           the state held them before chunk c's bank update:
 *           coda_block_write_snapshot writes them);
 *   block:  the call's keys [t0 - win, t0 + Lq), win = min(t0, W): the
 *           ring window (the W tokens before the chunk, which is what the
 *           ring holds when they all belong to this call) and the chunk
 *           itself, lower-right causal;
 * d describes the whole call: q / lam / out / rope tables / kb / vb at
 * token 0 (Lq, Lb are set from the chunks).  bf16, head_dim 64 or 128,
 * H / Hkv in {1, 2, 4, 8}, queries roped in-kernel (rope tables, no
 * q_noise), causal == 1; else CODA_EUNSUP before anything runs.  Outputs
 * equal those of coda_diff_attn_fwd on each chunk with the state's [ring |
 * exact | summary] prefix, up to the order of the softmax sums.
 * Replaces: the per-chunk attention of prefill_chunked
 *   (src/coda_gqa_l/attention.py:611-693) for chunks whose ring window lies
 *   in the call. */
int coda_prefill_attn_chunks(const coda_attn_desc* d, int n_chunks, int c_first, int blk, int L, int W,
                             int64_t snap_stride, int64_t al_stride, void* stream);

/* ------------------------------------------------------------------------
 * Standalone differential epilogue over rows of Dh:
 *   out = RMSNorm(sig - lam * noise) * w     (coda_diff_epilogue_fwd)
 *   out = sig - lam * noise                  (coda_diff_sub_only_fwd)
 * sig/noise/out are contiguous (num_rows, head_dim); lam is (num_rows,).
 * Replaces: diff_epilogue_forward_{bf16,fp16,fp32} and
 *   diff_sub_only_forward_{bf16,fp16,fp32}
 *   (kernels/coda_diff_epilogue/kernel_src/diff_epilogue.cu:465-568), bound
 *   as torch ops coda_kernels::diff_epilogue_forward / diff_sub_only_forward
 *   (kernels/coda_diff_epilogue/torch-ext/torch_binding.cpp:203-213).
 * ---------------------------------------------------------------------- */
int coda_diff_epilogue_fwd(int dtype, void* out, const void* sig, const void* noise,
                           const void* lam, const void* w, int num_rows, int head_dim,
                           float eps, void* stream);
int coda_diff_sub_only_fwd(int dtype, void* out, const void* sig, const void* noise,
                           const void* lam, int num_rows, int head_dim, void* stream);

/* The same two epilogues under the reference's own typed symbols and
 * argument lists, so its binding (torch_binding.cpp:203-213) links against
 * this library unchanged.  bf16 and fp16 elements are passed as their
 * 16-bit storage; stream is a hipStream_t.  Like the reference's they
 * return nothing: an argument error or a failed launch leaves its message
 * in coda_last_error().
 * Replaces: diff_epilogue_forward_bf16 / _fp16 / _fp32
 *   (kernels/coda_diff_epilogue/kernel_src/diff_epilogue.cu:465-516) and
 *   diff_sub_only_forward_bf16 / _fp16 / _fp32 (diff_epilogue.cu:520-566). */
void diff_epilogue_forward_bf16(uint16_t* output, const uint16_t* out_sig, const uint16_t* out_noise,
                                const uint16_t* lam, const uint16_t* weight, int num_rows, int head_dim,
                                float eps, void* stream);
void diff_epilogue_forward_fp16(uint16_t* output, const uint16_t* out_sig, const uint16_t* out_noise,
                                const uint16_t* lam, const uint16_t* weight, int num_rows, int head_dim,
                                float eps, void* stream);
void diff_epilogue_forward_fp32(float* output, const float* out_sig, const float* out_noise,
                                const float* lam, const float* weight, int num_rows, int head_dim,
                                float eps, void* stream);
void diff_sub_only_forward_bf16(uint16_t* output, const uint16_t* out_sig, const uint16_t* out_noise,
                                const uint16_t* lam, int num_rows, int head_dim, void* stream);
void diff_sub_only_forward_fp16(uint16_t* output, const uint16_t* out_sig, const uint16_t* out_noise,
                                const uint16_t* lam, int num_rows, int head_dim, void* stream);
void diff_sub_only_forward_fp32(float* output, const float* out_sig, const float* out_noise,
                                const float* lam, int num_rows, int head_dim, void* stream);

/* ------------------------------------------------------------------------
 * RoPE of a (B, Hx, L, Dh) tensor into out (same shape, own strides), with
 * (L, Dh/2) cos/sin tables, rounding after every multiply / add in the
 * element type exactly like the reference's eager apply_rope.
 * Replaces: apply_rope (src/coda_gqa_l/primitives.py:83-113) on the key
 *   path of step / prefill_chunked (attention.py:531-532, :598-600).
 * ---------------------------------------------------------------------- */
int coda_rope_fwd(int dtype, void* out, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                  const void* x, int64_t x_sb, int64_t x_sh, int64_t x_sl,
                  const void* cos_t, const void* sin_t, int B, int Hx, int L, int Dh,
                  int interleaved, void* stream);

/* ------------------------------------------------------------------------
 * Bounded-cache state (CoDAGQALandmarkStatePerf2, src/coda_gqa_l/state.py:24-54)
 * and the layer constants the bank kernels read.  Buffers are contiguous:
 *   k_buf, v_buf  (B, Hkv, Lbuf, Dh), Lbuf = W + Me + Ms, element type dtype
 *   allowed       (B, Lbuf) uint8 (torch.bool)
 *   g_recent      (B, W) float
 *   mem_last      (B, Me) int64
 *   exact_v_norm  (B, Hkv, Me, Dh) dtype       (NULL iff Me == 0)
 *   sum_lf_k_norm (B, Hkv, Ms, Dh - lf) dtype  (NULL iff Ms == 0)
 *   eta           (Hkv,) float: sigmoid(summary_eta_logit) rounded to dtype,
 *                 taken by the caller (the reference's torch op, on the host)
 * metrics: optional (CODA_NUM_COUNTERS,) int64 device counters, or NULL.
 * trace: optional int32 device buffer, or NULL; when set, the entry point
 *   records its slot decisions per sequence b:
 *     coda_decode_write / coda_decode_step (evicting steps only), 4 words at
 *       trace + 4 b: exact idx, exact flags (1 overwrite | 2 keep),
 *       summary idx, summary flags (1 keep | 2 new slot); -1 for an empty bank;
 *     coda_block_write (chunks that evict), 2 Te + Ts words at
 *       trace + (2 Te + Ts) b: exact idx [Te], exact flags [Te]
 *       (1 overwrite | 2 touch), summary idx [Ts].
 * ---------------------------------------------------------------------- */
enum {
  CODA_CNT_EXACT_HITS = 0, CODA_CNT_EXACT_INSERTS, CODA_CNT_EXACT_OVERWRITES,
  CODA_CNT_SUMMARY_UPDATES, CODA_CNT_SUMMARY_INSERTS, CODA_CNT_TOKENS_GATED_OUT,
  CODA_CNT_EXACT_FRUSTRATED, CODA_CNT_SUMMARY_FRUSTRATED, CODA_NUM_COUNTERS = 8
};

typedef struct {
  int dtype;
  int B, Hkv, Dh, W, Me, Ms, lf;      /* lf = low-frequency band start (Dh/2) */
  int active_exact, active_summary;   /* Ae <= Me, As <= Ms */
  void* k_buf;
  void* v_buf;
  uint8_t* allowed;
  float* g_recent;
  int64_t* mem_last;
  void* exact_v_norm;
  void* sum_lf_k_norm;
  const float* eta;
  int gated;                          /* write_policy == "gated" */
  float tau_exact, tau_summary;       /* gate thresholds (fp32 compare) */
  float tau_match, tau_novel;         /* exact-bank cosine thresholds */
  int refresh_on_hit, overwrite_on_insert;
  float energy_scale;                 /* sqrt(Dh / (Dh - lf)) */
  int64_t* metrics;
  int64_t* frustrated;                /* (3,) device int64 or NULL: exact, summary (not all used, kept) */
  int32_t* trace;                     /* decision record or NULL (above) */
  const int32_t* active;              /* (2,) device int32 or NULL: the active sizes [exact, summary]
                                         read by the kernels in place of active_exact / active_summary
                                         (dynamic expansion kept on the device, coda_bank_expand) */
} coda_bank_desc;

/* One decode token per sequence: ring FIFO write; when the ring is full the
 * evicted slot `ring_idx` (its absolute position pos - W) first goes through
 * the exact bank (V-cosine novelty, first-free / LRU slot, blend, norm cache,
 * LRU stamp) and the summary bank (LF-K cosine argmax, gated EMA, norm cache).
 * k_new, v_new: (B, Hkv, Dh) with strides (nb_sb, nb_sh); g_new: (B,) float.
 * ring_filled < W: write slot ring_filled, no eviction.
 * Replaces: MemoryBankMixin._write_one / _exact_update_one /
 *   _summary_update_one (src/coda_gqa_l/memory_banks.py:183-432). */
int coda_decode_write(const coda_bank_desc* s, const void* k_new, const void* v_new,
                      int64_t nb_sb, int64_t nb_sh, const float* g_new,
                      int ring_idx, int ring_filled, int64_t pos, void* stream);

/* One decode token of the hot path: ring / exact / summary update of the
 * evicted slot followed by attention of the token's query over the updated
 * cache (the reference's default step order, write then attend).  `a`
 * describes that attention: Lq = 1, prefix = the state cache of `s`
 * (Lp = Lbuf, contiguous), no block keys.  With a full ring the bank update
 * runs from a routing record (per-head cosine dots of the evicted row with
 * the norm caches + a snapshot of the bank metadata) and leaves the routing
 * record of the next token in the workspace.  bf16 with head_dim 64 / 128
 * and G <= 8: one launch, one workgroup per (head, sequence) doing the bank
 * update and the attention together; otherwise a bank kernel, then the
 * attention kernel.  The workspace holds two
 * records, picked by the parity of `pos`, followed by the attention
 * kernel's scratch.  routed (in/out, may be NULL): on entry nonzero when the
 * record for this call was left by the previous call on the same state and
 * workspace with nothing else modifying the state in between (otherwise a
 * routing kernel runs first); on return 1 when this call left the record of
 * the next token, else 0.  Ring still filling: coda_decode_write then
 * coda_diff_attn_fwd.  workspace >= coda_decode_step_workspace_bytes().
 * Replaces: CoDAGQALandmarkPerf2.step after its projections
 *   (src/coda_gqa_l/attention.py:526-536 -> memory_banks.py:183-432 and
 *   attention.py:476-514). */
int coda_decode_step_workspace_bytes(const coda_bank_desc* s, const coda_attn_desc* a, size_t* bytes);
int coda_decode_step(const coda_bank_desc* s, const coda_attn_desc* a, const void* k_new, const void* v_new,
                     int64_t nb_sb, int64_t nb_sh, const float* g_new, int ring_idx, int ring_filled,
                     int64_t pos, void* workspace, size_t workspace_bytes, int* routed, void* stream);

/* coda_decode_step with the new token's K before RoPE (the layer's k_proj
 * output): every kernel that writes or reads it ropes it with the query's
 * tables a->rope_cos / a->rope_sin (row 0, the token's own position in a
 * write-then-attend step; a->rope_interleaved picks the pairing), in the
 * reference's per-op rounding, so the ring holds the same bytes as after
 * coda_rope_fwd + coda_decode_step.  Needs the tables (16-byte aligned).
 * Replaces: the k RoPE of CoDAGQALandmarkPerf2.step together with the step
 *   (src/coda_gqa_l/attention.py:526-533). */
int coda_decode_step_raw_k(const coda_bank_desc* s, const coda_attn_desc* a, const void* k_new,
                           const void* v_new, int64_t nb_sb, int64_t nb_sh, const float* g_new,
                           int ring_idx, int ring_filled, int64_t pos, void* workspace,
                           size_t workspace_bytes, int* routed, void* stream);

/* Dynamic bank expansion after a bank update, on the device (no host
 * sync): from the frustration flags `frustrated` the update left (see
 * coda_bank_desc), with exact_count_mode 1 (a prefill chunk: the count of
 * frustrated exact tokens) or 0 (a decode step: whether any), and the
 * capacity ceilings ceil_exact / ceil_summary of the position the update
 * ran at (a host computation from the token count), grows active[0] /
 * active[1] like the reference and adds, when counters is not NULL, the
 * summary frustration (0 / 1) to counters[0] and the two growths to
 * counters[1] / counters[2].  ran_exact / ran_summary: whether the update
 * touched that bank.  active may be NULL (no expansion configured: only
 * the counters).  One workgroup of one thread.
 * Replaces: CoDAGQALandmarkPerf2._try_expand with its callers' frustration
 *   counts and metrics updates (src/coda_gqa_l/attention.py:358-390,
 *   memory_banks.py:333-337, 418-426, 744-766, 934-946). */
int coda_bank_expand(int32_t* active, const int64_t* frustrated, int ceil_exact, int ceil_summary,
                     int exact_count_mode, int ran_exact, int ran_summary, int64_t* counters, void* stream);

/* Candidate plan of a chunked prefill: for every chunk c (block_size
 * tokens, last one ragged) and sequence b, the evicted-token indices picked
 * by the reference's CPU topk(g_e, k, sorted=False) (libstdc++ nth_element /
 * partial_sort order, ties included), as positions into the time-ordered
 * [ring | block] sequence of that chunk.
 *   g_ring (B, W) float ring gates in slot order, g_seq (B, L) float (row
 *   stride g_sl), plan (n_chunks, B, Kmax) int32 written; n_ev / k per chunk
 *   follow from ring_filled, W, L, block_size; Kmax = max candidates.
 * Replaces: the candidate selection of _write_block_fast
 *   (src/coda_gqa_l/memory_banks.py:459-510). */
int coda_block_plan(const float* g_ring, int ring_head, int ring_filled, int W,
                    const float* g_seq, int64_t g_sb, int B, int L, int block_size,
                    int k_exact, int k_summary, int do_exact, int do_summary,
                    int32_t* plan, int Kmax, void* stream);

/* Bank update + ring write for one prefill chunk (block of `blk` tokens).
 * kb/vb: (B, Hkv, blk, Dh) roped keys / values of the chunk with strides
 * (b_sb, b_sh, b_sl); gb (B, blk) float with row stride g_sb; plan_c points
 * at this chunk's (B, Kmax) candidate rows of coda_block_plan.
 * The ring is kept circular: head = oldest slot, filled = occupancy.
 * One launch per chunk when the chunk's working set fits a CU's LDS (up to
 * 8 workgroups per (KV head, sequence); the workgroups of a sequence meet
 * at per-sequence sync words in the workspace), else four (route, decide,
 * apply, ring).  Calls that share a workspace must not overlap.
 * The last B + 1 8-byte words of the workspace (at (workspace_bytes / 8) * 8
 * bytes from its start, counting back) are its tail: a generation word per
 * sequence, then a status word.  The one-launch update adds 1 to the status
 * word for every workgroup whose bounded wait for the other heads of its
 * sequence gave up; that workgroup then stops, the chunk's update is
 * incomplete and the state must be treated as lost.  The caller zeroes the
 * workspace (or at least the status word) before the first call and reads
 * the status word after its calls; the library never clears it.  The
 * generation words need no clearing: they keep the sync words of
 * successive launches apart, replays of a captured graph included.
 * The waits need every workgroup of a sequence resident at once; they are
 * launched in one contiguous range, which in-order dispatch on one stream
 * guarantees, so other kernels running beside them on other streams can
 * delay them into a give-up. 
 * Replaces: _write_block_fast (memory_banks.py:438-564) with
 *   _exact_update_block_vectorized (:570-774, PyTorch branch) and
 *   _summary_update_block_hard (:780-950, PyTorch branch). */
int coda_block_write(const coda_bank_desc* s, const void* kb, const void* vb,
                     int64_t b_sb, int64_t b_sh, int64_t b_sl, const float* gb, int64_t g_sb,
                     int blk, int ring_head, int ring_filled, int64_t pos0,
                     const int32_t* plan_c, int Kmax, int Te, int Ts,
                     void* workspace, size_t workspace_bytes, void* stream);

/* coda_block_write that also copies the exact and summary slots it stages
 * (the state before this chunk's update) into snap_k / snap_v (B, Hkv,
 * Me + Ms, Dh), 16-byte aligned, and their visibility bytes into
 * snap_allowed (B, Me + Ms): the prefix of this chunk's attention for
 * coda_prefill_attn_chunks.  Only the one-launch update copies: a chunk it
 * does not run for (no candidates, more than 64 of a kind, Hkv > 64, or
 * its LDS beyond a CU) returns CODA_EUNSUP before anything runs.
 * Replaces: together with coda_prefill_attn_chunks, the chunk loop of
 *   prefill_chunked (src/coda_gqa_l/attention.py:611-724). */
int coda_block_write_snapshot(const coda_bank_desc* s, const void* kb, const void* vb,
                              int64_t b_sb, int64_t b_sh, int64_t b_sl, const float* gb, int64_t g_sb,
                              int blk, int ring_head, int ring_filled, int64_t pos0,
                              const int32_t* plan_c, int Kmax, int Te, int Ts,
                              void* workspace, size_t workspace_bytes, void* snap_k, void* snap_v,
                              uint8_t* snap_allowed, void* stream);

/* coda_block_write_snapshot for chunks c_first .. c_first + n_chunks - 1 of
 * a prefill call in one library call (the chunk loop on the host side of the
 * library): chunk c covers tokens [c blk, min(L, (c + 1) blk)) of kb / vb /
 * gb (given at token 0 of the call), its candidates are plan rows
 * (c, B, Kmax) of coda_block_plan (k_exact / k_summary per chunk, capped by
 * its evictions), its snapshot goes to snap_* advanced by (c - c_first)
 * snap_stride elements / snap_al_stride bytes, pos0 is the position of
 * chunk c_first.  The ring (head, filled) after the last chunk is returned
 * in ring_out[0 .. 1].  Every chunk must evict, and s carries no metrics,
 * frustration flags or trace (else CODA_EINVAL); CODA_EUNSUP when a chunk
 * would not take the one-launch update.  Either way nothing is enqueued.
 * Replaces: the chunk loop of prefill_chunked's bank maintenance
 *   (src/coda_gqa_l/attention.py:611-724, memory_banks.py:438-564). */
int coda_block_write_chain(const coda_bank_desc* s, const void* kb, const void* vb,
                           int64_t b_sb, int64_t b_sh, int64_t b_sl, const float* gb, int64_t g_sb,
                           int L, int blk, int c_first, int n_chunks, int ring_head, int ring_filled,
                           int64_t pos0, const int32_t* plan, int Kmax, int k_exact, int k_summary,
                           void* workspace, size_t workspace_bytes, void* snap_k, void* snap_v,
                           uint8_t* snap_allowed, int64_t snap_stride, int64_t snap_al_stride, int* ring_out,
                           void* stream);

/* Device scratch for coda_block_write. */
int coda_block_workspace_bytes(const coda_bank_desc* s, int Kmax, size_t* bytes);

/* Whether coda_block_write can run chunks with Te exact and Ts summary
 * candidates for these bank sizes (s->B > 0: at that batch; s->B == 0: at
 * every batch; no buffers needed): CODA_OK, or CODA_EUNSUP with a message
 * naming the LDS that the sizes need.  The kernels stage one head's norm
 * caches in LDS, so Me*(Dh+4) + Ms*(Dh/2+4) floats (plus the candidates)
 * must fit in a workgroup's 160 KiB.  The reference has no such limit; the
 * layer calls this at construction so that a configuration beyond it fails
 * there (memory_banks.py:438-564 is the path it guards). */
int coda_block_write_check(const coda_bank_desc* s, int Te, int Ts);

/* Number of times, since the library was loaded on the current device, that
 * a workgroup of the one-launch block write gave up waiting for the other
 * heads of its sequence (bounded wait, about 0.1 s; the chunk's results are
 * then wrong).  Zero in every correct run.  Synchronous; for tests.
 * No counterpart in the reference (the reference has no cross-workgroup
 * wait). */
int coda_block_sync_timeouts(unsigned int* out);

/* Sets the spin limit of the bounded waits of later coda_block_write /
 * coda_block_write_noalloc launches (default 2^20 sleeps, about 0.1 s) and
 * returns the previous one; a negative limit makes every wait give up at
 * once, without polling, so a test can take the failure path with every
 * kernel exiting normally.  Process-wide.
 * No counterpart in the reference: a test hook of the cross-workgroup wait. */
int coda_block_sync_spin_limit(int limit);

/* coda_block_write without a workspace argument and without any allocation:
 * the chunk's scratch (routing dots, metadata snapshot, decisions) lives in a
 * 16 MiB array of the library's own per GPU (static device memory, held until
 * the process ends), addressed through hipGetSymbolAddress once per device.
 * Same arguments, kernels, results and errors as coda_block_write; a chunk
 * whose scratch (coda_block_workspace_bytes) exceeds
 * coda_block_write_noalloc_max_bytes() is rejected with CODA_EINVAL before
 * anything runs.  Calls on one GPU share the array: calls that overlap on one
 * GPU (different streams, or threads) race, so serialise them.  The stream
 * must belong to the current device.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int coda_block_write_noalloc(const coda_bank_desc* s, const void* kb, const void* vb,
                             int64_t b_sb, int64_t b_sh, int64_t b_sl, const float* gb, int64_t g_sb,
                             int blk, int ring_head, int ring_filled, int64_t pos0,
                             const int32_t* plan_c, int Kmax, int Te, int Ts, void* stream);
size_t coda_block_write_noalloc_max_bytes(void);

/* Rotate a full circular ring (head != 0) into time order at slots 0..W-1
 * (k_buf, v_buf, g_recent, allowed), as the reference leaves it after every
 * prefill chunk (_set_recent_from_sequence, memory_banks.py:152-177).
 * workspace >= B * Hkv * W * Dh * 2 elements + B * W floats. */
int coda_ring_rotate(const coda_bank_desc* s, int ring_head, void* workspace,
                     size_t workspace_bytes, void* stream);

/* out row (o, i) = F.normalize(x row (o, i), dim=-1, eps=1e-6) over `len`
 * channels (len <= 128), rows at x + o*x_so + i*x_si (out likewise), with
 * the reference's rounding (fp32 sum of squares, norm rounded to the element
 * type, clamp_min(eps), rounded division).
 * Replaces: the norm-cache initialisation of init_state
 *   (src/coda_gqa_l/attention.py:309-316). */
int coda_unit_rows(int dtype, void* out, int64_t o_so, int64_t o_si, const void* x, int64_t x_so,
                   int64_t x_si, int64_t outer, int inner, int len, void* stream);

/* Host-only restatement check of the selection order used by the bank
 * kernels (no GPU needed): indices of torch's CPU topk(vals, k, largest,
 * sorted) for float / int64 keys, ties included.  No reference
 * counterpart: exported so the order can be tested against torch.topk. */
int coda_topk_order_host(const float* vals, int n, int k, int largest, int sorted, int64_t* out_idx);
int coda_topk_order_host_i64(const int64_t* vals, int n, int k, int largest, int sorted, int64_t* out_idx);

#ifdef __cplusplus
}
#endif

#endif /* CODA_MI355X_H */
