"""CoDAGQALandmarkPerf2: bounded differential attention with GQA on MI355X.

    out = RMSNorm( Attn(q, K, V) - lambda * Attn(R_theta(q), K, V) )
    K/V = [recent window W | exact landmarks Me | summary landmarks Ms]

Same constructor, parameters (names, shapes, init order), state object and
public methods as the reference (src/coda_gqa_l/attention.py:72-760), so
checkpoints, pickled states and callers carry over.  The projections are
GEMMs on the device; everything on the bounded path after them runs in the
HIP kernels of libcoda_mi355x.so:
  - decode: one bank kernel (ring + exact + summary) and one attention
    kernel per step, no host sync;
  - prefill: one candidate-plan kernel per call, then per chunk one
    attention kernel and three bank kernels, no host sync.
Host syncs remain only for the reference's data-dependent host ints
(dynamic bank expansion, the optional metrics dict).

The layer is inference-only on this path: a module in training mode raises
(the kernels have no backward).
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _hip, ops
from .memory_banks import METRIC_KEYS, DeviceMetrics, MemoryBankMixin
from .primitives import HeadwiseRMSNorm, RotaryEmbedding, apply_rope
from .state import CoDAGQALandmarkStatePerf2

__all__ = ["CoDAGQALandmarkPerf2", "CoDAGQALandmarkStatePerf2"]


class CoDAGQALandmarkPerf2(MemoryBankMixin, nn.Module):
    def __init__(
        self,
        *,
        embed_dim: int,
        num_heads: int,
        num_kv_heads: int,
        window: int,
        num_landmarks_exact: int,
        num_landmarks_summary: int,
        rope_base: float = 10_000.0,
        lambda_init_bias: float = -6.0,
        theta_init: float = math.pi / 2,
        write_policy: str = "gated",
        write_gate_init_bias: float = -2.0,
        write_gate_threshold_exact: float = 0.10,
        write_gate_threshold_summary: float = 0.05,
        exact_match_threshold: float = 0.90,
        exact_novelty_threshold: float = 0.70,
        exact_refresh_on_hit: bool = False,
        exact_candidates_per_block: int = 8,
        summary_eta_init_logit: float = -3.0,
        summary_candidates_per_block: int = 64,
        summary_overwrite_on_insert: bool = True,
        min_landmarks_exact: Optional[int] = None,
        max_landmarks_exact: Optional[int] = None,
        min_landmarks_summary: Optional[int] = None,
        max_landmarks_summary: Optional[int] = None,
        expansion_t_max: int = 1_000_000,
        mem_init: str = "random_normal",
        mask_unused_memory: bool = True,
        detach_evicted: bool = True,
        eps: float = 1e-6,
        collect_metrics: bool = False,
        head_norm_mode: str = "full",
        rope_interleaved: bool = True,
    ):
        super().__init__()
        if embed_dim % num_heads != 0:
            raise ValueError("embed_dim must be divisible by num_heads")
        if num_heads % num_kv_heads != 0:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        if window <= 0:
            raise ValueError("window must be positive")
        if num_landmarks_exact < 0 or num_landmarks_summary < 0:
            raise ValueError("num_landmarks_* must be non-negative")
        self.embed_dim = int(embed_dim)
        self.num_heads = int(num_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = self.embed_dim // self.num_heads
        if self.head_dim % 2 != 0:
            raise ValueError("head_dim must be even (RoPE requirement)")
        self.lf_start = self.head_dim // 2
        self.lf_dim = self.head_dim - self.lf_start
        self.energy_scale = math.sqrt(self.head_dim / self.lf_dim)
        self.window = int(window)
        me, ms = int(num_landmarks_exact), int(num_landmarks_summary)
        self.Me_min = int(min_landmarks_exact) if min_landmarks_exact is not None else me
        self.Me_max = int(max_landmarks_exact) if max_landmarks_exact is not None else me
        self.Ms_min = int(min_landmarks_summary) if min_landmarks_summary is not None else ms
        self.Ms_max = int(max_landmarks_summary) if max_landmarks_summary is not None else ms
        self.expansion_t_max = int(expansion_t_max)
        if self.Me_min > self.Me_max:
            raise ValueError(f"min_landmarks_exact ({self.Me_min}) > max ({self.Me_max})")
        if self.Ms_min > self.Ms_max:
            raise ValueError(f"min_landmarks_summary ({self.Ms_min}) > max ({self.Ms_max})")
        if self.Me_min < 0 or self.Ms_min < 0:
            raise ValueError("min_landmarks_* must be non-negative")
        self.Me = self.Me_max
        self.Ms = self.Ms_max
        self.Lbuf = self.window + self.Me + self.Ms

        D, H, Hkv, Dh = self.embed_dim, self.num_heads, self.num_kv_heads, self.head_dim
        # parameter creation order equals the reference's, so a seeded
        # construction yields identical weights
        self.q_proj = nn.Linear(D, H * Dh, bias=False)
        self.k_proj = nn.Linear(D, Hkv * Dh, bias=False)
        self.v_proj = nn.Linear(D, Hkv * Dh, bias=False)
        self.theta = nn.Parameter(torch.full((H, Dh // 2), float(theta_init)))
        self.lambda_proj = nn.Linear(D, H, bias=True)
        nn.init.constant_(self.lambda_proj.bias, float(lambda_init_bias))
        self.write_policy = write_policy
        self.write_proj = nn.Linear(D, 1, bias=True)
        nn.init.zeros_(self.write_proj.weight)
        nn.init.constant_(self.write_proj.bias, float(write_gate_init_bias))
        self.write_gate_threshold_exact = float(write_gate_threshold_exact)
        self.write_gate_threshold_summary = float(write_gate_threshold_summary)
        self.exact_match_threshold = float(exact_match_threshold)
        self.exact_novelty_threshold = float(exact_novelty_threshold)
        self.exact_refresh_on_hit = bool(exact_refresh_on_hit)
        self.exact_candidates_per_block = int(max(0, exact_candidates_per_block))
        self.summary_eta_logit = nn.Parameter(torch.full((Hkv,), float(summary_eta_init_logit)))
        self.summary_candidates_per_block = int(max(0, summary_candidates_per_block))
        self.summary_overwrite_on_insert = bool(summary_overwrite_on_insert)
        self.mem_init = mem_init
        self.mask_unused_memory = bool(mask_unused_memory)
        self.detach_evicted = bool(detach_evicted)
        self.collect_metrics = bool(collect_metrics)
        self.rope_interleaved = bool(rope_interleaved)
        self.rope = RotaryEmbedding(Dh, base=float(rope_base))
        self.head_norm_mode = head_norm_mode
        if head_norm_mode == "full":
            self.head_norm = HeadwiseRMSNorm(Dh, eps=eps)
        elif head_norm_mode == "identity":
            self.head_norm = nn.Identity()
        else:
            raise ValueError(f"head_norm_mode must be 'full' or 'identity', got {head_norm_mode!r}")
        self.o_proj = nn.Linear(H * Dh, D, bias=False)
        self._eps = float(eps)
        # prefill_core: run the chunks whose ring window lies in the call as a
        # bank chain with snapshots and grouped attention launches (False:
        # chunk by chunk, attention then bank update; the same results up to
        # the order of the softmax sums)
        self.pipelined_prefill = True
        # chunks per attention launch of the pipelined prefill (None: as many
        # as 256 MiB of bank snapshots hold, at most 1024)
        self.pipelined_group_chunks: Optional[int] = None
        self._check_bank_sizes()

    # ------------------------------------------------------------ state
    def init_state(self, *, batch_size: int, device: torch.device, dtype: torch.dtype,
                   mem_init: Optional[str] = None) -> CoDAGQALandmarkStatePerf2:
        """Zero buffers, N(0, 0.02) bank init, norm caches (attention.py:247-338).

        The random bank init draws from the torch CPU generator with the
        reference's call sequence, so a given torch.manual_seed yields the
        same initial banks as the reference's CPU path; the norm caches are
        computed on the device by the HIP normaliser.
        """
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("coda_gqa_l (MI355X build) keeps its state on a HIP device; got " + str(device))
        B, Hkv, Dh, W, Me, Ms = int(batch_size), self.num_kv_heads, self.head_dim, self.window, self.Me, self.Ms
        mode = mem_init if mem_init is not None else self.mem_init
        if mode not in ("zeros", "random_normal"):
            raise ValueError("mem_init must be 'zeros' or 'random_normal'")
        k_host = torch.zeros((B, Hkv, self.Lbuf, Dh), dtype=dtype)
        v_host = torch.zeros((B, Hkv, self.Lbuf, Dh), dtype=dtype)
        if mode == "random_normal":
            if Me > 0:
                k_host[:, :, W:W + Me, :].normal_(mean=0.0, std=0.02)
                v_host[:, :, W:W + Me, :].normal_(mean=0.0, std=0.02)
            if Ms > 0:
                k_host[:, :, W + Me:, self.lf_start:].normal_(mean=0.0, std=0.02)
                v_host[:, :, W + Me:, :].normal_(mean=0.0, std=0.02)
        k_buf = k_host.to(device)
        v_buf = v_host.to(device)
        st = CoDAGQALandmarkStatePerf2(
            k_buf=k_buf, v_buf=v_buf, allowed=torch.zeros((B, self.Lbuf), dtype=torch.bool, device=device),
            g_recent=torch.zeros((B, W), dtype=torch.float32, device=device), recent_idx=0, recent_filled=0,
            mem_last_exact=torch.zeros((B, Me), dtype=torch.int64, device=device), pos=0,
            active_exact=self.Me_min if Me > 0 else 0, active_summary=self.Ms_min if Ms > 0 else 0)
        L = _hip.lib()
        code = _hip.dtype_code(dtype)
        stream = _hip.stream_of(k_buf)
        if Me > 0:
            st._exact_v_norm = torch.empty((B, Hkv, Me, Dh), dtype=dtype, device=device)
            _hip.check(L.coda_unit_rows(code, st._exact_v_norm.data_ptr(), Me * Dh, Dh,
                                        v_buf[:, :, W:W + Me].data_ptr(), self.Lbuf * Dh, Dh, B * Hkv, Me, Dh,
                                        stream))
        if Ms > 0:
            LF = self.lf_dim
            st._sum_lf_k_norm = torch.empty((B, Hkv, Ms, LF), dtype=dtype, device=device)
            _hip.check(L.coda_unit_rows(code, st._sum_lf_k_norm.data_ptr(), Ms * LF, LF,
                                        k_buf[:, :, W + Me:, self.lf_start:].data_ptr(), self.Lbuf * Dh, Dh,
                                        B * Hkv, Ms, LF, stream))
        if self.collect_metrics:
            st.metrics = DeviceMetrics({k: (0.0 if k.endswith("ratio") else 0) for k in METRIC_KEYS})
            st.metrics["active_exact"] = st.active_exact
            st.metrics["active_summary"] = st.active_summary
        return st

    # ------------------------------------------------------------ expansion
    def _log_ceiling(self, tokens_seen: int) -> Tuple[int, int]:
        """Capacity ceiling after `tokens_seen` tokens (attention.py:344-356)."""
        if self.expansion_t_max <= 0:
            return self.Me_max, self.Ms_max
        ratio = min(math.log(1 + tokens_seen) / math.log(1 + self.expansion_t_max), 1.0)
        return (self.Me_min + int((self.Me_max - self.Me_min) * ratio),
                self.Ms_min + int((self.Ms_max - self.Ms_min) * ratio))

    def _try_expand(self, state: CoDAGQALandmarkStatePerf2, frustrated_exact: int, frustrated_summary: int) -> None:
        """Grow the active bank sizes under pressure (attention.py:358-390)."""
        if self.Me_min == self.Me_max and self.Ms_min == self.Ms_max:
            return
        if frustrated_exact <= 0 and frustrated_summary <= 0:
            return
        ce, cs = self._log_ceiling(state.pos)
        de = ds = 0
        if frustrated_exact > 0 and state.active_exact < ce:
            de = min(frustrated_exact, ce - state.active_exact)
            state.active_exact += de
        if frustrated_summary > 0 and state.active_summary < cs:
            ds = min(frustrated_summary, cs - state.active_summary)
            state.active_summary += ds
        if state.metrics is not None:
            state.metrics["active_exact"] = state.active_exact
            state.metrics["active_summary"] = state.active_summary
            state.metrics["expansions_exact"] += de
            state.metrics["expansions_summary"] += ds

    # ------------------------------------------------------------ projections
    def _inference_only(self):
        if self.training:
            raise NotImplementedError("CoDAGQALandmarkPerf2 on MI355X is inference-only (no backward kernels); "
                                      "call .eval()")
        # a give-up of an earlier prefill call's bank update, once its status
        # copy has landed (no host sync)
        if self.__dict__.get("_status_pending"):
            self.check_bank_status(wait=False)

    def _project_q(self, x: torch.Tensor) -> torch.Tensor:
        """(B, L, D) -> (B, H, L, Dh) view of the projection."""
        B, L, _ = x.shape
        return self.q_proj(x).view(B, L, self.num_heads, self.head_dim).permute(0, 2, 1, 3)

    def _project_kv_raw(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        B, L, _ = x.shape
        k = self.k_proj(x).view(B, L, self.num_kv_heads, self.head_dim).permute(0, 2, 1, 3)
        v = self.v_proj(x).view(B, L, self.num_kv_heads, self.head_dim).permute(0, 2, 1, 3)
        return k, v

    def _write_gate(self, x: torch.Tensor) -> torch.Tensor:
        """(B, L) float32 write gate (attention.py:406-410)."""
        B, L, _ = x.shape
        if self.write_policy == "none":
            return torch.ones((B, L), dtype=torch.float32, device=x.device)
        return torch.sigmoid(self.write_proj(x)).squeeze(-1).to(torch.float32)

    def _lambda(self, x: torch.Tensor) -> torch.Tensor:
        """(B, H, L) view of sigmoid(lambda_proj(x))."""
        return torch.sigmoid(self.lambda_proj(x)).permute(0, 2, 1)

    def _theta_tables(self, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        """cos / sin of the noise angles in the compute dtype (attention.py:504-506)."""
        th = self.theta
        return self._derived("theta", th, dtype, lambda: (torch.cos(th).to(dtype=dtype).contiguous(),
                                                          torch.sin(th).to(dtype=dtype).contiguous()))

    def _rms_weight(self, dtype) -> Optional[torch.Tensor]:
        if self.head_norm_mode != "full":
            return None
        w = self.head_norm.weight
        return self._derived("rms_w", w, dtype, lambda: w.detach().to(dtype).contiguous())

    # ------------------------------------------------------------ projection front end
    def _rope_rows(self, p0: int, L: int, device, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        """RoPE tables (L, Dh/2) of positions p0 .. p0 + L - 1: rows of one
        cached table, grown by doubling; every element is the same fp32
        product and cos / sin as in a table made for these positions alone."""
        cache = self.__dict__.setdefault("_rope_cache", {})
        key = (torch.device(device), dtype)
        tab = cache.get(key)
        need = int(p0) + int(L)
        if tab is None or tab[0].shape[0] < need:
            n = 1 << max(12, (need - 1).bit_length())
            c, s_ = self.rope(seq_len=n, offset=0, device=device, dtype=dtype)
            tab = cache[key] = (c.contiguous(), s_.contiguous())
        return tab[0][p0:need], tab[1][p0:need]

    def _proj_pack(self, dtype: torch.dtype):
        """Packed [q | k | v | lambda | write] weights (n_feat, D) in `dtype`,
        float32 biases (zero for a linear without one) and the weights'
        layout code for coda_project, per parameter version; with half-split
        RoPE each k head's rows are reordered to the pairs (i, i + Dh/2) on
        adjacent rows.  Where the row kernel serves D the weights are kept in
        its fragment tiles (coda_project_pack, layout 1), else row-major (0)."""
        lins = (self.q_proj, self.k_proj, self.v_proj, self.lambda_proj, self.write_proj)
        ps = [t for lin in lins for t in (lin.weight, lin.bias) if t is not None]
        tag = tuple((t._version, t.data_ptr(), t.dtype, t.device) for t in ps) + (self.rope_interleaved,
                                                                                 self.write_policy)
        cache = self.__dict__.setdefault("_derived_cache", {})
        hit = cache.get(("proj", dtype))
        if hit is not None and hit[0] == tag:
            return hit[1]
        H, Hkv, Dh = self.num_heads, self.num_kv_heads, self.head_dim
        gate = self.write_policy != "none"
        with torch.no_grad():
            dev = self.q_proj.weight.device
            wk, bk = self.k_proj.weight, self.k_proj.bias
            if not self.rope_interleaved:
                half = Dh // 2
                pair = torch.stack([torch.arange(half), torch.arange(half) + half], 1).reshape(-1)
                perm = (torch.arange(Hkv)[:, None] * Dh + pair[None]).reshape(-1).to(dev)
                wk = wk[perm]
                bk = bk[perm] if bk is not None else None
            ws = [self.q_proj.weight, wk, self.v_proj.weight, self.lambda_proj.weight]
            bt = [self.q_proj.bias, bk, self.v_proj.bias, self.lambda_proj.bias]
            if gate:
                ws.append(self.write_proj.weight)
                bt.append(self.write_proj.bias)
            w = torch.cat([t.detach() for t in ws]).to(dtype)
            b = torch.cat([t.detach().float() if t is not None else torch.zeros(wt.shape[0], device=dev)
                           for t, wt in zip(bt, ws)])
            b = torch.cat([b, torch.zeros((-b.numel()) % 4, device=dev)])
            w = w.contiguous()
            layout = 0
            if dtype == torch.bfloat16 and w.is_cuda:
                n_feat, D = w.shape
                wt = torch.empty((-(-n_feat // 64) * 64, D), dtype=dtype, device=dev)
                rc = _hip.lib().coda_project_pack(w.data_ptr(), n_feat, D, D, wt.data_ptr(), _hip.stream_of(wt))
                if rc == _hip.CODA_OK:
                    w, layout = wt, 1
                elif rc != _hip.CODA_EUNSUP:
                    _hip.check(rc)
        val = (w, b.contiguous(), layout)
        cache[("proj", dtype)] = (tag, val)
        return val

    def _proj_desc(self, x: torch.Tensor, M: int, L: int, cos: torch.Tensor, sin: torch.Tensor):
        d = _hip.ProjDesc()
        d.dtype, d.M, d.D, d.L = _hip.dtype_code(x.dtype), M, self.embed_dim, L
        d.H, d.Hkv, d.Dh = self.num_heads, self.num_kv_heads, self.head_dim
        d.rope_interleaved, d.gate = int(self.rope_interleaved), int(self.write_policy != "none")
        d.rope_cos, d.rope_sin = cos.data_ptr(), sin.data_ptr()
        return d

    def _fused_front_ok(self, x: torch.Tensor) -> bool:
        """Whether coda_project serves x: bf16, at most 64 token rows, D a
        multiple of 64, head_dim a multiple of 4."""
        B, L, D = x.shape
        return x.dtype == torch.bfloat16 and B * L <= 64 and D % 64 == 0 and self.head_dim % 4 == 0

    def _front(self, x: torch.Tensor, p0: int, fused: bool = False):
        """Projections of x (B, L, D) at positions p0 ..: q (B,H,L,Dh)
        pre-RoPE, k (B,Hkv,L,Dh) roped, v (B,Hkv,L,Dh), g (B,L) float32,
        lam (B,H,L), and the RoPE tables (L, Dh/2) (attention.py:396-410,
        592-608).  fused (decode-shaped input, _fused_front_ok): one launch of
        the hand-written projection kernel with its RoPE and sigmoid
        epilogues (coda_project), outputs in the torch path's layouts.
        Otherwise the torch linears and the RoPE kernel.  A fused form for
        many token rows (a library GEMM over the packed weights, an epilogue
        kernel in place, q / k / v / lambda as strided views of its output)
        faulted the GPU once in a full-size prefill, with no cause shown; it
        was removed, and prefill keeps the torch linears."""
        B, L, D = x.shape
        H, Hkv, Dh = self.num_heads, self.num_kv_heads, self.head_dim
        Fq, Fk = H * Dh, Hkv * Dh
        M = B * L
        if fused:
            if not self._fused_front_ok(x):
                raise NotImplementedError(
                    "the fused projection front end serves bf16 inputs of at most 64 token rows (decode); many "
                    "rows take the torch linears: a many-row fused form (an in-place epilogue over a library GEMM, "
                    "q / k / v / lambda as strided views of its output) faulted the GPU in a full-size run with no "
                    "cause shown, and was removed")
            cos, sin = self._rope_rows(p0, L, x.device, x.dtype)
            d = self._proj_desc(x, M, L, cos, sin)
            g = torch.empty((B, L), dtype=torch.float32, device=x.device)
            d.g = g.data_ptr()
            xs = x if (x.is_contiguous() and x.data_ptr() % 16 == 0) else x.contiguous()
            w, b, d.w_layout = self._proj_pack(x.dtype)
            q = torch.empty((B, L, Fq), dtype=x.dtype, device=x.device)
            k = torch.empty((B, L, Hkv, Dh), dtype=x.dtype, device=x.device)
            v = torch.empty((B, L, Fk), dtype=x.dtype, device=x.device)
            lam = torch.empty((B, L, H), dtype=x.dtype, device=x.device)
            d.x, d.x_sm, d.w, d.bias = xs.data_ptr(), D, w.data_ptr(), b.data_ptr()
            d.q, d.q_sm, d.k, d.k_sm, d.v, d.v_sm = q.data_ptr(), Fq, k.data_ptr(), Fk, v.data_ptr(), Fk
            d.lam, d.lam_sm = lam.data_ptr(), H
            nb = self.__dict__.setdefault("_proj_ws_bytes", {})
            key = (M, D, H, Hkv, Dh, d.gate)
            if key not in nb:
                n = ctypes.c_size_t(0)
                _hip.check(_hip.lib().coda_project_workspace_bytes(d, n))
                nb[key] = n.value
            ws = None
            if nb[key]:
                cache = self.__dict__.setdefault("_proj_ws", {})
                ws = cache.get(str(x.device))
                if ws is None or ws.numel() < nb[key]:
                    ws = cache[str(x.device)] = torch.empty(nb[key], dtype=torch.uint8, device=x.device)
            d.workspace, d.workspace_bytes = _hip.ptr(ws), nb[key]
            _hip.check(_hip.lib().coda_project(d, _hip.stream_of(x)))
            return (q.view(B, L, H, Dh).permute(0, 2, 1, 3), k.permute(0, 2, 1, 3),
                    v.view(B, L, Hkv, Dh).permute(0, 2, 1, 3), g, lam.permute(0, 2, 1), cos, sin)
        cos, sin = self.rope(seq_len=L, offset=p0, device=x.device, dtype=x.dtype)
        cos, sin = cos.contiguous(), sin.contiguous()
        q = self._project_q(x)
        k_raw, v = self._project_kv_raw(x)
        # roped keys in the token-major layout of v, so K and V share strides
        k = torch.empty((B, L, Hkv, Dh), dtype=x.dtype, device=x.device).permute(0, 2, 1, 3)
        apply_rope(k_raw, cos, sin, interleaved=self.rope_interleaved, out=k)
        return q, k, v, self._write_gate(x), self._lambda(x), cos, sin

    # ------------------------------------------------------------ decode
    def decode_attend_core(self, q: torch.Tensor, lam: torch.Tensor, state: CoDAGQALandmarkStatePerf2,
                           rope_cos: torch.Tensor, rope_sin: torch.Tensor,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Attention of one token over the bounded cache: q (B,H,1,Dh)
        pre-RoPE, lam (B,H,1), tables (1, Dh/2) at the query position.
        Returns head outputs (B, 1, H, Dh)."""
        B = q.shape[0]
        H, Dh = self.num_heads, self.head_dim
        if out is None:
            out = torch.empty((B, 1, H, Dh), dtype=q.dtype, device=q.device)
        ct, sn = self._theta_tables(q.dtype)
        ops.bounded_attention(
            q=q, rope_cos=rope_cos.contiguous(), rope_sin=rope_sin.contiguous(),
            rope_interleaved=self.rope_interleaved, theta_cos=ct, theta_sin=sn, k_prefix=state.k_buf,
            v_prefix=state.v_buf, allowed=state.allowed if self.mask_unused_memory else None, k_block=None,
            v_block=None, lam=lam, rms_weight=self._rms_weight(q.dtype), eps=self._eps,
            out=out.permute(0, 2, 1, 3))
        return out

    def decode_step_core(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, g_new: torch.Tensor,
                         lam: torch.Tensor, state: CoDAGQALandmarkStatePerf2, rope_cos: torch.Tensor,
                         rope_sin: torch.Tensor, out: Optional[torch.Tensor] = None,
                         k_roped: bool = True) -> torch.Tensor:
        """Write one token into the bounded cache, then attend with its query
        (attention.py:526-536 after the projections), as one library call.

        q (B,H,1,Dh) pre-RoPE, k_new (B,Hkv,1,Dh) roped (k_roped False: the
        raw k projection, roped inside the step with the same tables), v_new,
        g_new (B,) float32, lam (B,H,1), tables (1, Dh/2) at the token's
        position.  Returns head outputs (B, 1, H, Dh)."""
        B = q.shape[0]
        H, Dh = self.num_heads, self.head_dim
        if out is None:
            out = torch.empty((B, 1, H, Dh), dtype=q.dtype, device=q.device)
        if self._decode_step_planned(state, q, k_new, v_new, g_new, lam, rope_cos, rope_sin, out, k_roped):
            return out
        self._check_state(state)
        ct, sn = self._theta_tables(q.dtype)
        desc, keep = ops.attention_desc(
            q=q, rope_cos=rope_cos.contiguous(), rope_sin=rope_sin.contiguous(),
            rope_interleaved=self.rope_interleaved, theta_cos=ct, theta_sin=sn, k_prefix=state.k_buf,
            v_prefix=state.v_buf, allowed=state.allowed if self.mask_unused_memory else None, k_block=None,
            v_block=None, lam=lam, rms_weight=self._rms_weight(q.dtype), eps=self._eps,
            out=out.permute(0, 2, 1, 3))
        self._decode_step(state, k_new=k_new, v_new=v_new, g_new=g_new, attn_desc=desc, k_roped=k_roped)
        return out

    def attend_step(self, x: torch.Tensor, state: CoDAGQALandmarkStatePerf2, *,
                    query_pos: Optional[int] = None) -> torch.Tensor:
        """Attend one token over the current cache (attention.py:476-514)."""
        self._inference_only()
        _hip.require_device(x)
        B, L, _ = x.shape
        assert L == 1
        self._check_state(state)
        qp = int(state.pos if query_pos is None else query_pos)
        cos, sin = self.rope(seq_len=1, offset=qp, device=x.device, dtype=x.dtype)
        heads = self.decode_attend_core(self._project_q(x), self._lambda(x), state, cos, sin)
        return self.o_proj(heads.view(B, 1, self.num_heads * self.head_dim))

    def step(self, x: torch.Tensor, state: CoDAGQALandmarkStatePerf2, *, attend: bool = True,
             write_cache: bool = True, include_current_in_attention: bool = True
             ) -> Tuple[torch.Tensor, CoDAGQALandmarkStatePerf2]:
        """One decode token (attention.py:516-547): by default write, then attend."""
        self._inference_only()
        _hip.require_device(x)
        B, L, _ = x.shape
        assert L == 1
        q_pos = int(state.pos)

        def write():
            k_raw, v_new = self._project_kv_raw(x)
            cosk, sink = self.rope(seq_len=1, offset=q_pos, device=x.device, dtype=x.dtype)
            k_new = apply_rope(k_raw, cosk, sink, interleaved=self.rope_interleaved)
            self._write_one(state, k_new=k_new, v_new=v_new, g_new=self._write_gate(x))

        if attend and include_current_in_attention and write_cache:
            y = self._step_fast(x, state)
            if y is not None:
                return y, state
            self._check_state(state)
            if self._fused_front_ok(x):
                # one launch for q / k (roped) / v / lambda / gate
                q, k_new, v_new, g, lam, cos, sin = self._front(x, q_pos, fused=True)
                heads = self.decode_step_core(q, k_new, v_new, g.reshape(B), lam, state, cos, sin, k_roped=True)
                return self.o_proj(heads.view(B, 1, self.num_heads * self.head_dim)), state
            # the raw k projection: the step ropes it with the query's tables
            cos, sin = self.rope(seq_len=1, offset=q_pos, device=x.device, dtype=x.dtype)
            k_raw, v_new = self._project_kv_raw(x)
            heads = self.decode_step_core(self._project_q(x), k_raw, v_new, self._write_gate(x).reshape(B),
                                          self._lambda(x), state, cos.contiguous(), sin.contiguous(), k_roped=False)
            return self.o_proj(heads.view(B, 1, self.num_heads * self.head_dim)), state
        y = self.attend_step(x, state, query_pos=q_pos) if attend else torch.zeros_like(x)
        if write_cache:
            write()
        return y, state

    def _step_fast(self, x: torch.Tensor, st: CoDAGQALandmarkStatePerf2) -> Optional[torch.Tensor]:
        """A steady-state decode step (full ring, fixed bank sizes, no
        metrics or traces, bf16 decode-shaped input) from descriptors and
        buffers cached per state: per token the host sets the input and
        RoPE-row pointers, makes two library calls (coda_project, then
        coda_decode_step on its outputs) and the o_proj GEMM.  Returns None
        when the general path must run; the cache is rebuilt whenever a
        parameter, the state's tensors (object, storage or in-place version)
        or the batch changes."""
        if not self._fused_front_ok(x) or st.metrics is not None or st.recent_filled < self.window or \
                self._expandable() or (self.Me == 0 and self.Ms == 0) or self._tracing():
            return None
        fp = self.__dict__.get("_fast")
        ts = (st.k_buf, st.v_buf, st.allowed, st.g_recent, st.mem_last_exact, st._exact_v_norm, st._sum_lf_k_norm)
        vers = tuple(-1 if t is None else t._version for t in ts)
        pvers = self._param_key()
        B = x.shape[0]
        if fp is None or fp["st"] is not st or fp["vers"] != vers or fp["pvers"] != pvers or fp["B"] != B or \
                fp["ptrs"] != tuple(-1 if t is None else t.data_ptr() for t in ts) or fp["dev"] != x.device:
            fp = self._build_step_fast(x, st, ts, vers, pvers)
            if fp is None:
                return None
        if not (x.is_contiguous() and x.data_ptr() % 16 == 0):
            x = x.contiguous()
        pos = int(st.pos)
        cos_t, sin_t = fp["tab"]
        if pos >= cos_t.shape[0]:
            cos_t, sin_t = self._rope_rows(0, pos + 1, x.device, x.dtype)
            fp["tab"] = (cos_t, sin_t)
        row = fp["row_bytes"] * pos
        d, a = fp["proj"], fp["attn"]
        d.x = x.data_ptr()
        d.rope_cos = a.rope_cos = cos_t.data_ptr() + row
        d.rope_sin = a.rope_sin = sin_t.data_ptr() + row
        stream = _hip.stream_of(x)
        _hip.check(fp["project"](fp["proj_ref"], stream))
        routed = fp["routed"]
        routed.value = 1 if fp["record_pos"] == pos else 0
        j = int(st.recent_idx)
        _hip.check(fp["step"](fp["bank_ref"], fp["attn_ref"], fp["k_ptr"], fp["v_ptr"], fp["k_sb"], fp["k_sh"],
                              fp["g_ptr"], j, int(st.recent_filled), pos, fp["ws_ptr"], fp["ws_bytes"],
                              fp["routed_ref"], stream))
        st.recent_idx = 0 if j + 1 == self.window else j + 1
        st.pos = pos + 1
        fp["record_pos"] = pos + 1 if routed.value else -1
        # the general path's carried-record tag no longer matches this state
        self.__dict__["_route_tag"] = None
        return self.o_proj(fp["heads_flat"])

    def _param_key(self) -> tuple:
        """Identity and in-place version of every parameter of the layer and
        of its (leaf) submodules, without the recursive module walk."""
        out = []
        for p in self._parameters.values():
            if p is not None:
                out += (id(p), p._version)
        for mod in self._modules.values():
            for p in mod._parameters.values():
                if p is not None:
                    out += (id(p), p._version)
        return tuple(out)

    def _build_step_fast(self, x, st, ts, vers, pvers):
        """Descriptors and persistent buffers of _step_fast (see there)."""
        self.__dict__["_fast"] = None
        self._check_state(st)
        ts = (st.k_buf, st.v_buf, st.allowed, st.g_recent, st.mem_last_exact, st._exact_v_norm, st._sum_lf_k_norm)
        vers = tuple(-1 if t is None else t._version for t in ts)
        B, L, D = x.shape
        H, Hkv, Dh = self.num_heads, self.num_kv_heads, self.head_dim
        dev, dt = x.device, x.dtype
        if st.k_buf.dtype != dt:
            return None
        Fq, Fk = H * Dh, Hkv * Dh
        q = torch.empty((B, 1, Fq), dtype=dt, device=dev)
        k = torch.empty((B, 1, Hkv, Dh), dtype=dt, device=dev)
        v = torch.empty((B, 1, Fk), dtype=dt, device=dev)
        lam = torch.empty((B, 1, H), dtype=dt, device=dev)
        g = torch.empty((B, 1), dtype=torch.float32, device=dev)
        heads = torch.empty((B, 1, H, Dh), dtype=dt, device=dev)
        pos = int(st.pos)
        cos_t, sin_t = self._rope_rows(0, pos + 1, dev, dt)
        cos_t, sin_t = self.__dict__["_rope_cache"][(torch.device(dev), dt)]
        d = self._proj_desc(x, B, 1, cos_t, sin_t)
        w, b, d.w_layout = self._proj_pack(dt)
        d.x_sm, d.w, d.bias = D, w.data_ptr(), b.data_ptr()
        d.q, d.q_sm, d.k, d.k_sm, d.v, d.v_sm = q.data_ptr(), Fq, k.data_ptr(), Fk, v.data_ptr(), Fk
        d.lam, d.lam_sm, d.g = lam.data_ptr(), H, g.data_ptr()
        nb = ctypes.c_size_t(0)
        _hip.check(_hip.lib().coda_project_workspace_bytes(d, nb))
        pws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=dev) if nb.value else None
        d.workspace, d.workspace_bytes = _hip.ptr(pws), nb.value
        qv = q.view(B, 1, H, Dh).permute(0, 2, 1, 3)
        lamv = lam.permute(0, 2, 1)
        ct, sn = self._theta_tables(dt)
        a, keep = ops.attention_desc(
            q=qv, rope_cos=cos_t[pos:pos + 1], rope_sin=sin_t[pos:pos + 1], rope_interleaved=self.rope_interleaved,
            theta_cos=ct, theta_sin=sn, k_prefix=st.k_buf, v_prefix=st.v_buf,
            allowed=st.allowed if self.mask_unused_memory else None, k_block=None, v_block=None, lam=lamv,
            rms_weight=self._rms_weight(dt), eps=self._eps, out=heads.permute(0, 2, 1, 3))
        eta = self._eta_f32(dev, st.k_buf.dtype) if self.Ms > 0 else None
        bank = self._bank_desc(st, eta, None, None)
        nb = ctypes.c_size_t(0)
        _hip.check(_hip.lib().coda_decode_step_workspace_bytes(bank, a, nb))
        ws = self._route_workspace(dev, nb.value)
        # a record the general path left for this very state and position
        routed_pos = pos if self.__dict__.get("_route_tag") == self._route_key(st, ws) else -1
        L_ = _hip.lib()
        routed = ctypes.c_int(0)

        fp = {"st": st, "vers": vers, "pvers": pvers, "B": B, "dev": dev,
              "ptrs": tuple(-1 if t is None else t.data_ptr() for t in ts),
              "tab": (cos_t, sin_t), "row_bytes": (Dh // 2) * cos_t.element_size(),
              "proj": d, "proj_ref": ctypes.byref(d), "attn": a, "attn_ref": ctypes.byref(a),
              "bank": bank, "bank_ref": ctypes.byref(bank),
              "keep": (keep, q, k, v, lam, g, heads, w, b, pws, ws, ct, sn, eta, self._rms_weight(dt)),
              "k_ptr": k.data_ptr(), "v_ptr": v.data_ptr(), "k_sb": Fk, "k_sh": Dh, "g_ptr": g.data_ptr(),
              "ws_ptr": _hip.ptr(ws), "ws_bytes": nb.value, "routed": routed, "routed_ref": ctypes.byref(routed),
              "record_pos": routed_pos, "project": L_.coda_project, "step": L_.coda_decode_step,
              "heads_flat": heads.view(B, 1, H * Dh)}
        self.__dict__["_fast"] = fp
        return fp

    # ------------------------------------------------------------ prefill
    def prefill_core(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, lam: torch.Tensor,
                     rope_cos: torch.Tensor, rope_sin: torch.Tensor, state: CoDAGQALandmarkStatePerf2, *,
                     block_size: int, write_cache: bool = True, return_heads: bool = True,
                     out: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
        """The chunk loop after the projections (attention.py:611-724).

        q (B,H,L,Dh) pre-RoPE; k (B,Hkv,L,Dh) post-RoPE; v (B,Hkv,L,Dh);
        g (B,L) float32; lam (B,H,L); tables (L, Dh/2) of the positions.
        Returns head outputs (B, L, H, Dh) when return_heads.
        """
        B, H, L, Dh = q.shape
        if return_heads and out is None:
            out = torch.empty((B, L, H, Dh), dtype=q.dtype, device=q.device)
        ct, sn = self._theta_tables(q.dtype)
        w = self._rms_weight(q.dtype)
        self._check_state(state)
        g = g if g.stride(-1) == 1 else g.contiguous()
        plan = kmax = None
        do_e = do_s = False
        ws = eta = None
        head = int(state.recent_idx) if state.recent_filled >= self.window else 0
        filled = int(state.recent_filled)
        if write_cache:
            te = min(self.exact_candidates_per_block, block_size) if self.Me > 0 else 0
            ts = min(self.summary_candidates_per_block, block_size) if self.Ms > 0 else 0
            ck = (B, state.k_buf.dtype, te, ts, self.Me_max, self.Ms_max)
            if self.__dict__.get("_block_checked") != ck:
                self._block_check(B, state.k_buf.dtype, te, ts)
                self.__dict__["_block_checked"] = ck
            plan, kmax, do_e, do_s = self._plan_candidates(state, g, L, block_size)
            ws = self._block_workspace(state, kmax)
            eta = self._eta_f32(q.device, state.k_buf.dtype) if self.Ms > 0 else None
        p0 = int(state.pos)
        t = 0
        c = 0
        if write_cache and return_heads and self.pipelined_prefill and self._pipelined_ok(q, k, v, state, block_size):
            # chunks whose ring window lies in this call: the bank chain
            # leaves per-chunk snapshots, then one attention launch per group
            c0 = 0 if state.recent_filled == 0 else -(-self.window // block_size)
            n_chunks = -(-L // block_size)
            if c0 < n_chunks:
                while c < c0:
                    blk = block_size
                    ops.bounded_attention(
                        q=q[:, :, t:t + blk], rope_cos=rope_cos[t:t + blk], rope_sin=rope_sin[t:t + blk],
                        rope_interleaved=self.rope_interleaved, theta_cos=ct, theta_sin=sn, k_prefix=state.k_buf,
                        v_prefix=state.v_buf, allowed=state.allowed if self.mask_unused_memory else None,
                        k_block=k[:, :, t:t + blk], v_block=v[:, :, t:t + blk], lam=lam[:, :, t:t + blk],
                        rms_weight=w, eps=self._eps, out=out[:, t:t + blk].permute(0, 2, 1, 3))
                    head, filled = self._write_block(
                        state, k_blk=k[:, :, t:t + blk], v_blk=v[:, :, t:t + blk], g_blk=g[:, t:t + blk],
                        pos0=p0 + t, ring_head=head, ring_filled=filled, plan_c=plan[c], kmax=kmax, do_e=do_e,
                        do_s=do_s, workspace=ws, eta=eta)
                    state.pos = p0 + t + blk
                    t += blk
                    c += 1
                c, t, head, filled = self._prefill_pipelined(
                    q, k, v, g, lam, rope_cos, rope_sin, state, block_size, out, ct, sn, w, plan, kmax, do_e, do_s,
                    ws, eta, c, head, filled, p0)
        while t < L:
            blk = min(int(block_size), L - t)
            if return_heads:
                ops.bounded_attention(
                    q=q[:, :, t:t + blk], rope_cos=rope_cos[t:t + blk], rope_sin=rope_sin[t:t + blk],
                    rope_interleaved=self.rope_interleaved, theta_cos=ct, theta_sin=sn, k_prefix=state.k_buf,
                    v_prefix=state.v_buf, allowed=state.allowed if self.mask_unused_memory else None,
                    k_block=k[:, :, t:t + blk], v_block=v[:, :, t:t + blk], lam=lam[:, :, t:t + blk],
                    rms_weight=w, eps=self._eps, out=out[:, t:t + blk].permute(0, 2, 1, 3))
            if write_cache:
                head, filled = self._write_block(
                    state, k_blk=k[:, :, t:t + blk], v_blk=v[:, :, t:t + blk], g_blk=g[:, t:t + blk],
                    pos0=p0 + t, ring_head=head, ring_filled=filled, plan_c=plan[c], kmax=kmax, do_e=do_e,
                    do_s=do_s, workspace=ws, eta=eta)
                state.pos = p0 + t + blk
            t += blk
            c += 1
        if write_cache:
            self._ring_to_time_order(state, head, filled)
            self._queue_status_check(ws)
        return out

    def _pipelined_ok(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, state: CoDAGQALandmarkStatePerf2,
                      block_size: int) -> bool:
        """Whether prefill_core's chunks may run as a bank chain with
        snapshots followed by one attention launch per group: the conditions
        of coda_prefill_attn_chunks (bf16, head_dim 64 / 128, G in {1, 2,
        4, 8}, the MFMA flash path, 31-bit per-lane key offsets) and banks
        with candidates, so that every chunk's update is one launch."""
        B, H, L, Dh = q.shape
        G = H // self.num_kv_heads
        return (q.dtype == torch.bfloat16 and state.k_buf.dtype == torch.bfloat16 and Dh in (64, 128) and
                G in (1, 2, 4, 8) and self.Me + self.Ms > 0 and min(int(block_size), L) * G > 8 and
                k.stride() == v.stride() and k.stride(-1) == 1 and
                (self.window + int(block_size) + 64) * k.stride(2) < (1 << 30) and
                (self.Me > 0 and self.exact_candidates_per_block > 0 or
                 self.Ms > 0 and self.summary_candidates_per_block > 0))

    def _prefill_pipelined(self, q, k, v, g, lam, rope_cos, rope_sin, state, block_size, out, ct, sn, w, plan, kmax,
                           do_e, do_s, ws, eta, c, head, filled, p0):
        """Chunks c .. of prefill_core whose ring window lies in this call
        (attention.py:611-724): per group of chunks, first every chunk's bank
        update in order, each leaving the bank slots it starts from in a
        snapshot, then the group's attention in one launch over the call's
        keys (coda_prefill_attn_chunks).  Falls back to the chunk-by-chunk
        loop (returning where it stopped) when the one-launch bank update
        does not run."""
        B, H, L, Dh = q.shape
        Hkv, W, S = self.num_kv_heads, self.window, self.Me + self.Ms
        blk = int(block_size)
        n_chunks = -(-L // blk)
        # snapshot buffers of up to 256 MiB (at most 1024 chunks), made once
        # per shape and kept: calls of any length reuse them
        per_chunk = 2 * B * Hkv * S * Dh * q.element_size()
        cap = max(1, min(1024, (256 << 20) // max(per_chunk, 1)))
        if self.pipelined_group_chunks is not None:
            cap = max(1, min(cap, int(self.pipelined_group_chunks)))
        group = min(n_chunks - c, cap)
        cache = self.__dict__.setdefault("_snap_cache", {})
        key = (str(q.device), q.dtype, B, Hkv, S, Dh)
        buf = cache.get(key)
        if buf is None or buf[0].shape[0] != cap:
            buf = cache[key] = (torch.empty((cap, B, Hkv, S, Dh), dtype=q.dtype, device=q.device),
                                torch.empty((cap, B, Hkv, S, Dh), dtype=q.dtype, device=q.device),
                                torch.empty((cap, B, S), dtype=torch.uint8, device=q.device))
        sk, sv, sa = buf
        # chunks that evict run as one chain call when no metrics, flags or
        # traces are collected per chunk
        chain = (state.metrics is None and not (self._expandable() and not self.training) and
                 not self._tracing() and ws is not None)
        ring = (ctypes.c_int * 2)()
        while c < n_chunks:
            ca = c
            cb = min(n_chunks, ca + group)
            cc = ca
            while cc < cb:
                t = cc * blk
                n = min(blk, L - t)
                if chain and filled + n > W:
                    d = self._bank_desc(state, eta, None, None)
                    rc = _hip.lib().coda_block_write_chain(
                        d, k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2), g.data_ptr(),
                        g.stride(0), L, blk, cc, cb - cc, head, filled, p0 + t, plan.data_ptr(), kmax,
                        self.exact_candidates_per_block if do_e else 0,
                        self.summary_candidates_per_block if do_s else 0, ws.data_ptr(), ws.numel(),
                        sk[cc - ca].data_ptr(), sv[cc - ca].data_ptr(), sa[cc - ca].data_ptr(), sk[0].numel(),
                        sa[0].numel(), ring, _hip.stream_of(k))
                    if rc == _hip.CODA_OK:
                        head, filled = int(ring[0]), int(ring[1])
                        state.pos = p0 + min(L, cb * blk)
                        break
                    if rc != _hip.CODA_EUNSUP:
                        _hip.check(rc)
                    chain = False
                r = self._write_block(
                    state, k_blk=k[:, :, t:t + n], v_blk=v[:, :, t:t + n], g_blk=g[:, t:t + n], pos0=p0 + t,
                    ring_head=head, ring_filled=filled, plan_c=plan[cc], kmax=kmax, do_e=do_e, do_s=do_s,
                    workspace=ws, eta=eta, snap=(sk[cc - ca], sv[cc - ca], sa[cc - ca]))
                if r is None:
                    # the one-launch update does not run here: this group's
                    # earlier chunks get their attention, the rest run chunk by chunk
                    if cc > ca:
                        self._attend_chunks(q, k, v, lam, rope_cos, rope_sin, sk, sv, sa, out, ct, sn, w, ca, cc, blk,
                                            L)
                    return cc, t, head, filled
                head, filled = r
                state.pos = p0 + t + n
                cc += 1
            self._attend_chunks(q, k, v, lam, rope_cos, rope_sin, sk, sv, sa, out, ct, sn, w, ca, cb, blk, L)
            c = cb
        return n_chunks, L, head, filled

    def _attend_chunks(self, q, k, v, lam, rope_cos, rope_sin, sk, sv, sa, out, ct, sn, w, ca, cb, blk, L):
        """The attention of chunks ca .. cb - 1 from their bank snapshots
        (sk / sv / sa[0 ..]) in one launch."""
        d, keep = ops.attention_desc(
            q=q, rope_cos=rope_cos, rope_sin=rope_sin, rope_interleaved=self.rope_interleaved, theta_cos=ct,
            theta_sin=sn, k_prefix=sk[0], v_prefix=sv[0], allowed=sa[0] if self.mask_unused_memory else None,
            k_block=k, v_block=v, lam=lam, rms_weight=w, eps=self._eps, out=out.permute(0, 2, 1, 3))
        _hip.check(_hip.lib().coda_prefill_attn_chunks(d, cb - ca, ca, blk, L, self.window, sk[0].numel(),
                                                       sa[0].numel(), _hip.stream_of(q)))
        # (the last grouped launch, for measurement: its chunks' snapshots
        # stay in the buffers until the next call)
        self.__dict__["_last_chunk_group"] = (ca, cb, blk, L)

    def prefill_chunked(self, x_seq: torch.Tensor, state: CoDAGQALandmarkStatePerf2, *, block_size: int = 256,
                        write_cache: bool = True, return_outputs: bool = True
                        ) -> Tuple[Optional[torch.Tensor], CoDAGQALandmarkStatePerf2]:
        """Chunked prefill over the bounded cache (attention.py:567-728)."""
        self._inference_only()
        _hip.require_device(x_seq)
        B, L, _ = x_seq.shape
        if L == 0:
            return (x_seq[:, :0, :].clone() if return_outputs else None), state
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        p0 = int(state.pos)
        q, k, v, g, lam, cos, sin = self._front(x_seq, p0, fused=False)
        heads = self.prefill_core(q, k, v, g, lam, cos, sin, state, block_size=block_size, write_cache=write_cache,
                                  return_heads=return_outputs)
        if not return_outputs:
            return None, state
        return self.o_proj(heads.view(B, L, self.num_heads * self.head_dim)), state

    # ------------------------------------------------------------ utility
    def cache_bytes(self, *, batch_size: int, dtype: torch.dtype) -> int:
        """Inference state size in bytes (attention.py:734-751)."""
        B = int(batch_size)
        e = torch.tensor([], dtype=dtype).element_size()
        kv = 2 * B * self.num_kv_heads * self.Lbuf * self.head_dim * e
        exact_norm = B * self.num_kv_heads * self.Me * self.head_dim * e if self.Me > 0 else 0
        sum_norm = B * self.num_kv_heads * self.Ms * self.lf_dim * e if self.Ms > 0 else 0
        return int(kv + exact_norm + sum_norm + B * self.window * 4 + B * self.Lbuf + B * self.Me * 8)

    def reset_metrics(self, state: CoDAGQALandmarkStatePerf2) -> None:
        """Zero every metrics counter (attention.py:753-760)."""
        if state.metrics is not None:
            for k in state.metrics:
                state.metrics[k] = 0 if isinstance(state.metrics[k], int) else 0.0
