"""The bounded differential-attention layer of the reference, restated on CPU.

TEST INFRASTRUCTURE ONLY (parity checker). Follows the CPU branches of
src/coda_gqa_l/attention.py (CoDAGQALandmarkPerf2, :72-760). Parameter and
buffer names match the reference so ``load_state_dict`` moves weights between
the reference, this oracle and the product module unchanged.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Dict, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import banks
from .prims import expand_kv, head_rms_norm, noise_rotation, rope, rope_inv_freq, rope_tables, unit

try:
    from torch.nn.attention.bias import causal_lower_right as _lower_right
except ImportError:  # pragma: no cover - torch < 2.5
    _lower_right = None


@dataclass
class OracleState:
    """Same fields, order and meaning as src/coda_gqa_l/state.py:24-54."""

    k_buf: torch.Tensor
    v_buf: torch.Tensor
    allowed: torch.Tensor
    g_recent: torch.Tensor
    recent_idx: int
    recent_filled: int
    mem_last_exact: torch.Tensor
    pos: int
    active_exact: int = 0
    active_summary: int = 0
    _exact_v_norm: Optional[torch.Tensor] = field(default=None, repr=False)
    _sum_lf_k_norm: Optional[torch.Tensor] = field(default=None, repr=False)
    metrics: Optional[Dict[str, Any]] = field(default=None, repr=False)


class _Norm(nn.Module):
    def __init__(self, dh, eps):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dh))

    def forward(self, x):
        return head_rms_norm(x, self.weight, self.eps)


class _Rope(nn.Module):
    def __init__(self, dh, base):
        super().__init__()
        self.register_buffer("inv_freq", rope_inv_freq(dh, base), persistent=False)


METRIC_KEYS = ("exact_hits", "exact_inserts", "exact_overwrites", "exact_fill_ratio",
               "summary_updates", "summary_inserts", "summary_fill_ratio", "tokens_gated_out",
               "total_evictions", "exact_frustrated", "summary_frustrated", "active_exact",
               "active_summary", "expansions_exact", "expansions_summary")


class OracleLayer(nn.Module):
    """CPU restatement of CoDAGQALandmarkPerf2 (attention.py:89-241 constructor)."""

    def __init__(self, *, embed_dim, num_heads, num_kv_heads, window, num_landmarks_exact,
                 num_landmarks_summary, rope_base=10_000.0, lambda_init_bias=-6.0,
                 theta_init=math.pi / 2, write_policy="gated", write_gate_init_bias=-2.0,
                 write_gate_threshold_exact=0.10, write_gate_threshold_summary=0.05,
                 exact_match_threshold=0.90, exact_novelty_threshold=0.70,
                 exact_refresh_on_hit=False, exact_candidates_per_block=8,
                 summary_eta_init_logit=-3.0, summary_candidates_per_block=64,
                 summary_overwrite_on_insert=True, min_landmarks_exact=None,
                 max_landmarks_exact=None, min_landmarks_summary=None,
                 max_landmarks_summary=None, expansion_t_max=1_000_000,
                 mem_init="random_normal", mask_unused_memory=True, detach_evicted=True,
                 eps=1e-6, collect_metrics=False, head_norm_mode="full", rope_interleaved=True):
        super().__init__()
        if embed_dim % num_heads or num_heads % num_kv_heads or window <= 0:
            raise ValueError("bad head / window configuration")
        self.embed_dim, self.num_heads, self.num_kv_heads = int(embed_dim), int(num_heads), int(num_kv_heads)
        self.head_dim = self.embed_dim // self.num_heads
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
        self.Me, self.Ms = self.Me_max, self.Ms_max
        self.Lbuf = self.window + self.Me + self.Ms

        D, H, Hkv, Dh = self.embed_dim, self.num_heads, self.num_kv_heads, self.head_dim
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
        self.rope = _Rope(Dh, float(rope_base))
        self.head_norm_mode = head_norm_mode
        self.head_norm = _Norm(Dh, eps) if head_norm_mode == "full" else nn.Identity()
        self.o_proj = nn.Linear(H * Dh, D, bias=False)

    # ---------------------------------------------------------------- state
    def init_state(self, *, batch_size, dtype, mem_init=None, device=None):
        """attention.py:247-338; CPU generator, same normal_ call order."""
        B, Hkv, Dh, W, Me, Ms = int(batch_size), self.num_kv_heads, self.head_dim, self.window, self.Me, self.Ms
        k_buf = torch.zeros((B, Hkv, self.Lbuf, Dh), dtype=dtype)
        v_buf = torch.zeros((B, Hkv, self.Lbuf, Dh), dtype=dtype)
        mode = mem_init if mem_init is not None else self.mem_init
        if mode == "random_normal":
            if Me > 0:
                k_buf[:, :, W:W + Me, :].normal_(mean=0.0, std=0.02)
                v_buf[:, :, W:W + Me, :].normal_(mean=0.0, std=0.02)
            if Ms > 0:
                k_buf[:, :, W + Me:, self.lf_start:].normal_(mean=0.0, std=0.02)
                v_buf[:, :, W + Me:, :].normal_(mean=0.0, std=0.02)
        elif mode != "zeros":
            raise ValueError("mem_init must be 'zeros' or 'random_normal'")
        st = OracleState(k_buf=k_buf, v_buf=v_buf, allowed=torch.zeros((B, self.Lbuf), dtype=torch.bool),
                         g_recent=torch.zeros((B, W), dtype=torch.float32), recent_idx=0, recent_filled=0,
                         mem_last_exact=torch.zeros((B, Me), dtype=torch.int64), pos=0,
                         active_exact=self.Me_min if Me > 0 else 0,
                         active_summary=self.Ms_min if Ms > 0 else 0)
        if Me > 0:
            st._exact_v_norm = unit(v_buf[:, :, W:W + Me]).clone()
        if Ms > 0:
            st._sum_lf_k_norm = unit(k_buf[:, :, W + Me:, self.lf_start:]).clone()
        if self.collect_metrics:
            st.metrics = {k: (0.0 if k.endswith("ratio") else 0) for k in METRIC_KEYS}
            st.metrics["active_exact"] = st.active_exact
            st.metrics["active_summary"] = st.active_summary
        return st

    def _log_ceiling(self, t):
        """attention.py:344-356."""
        if self.expansion_t_max <= 0:
            return self.Me_max, self.Ms_max
        r = min(math.log(1 + t) / math.log(1 + self.expansion_t_max), 1.0)
        return (self.Me_min + int((self.Me_max - self.Me_min) * r),
                self.Ms_min + int((self.Ms_max - self.Ms_min) * r))

    def _try_expand(self, st, fr_e, fr_s):
        """attention.py:358-390."""
        if self.Me_min == self.Me_max and self.Ms_min == self.Ms_max:
            return
        if fr_e <= 0 and fr_s <= 0:
            return
        ce, cs = self._log_ceiling(st.pos)
        de = ds = 0
        if fr_e > 0 and st.active_exact < ce:
            de = min(fr_e, ce - st.active_exact)
            st.active_exact += de
        if fr_s > 0 and st.active_summary < cs:
            ds = min(fr_s, cs - st.active_summary)
            st.active_summary += ds
        if st.metrics is not None:
            st.metrics["active_exact"] = st.active_exact
            st.metrics["active_summary"] = st.active_summary
            st.metrics["expansions_exact"] += de
            st.metrics["expansions_summary"] += ds

    # ---------------------------------------------------------- projections
    def project(self, x):
        """q (B,H,L,Dh), k_raw, v (B,Hkv,L,Dh), gate (B,L) fp32, lambda (B,H,L,1).

        attention.py:396-410 and :508 / :603-604.
        """
        B, L, _ = x.shape
        q = self.q_proj(x).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(x).view(B, L, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(B, L, self.num_kv_heads, self.head_dim).transpose(1, 2)
        if self.write_policy == "none":
            g = torch.ones((B, L), dtype=torch.float32)
        else:
            g = torch.sigmoid(self.write_proj(x)).squeeze(-1).to(torch.float32)
        lam = torch.sigmoid(self.lambda_proj(x)).transpose(1, 2).unsqueeze(-1)
        return q, k, v, g, lam

    def rope_tables(self, L, offset, dtype):
        return rope_tables(self.rope.inv_freq, L, offset, dtype)

    def theta_tables(self, dtype):
        return torch.cos(self.theta).to(dtype=dtype), torch.sin(self.theta).to(dtype=dtype)

    # ------------------------------------------------------------ attention
    def two_stream(self, q, q_noise, k, v, mask, lam, is_causal=False):
        """CPU branch of _sdpa_stacked_two_stream, attention.py:438-464."""
        g = self.num_heads // self.num_kv_heads
        ke, ve = expand_kv(k, g), expand_kv(v, g)
        o_s = F.scaled_dot_product_attention(q, ke, ve, attn_mask=mask, is_causal=is_causal)
        o_n = F.scaled_dot_product_attention(q_noise, ke, ve, attn_mask=mask, is_causal=is_causal)
        return self.head_norm(o_s - lam * o_n)

    def out_proj(self, oh):
        B, H, L, Dh = oh.shape
        return self.o_proj(oh.transpose(1, 2).contiguous().view(B, L, H * Dh))

    def attend_core(self, q, lam, st, qp):
        """Heads (B,H,1,Dh) of one token: q pre-RoPE (B,H,1,Dh), lam (B,H,1,1)
        (attention.py:486-514 after the projections)."""
        B = q.shape[0]
        k_att, v_att, mask = st.k_buf, st.v_buf, None
        if self.mask_unused_memory:
            if not bool(st.allowed.any()):
                return torch.zeros_like(q)
            if not bool(st.allowed.all()):
                if B == 1:
                    vi = st.allowed[0].nonzero(as_tuple=True)[0]
                    k_att, v_att = st.k_buf[:, :, vi], st.v_buf[:, :, vi]
                else:
                    mask = st.allowed[:, None, None, :]
        c, s = self.rope_tables(1, qp, q.dtype)
        q = rope(q, c, s, self.rope_interleaved)
        ct, sn = self.theta_tables(q.dtype)
        qn = noise_rotation(q, ct, sn)
        return self.two_stream(q, qn, k_att, v_att, mask, lam)

    def attend_step(self, x, st, *, query_pos=None):
        """attention.py:476-514."""
        B, L, _ = x.shape
        assert L == 1
        if self.mask_unused_memory and not bool(st.allowed.any()):
            return torch.zeros_like(x)
        q = self.q_proj(x).view(B, L, self.num_heads, self.head_dim).transpose(1, 2)
        qp = st.pos if query_pos is None else int(query_pos)
        lam = torch.sigmoid(self.lambda_proj(x)).transpose(1, 2).unsqueeze(-1)
        return self.out_proj(self.attend_core(q, lam, st, qp))

    def _new_kv(self, x, q_pos):
        B, L, _ = x.shape
        k = self.k_proj(x).view(B, L, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(B, L, self.num_kv_heads, self.head_dim).transpose(1, 2)
        c, s = self.rope_tables(1, q_pos, x.dtype)
        k = rope(k, c, s, self.rope_interleaved)
        if self.write_policy == "none":
            g = torch.ones((B, L), dtype=torch.float32)
        else:
            g = torch.sigmoid(self.write_proj(x)).squeeze(-1).to(torch.float32)
        return k, v, g

    def step(self, x, st, *, attend=True, write_cache=True, include_current_in_attention=True, trace=None):
        """attention.py:516-547."""
        B, L, _ = x.shape
        assert L == 1
        qp = int(st.pos)
        if attend and include_current_in_attention and write_cache:
            k, v, g = self._new_kv(x, qp)
            banks.write_one(self, st, k, v, g, trace)
            return self.attend_step(x, st, query_pos=qp), st
        y = self.attend_step(x, st, query_pos=qp) if attend else torch.zeros_like(x)
        if write_cache:
            k, v, g = self._new_kv(x, qp)
            banks.write_one(self, st, k, v, g, trace)
        return y, st

    def prefill_core(self, q_seq, k_seq, v_seq, g_seq, lam_seq, st, *, block_size, write_cache=True,
                     return_heads=True, trace=None):
        """Chunk loop after the projections (attention.py:611-724).

        q_seq (B,H,L,Dh) roped, k_seq (B,Hkv,L,Dh) roped, v_seq, g_seq (B,L)
        fp32, lam_seq (B,H,L,1).  Returns heads (B,H,L,Dh) or None.
        """
        B, H, L, Dh = q_seq.shape
        p0 = int(st.pos)
        ct, sn = self.theta_tables(q_seq.dtype)
        outs = []
        t = 0
        while t < L:
            blk = min(int(block_size), L - t)
            pos0 = p0 + t
            q = q_seq[:, :, t:t + blk]
            kb, vb, gb, lam = k_seq[:, :, t:t + blk], v_seq[:, :, t:t + blk], g_seq[:, t:t + blk], lam_seq[:, :, t:t + blk]
            packed = B == 1 and self.mask_unused_memory and not self.training and not bool(st.allowed[0].all())
            if packed:
                vi = st.allowed[0].nonzero(as_tuple=True)[0]
                k_all = torch.cat([st.k_buf[:, :, vi], kb], dim=2)
                v_all = torch.cat([st.v_buf[:, :, vi], vb], dim=2)
            else:
                k_all = torch.cat([st.k_buf, kb], dim=2)
                v_all = torch.cat([st.v_buf, vb], dim=2)
            Lk = k_all.shape[2]
            causal = False
            if Lk == blk:
                mask, causal = None, True
            elif _lower_right is not None and B == 1 and (packed or bool(st.allowed[0].all()) or not self.mask_unused_memory):
                mask = _lower_right(blk, Lk)
            else:
                pre = torch.ones((blk, Lk - blk), dtype=torch.bool)
                cm = torch.cat([pre, torch.tril(torch.ones((blk, blk), dtype=torch.bool))], dim=1)
                if packed:
                    mask = cm.view(1, 1, blk, Lk)
                else:
                    if self.mask_unused_memory:
                        ok = torch.cat([st.allowed, torch.ones((B, blk), dtype=torch.bool)], dim=1)
                    else:
                        ok = torch.ones((B, Lk), dtype=torch.bool)
                    mask = cm.view(1, 1, blk, Lk) & ok[:, None, None, :]
            if return_heads:
                qn = noise_rotation(q, ct, sn)
                outs.append(self.two_stream(q, qn, k_all, v_all, mask, lam, causal))
            if write_cache:
                banks.write_block(self, st, kb, vb, gb, pos0, trace)
            t += blk
        return torch.cat(outs, dim=2) if return_heads else None

    def project_seq(self, x_seq, p0):
        """Hoisted projections of prefill_chunked (attention.py:590-608):
        q, k roped with the tables of positions p0.., v, g, lam."""
        B, L, _ = x_seq.shape
        q_seq, k_raw, v_seq, g_seq, lam_seq = self.project(x_seq)
        c, s = self.rope_tables(L, p0, x_seq.dtype)
        return (rope(q_seq, c, s, self.rope_interleaved), rope(k_raw, c, s, self.rope_interleaved), v_seq, g_seq,
                lam_seq)

    def prefill_chunked(self, x_seq, st, *, block_size=256, write_cache=True, return_outputs=True, trace=None):
        """attention.py:567-728 (hoisted projections, chunk loop, mask policy)."""
        B, L, _ = x_seq.shape
        if L == 0:
            return (x_seq[:, :0, :].clone() if return_outputs else None), st
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        q_seq, k_seq, v_seq, g_seq, lam_seq = self.project_seq(x_seq, int(st.pos))
        heads = self.prefill_core(q_seq, k_seq, v_seq, g_seq, lam_seq, st, block_size=block_size,
                                  write_cache=write_cache, return_heads=return_outputs, trace=trace)
        return (self.out_proj(heads) if return_outputs else None), st

    def cache_bytes(self, *, batch_size, dtype):
        """attention.py:734-751."""
        B, e = int(batch_size), torch.tensor([], dtype=dtype).element_size()
        kv = 2 * B * self.num_kv_heads * self.Lbuf * self.head_dim * e
        en = B * self.num_kv_heads * self.Me * self.head_dim * e if self.Me > 0 else 0
        sn = B * self.num_kv_heads * self.Ms * self.lf_dim * e if self.Ms > 0 else 0
        return int(kv + en + sn + B * self.window * 4 + B * self.Lbuf + B * self.Me * 8)
