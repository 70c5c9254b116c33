"""Operator-level checkers: attention, epilogue, bank routing, unbounded layer.

TEST INFRASTRUCTURE ONLY (parity checker). Each function restates the CPU
semantics of one reference operator seam so the product's HIP entry points
can be compared operator by operator.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .prims import expand_kv, head_rms_norm, noise_rotation, rope, rope_inv_freq, rope_tables

NEG_BIG = -(2 ** 62)


def lower_right_mask(Lq: int, Lk: int) -> torch.Tensor:
    """Query i sees keys [0, Lk-Lq+i]; triton_diff_flash/kernel.py:99-105 semantics."""
    return torch.ones(Lq, Lk, dtype=torch.bool).tril(diagonal=Lk - Lq)


def diff_attention(q, q_noise, k, v, lam, rms_weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                   is_causal: bool = False, sm_scale: Optional[float] = None, mask=None):
    """RMSNorm(Attn(q) - lam*Attn(q_noise)) over GQA-shared K/V.

    Restates triton_diff_flash/__init__.py:45-83 (its fallback) with the
    documented lower-right causal alignment of :107 and an optional sm_scale.
    """
    B, H, Lq, Dh = q.shape
    g = H // k.shape[1]
    ke, ve = expand_kv(k, g), expand_kv(v, g)
    if is_causal and mask is None:
        mask = lower_right_mask(Lq, k.shape[2])
    o_s = F.scaled_dot_product_attention(q, ke, ve, attn_mask=mask, scale=sm_scale)
    o_n = F.scaled_dot_product_attention(q_noise, ke, ve, attn_mask=mask, scale=sm_scale)
    out = o_s - lam * o_n
    if rms_weight is not None:
        out = out * torch.rsqrt(out.pow(2).mean(dim=-1, keepdim=True) + eps) * rms_weight
    return out


def diff_epilogue(out_sig, out_noise, lam, weight, eps=1e-6):
    """Sub + RMSNorm + weight, kernels/coda_diff_epilogue/torch-ext/coda_kernels/__init__.py:62-65."""
    d = out_sig - lam * out_noise
    return d * d.pow(2).mean(dim=-1, keepdim=True).add(eps).rsqrt() * weight


def diff_sub_only(out_sig, out_noise, lam):
    """Sub only, coda_kernels/__init__.py:95-96."""
    return out_sig - lam * out_noise


def exact_route(v_sel_norm, mem_v_norm, used, last, gate_sel, pos_sel, *, tau_gate, tau_match,
                tau_novel, refresh_on_hit=False, active_exact=-1):
    """Exact-bank routing with the CPU-path semantics (memory_banks.py:635-697).

    Same signature / outputs as triton_bank_routing/__init__.py:46-80 but the
    vectorised PyTorch branch rules (LRU topk, cumsum rank, skip tokens touch).
    Returns (idx_tok i64, overwrite_tok bool, touch_tok bool, last_out i64).
    """
    B, Hkv, T, Dh = v_sel_norm.shape
    Me = mem_v_norm.shape[2]
    Ae = active_exact if 0 < active_exact < Me else Me
    keep = gate_sel >= tau_gate
    sc = torch.matmul(v_sel_norm.reshape(B * Hkv, T, Dh),
                      mem_v_norm.reshape(B * Hkv, Me, Dh).transpose(1, 2)).view(B, Hkv, T, Me).mean(dim=1)
    if Ae < Me:
        sc.masked_fill_((torch.arange(Me).unsqueeze(0) >= Ae).unsqueeze(1), -1e9)
    sc.masked_fill_(~used[:, None, :], -1e9)
    best, best_idx = sc.max(dim=-1)
    any_used = used.any(dim=-1)
    novel = (~any_used[:, None]) | (best < tau_novel)
    hit = any_used[:, None] & (best >= tau_match)
    nk = novel & keep
    rk = last.clone()
    rk[~used] = NEG_BIG
    if Ae < Me:
        rk[:, Ae:] = NEG_BIG
    n_lru = min(T, Ae)
    _, lru = torch.topk(rk, k=n_lru, dim=1, largest=False, sorted=True)
    rank = nk.to(torch.int64).cumsum(dim=1) - 1
    cap = nk & (rank < Ae)
    idx = torch.where(cap, lru.gather(1, rank.clamp(min=0, max=max(n_lru - 1, 0))), best_idx)
    touch = keep & (~novel | cap)
    ow = keep & (cap | hit) if refresh_on_hit else cap
    tm = torch.zeros((B, Me), dtype=torch.int8).scatter_reduce_(1, idx, touch.to(torch.int8), reduce="amax",
                                                                include_self=True)
    pv = torch.full((B, Me), NEG_BIG, dtype=torch.int64).scatter_reduce_(
        1, idx, torch.where(touch, pos_sel, torch.full_like(pos_sel, NEG_BIG)), reduce="amax", include_self=True)
    return idx, ow, touch, torch.where(tm.to(torch.bool), pv, last)


def summary_update(k_sel, v_sel, w_tok, mem_k, mem_v, used, mem_lf_k_norm, *, eta_logit, energy_scale,
                   lf_start, overwrite_on_insert, active_summary=-1):
    """Summary-bank route + accumulate + EMA with CPU-path semantics.

    Same outputs as triton_summary_bank.py:188-271 (mem_k_out, mem_v_out,
    used_out, route_idx int32) but with memory_banks.py:866-918 rules: global
    first-occurrence argmax, candidate-order dtype accumulation. ``eta_logit``
    may be a float or a per-KV-head tensor.
    """
    B, Hkv, T, Dh = k_sel.shape
    Ms = mem_k.shape[2]
    As = active_summary if 0 < active_summary < Ms else Ms
    lf = lf_start
    kn = F.normalize(k_sel[..., lf:], dim=-1, eps=1e-6)
    sc = torch.matmul(kn.reshape(B * Hkv, T, Dh - lf),
                      mem_lf_k_norm.reshape(B * Hkv, Ms, Dh - lf).transpose(1, 2)).view(B, Hkv, T, Ms).mean(dim=1)
    if As < Ms:
        sc.masked_fill_((torch.arange(Ms).unsqueeze(0) >= As).unsqueeze(1), -1e9)
    idx = sc.argmax(dim=-1)
    dt = mem_k.dtype
    w = w_tok.to(dt)
    count = torch.zeros(B, Ms, dtype=dt).scatter_add_(1, idx, w)
    ix = idx.unsqueeze(1).unsqueeze(-1).expand(B, Hkv, T, Dh)
    w4 = w.view(B, 1, T, 1)
    sk = torch.zeros(B, Hkv, Ms, Dh, dtype=dt).scatter_add_(2, ix, k_sel * w4)
    sv = torch.zeros(B, Hkv, Ms, Dh, dtype=dt).scatter_add_(2, ix, v_sel * w4)
    el = eta_logit if torch.is_tensor(eta_logit) else torch.full((Hkv,), float(eta_logit))
    eta = torch.sigmoid(el).to(dtype=dt).view(1, -1, 1, 1)
    c4 = count.view(B, 1, Ms, 1)
    active = c4 > 0
    ak, av = sk / c4.clamp_min(1e-6), sv / c4.clamp_min(1e-6)
    eta_eff = torch.where((~used).view(B, 1, Ms, 1) & active, torch.ones_like(eta), eta) if overwrite_on_insert else eta
    dk = torch.zeros_like(ak)
    dk[..., lf:] = ak[..., lf:] * energy_scale - mem_k[..., lf:]
    nk = torch.where(active, mem_k + eta_eff * dk, mem_k)
    nv = torch.where(active, mem_v + eta_eff * (av - mem_v), mem_v)
    return nk, nv, used | (count > 0), idx.to(torch.int32)


class OracleUnbounded(nn.Module):
    """Unbounded CoDA-GQA forward, src/coda_gqa_l/baseline.py:22-147 (config C4 path)."""

    def __init__(self, *, embed_dim, num_heads, num_kv_heads, rope_base=10_000.0, lambda_init_bias=-6.0,
                 theta_init=math.pi / 2, eps=1e-6, head_norm_mode="full", rope_interleaved=True):
        super().__init__()
        self.embed_dim, self.num_heads, self.num_kv_heads = embed_dim, num_heads, num_kv_heads
        self.head_dim = embed_dim // num_heads
        D, H, Hkv, Dh = embed_dim, num_heads, num_kv_heads, self.head_dim
        self.q_proj = nn.Linear(D, H * Dh, bias=False)
        self.k_proj = nn.Linear(D, Hkv * Dh, bias=False)
        self.v_proj = nn.Linear(D, Hkv * Dh, bias=False)
        self.theta = nn.Parameter(torch.full((H, Dh // 2), theta_init))
        self.lambda_proj = nn.Linear(D, H, bias=True)
        nn.init.constant_(self.lambda_proj.bias, lambda_init_bias)
        self.rope = nn.Module()
        self.rope.register_buffer("inv_freq", rope_inv_freq(Dh, rope_base), persistent=False)
        self.head_norm_mode = head_norm_mode
        if head_norm_mode == "full":
            self.head_norm = nn.Module()
            self.head_norm.weight = nn.Parameter(torch.ones(Dh))
            self.head_norm.eps = eps
        self.rope_interleaved = bool(rope_interleaved)
        self.o_proj = nn.Linear(H * Dh, D, bias=False)

    def forward(self, x, *, is_causal=True, attention_mask=None, past_key_value=None):
        B, L, D = x.shape
        H, Hkv, Dh = self.num_heads, self.num_kv_heads, self.head_dim
        q = self.q_proj(x).view(B, L, H, Dh).transpose(1, 2)
        k = self.k_proj(x).view(B, L, Hkv, Dh).transpose(1, 2)
        v = self.v_proj(x).view(B, L, Hkv, Dh).transpose(1, 2)
        off = past_key_value[0].size(2) if past_key_value is not None else 0
        c, s = rope_tables(self.rope.inv_freq, L, off, q.dtype)
        q, k = rope(q, c, s, self.rope_interleaved), rope(k, c, s, self.rope_interleaved)
        if past_key_value is not None:
            k = torch.cat([past_key_value[0], k], dim=2)
            v = torch.cat([past_key_value[1], v], dim=2)
        kv = (k, v)
        g = H // Hkv
        ke, ve = expand_kv(k, g), expand_kv(v, g)
        lam = torch.sigmoid(self.lambda_proj(x)).transpose(1, 2).unsqueeze(-1)
        qn = noise_rotation(q, torch.cos(self.theta).to(q.dtype), torch.sin(self.theta).to(q.dtype))
        cf = is_causal if attention_mask is None else False
        o_s = F.scaled_dot_product_attention(q, ke, ve, attn_mask=attention_mask, is_causal=cf)
        o_n = F.scaled_dot_product_attention(qn, ke, ve, attn_mask=attention_mask, is_causal=cf)
        out = o_s - lam * o_n
        if self.head_norm_mode == "full":
            out = head_rms_norm(out, self.head_norm.weight, self.head_norm.eps)
        return self.o_proj(out.transpose(1, 2).contiguous().view(B, L, D)), kv
