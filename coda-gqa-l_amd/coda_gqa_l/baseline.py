"""Unbounded differential attention (the Phase-1 layer), on MI355X.

Same constructor, parameters and forward contract as the reference's
CoDAGQA (src/coda_gqa_l/baseline.py:22-147): returns (y, (k_total,
v_total)).  RoPE of keys runs in the rope kernel; RoPE of queries, the noise
rotation, GQA sharing, the causal mask, the lambda difference and the head
norm run inside one attention kernel (no repeat_kv copies, one K/V pass).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _hip, ops
from .primitives import HeadwiseRMSNorm, RotaryEmbedding, apply_rope


class CoDAGQA(nn.Module):
    def __init__(self, *, embed_dim: int, num_heads: int, num_kv_heads: int, rope_base: float = 10_000.0,
                 lambda_init_bias: float = -6.0, theta_init: float = math.pi / 2, eps: float = 1e-6,
                 head_norm_mode: str = "full", rope_interleaved: bool = True):
        super().__init__()
        if embed_dim % num_heads != 0:
            raise ValueError("embed_dim must be divisible by num_heads.")
        if num_heads % num_kv_heads != 0:
            raise ValueError("num_heads must be divisible by num_kv_heads (GQA constraint).")
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = embed_dim // num_heads
        if self.head_dim % 2 != 0:
            raise ValueError("head_dim must be even (required by RoPE + pairwise rotations).")
        self.q_proj = nn.Linear(embed_dim, num_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(embed_dim, num_kv_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(embed_dim, num_kv_heads * self.head_dim, bias=False)
        self.theta = nn.Parameter(torch.full((num_heads, self.head_dim // 2), theta_init))
        self.lambda_proj = nn.Linear(embed_dim, num_heads, bias=True)
        nn.init.constant_(self.lambda_proj.bias, lambda_init_bias)
        self.rope = RotaryEmbedding(self.head_dim, base=rope_base)
        self.head_norm_mode = head_norm_mode
        if head_norm_mode == "full":
            self.head_norm = HeadwiseRMSNorm(self.head_dim, eps=eps)
        elif head_norm_mode == "identity":
            self.head_norm = nn.Identity()
        else:
            raise ValueError(f"head_norm_mode must be 'full' or 'identity', got {head_norm_mode!r}")
        self.rope_interleaved = bool(rope_interleaved)
        self.o_proj = nn.Linear(num_heads * self.head_dim, embed_dim, bias=False)
        self._eps = float(eps)

    def attention_core(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lam: torch.Tensor,
                       rope_cos: Optional[torch.Tensor], rope_sin: Optional[torch.Tensor], *, causal: int,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """q (B,H,Lq,Dh) pre-RoPE (tables given) or post-RoPE; k, v
        (B,Hkv,Lk,Dh) post-RoPE; lam (B,H,Lq); causal 0 / 1 (lower-right) /
        2 (upper-left).  Returns head outputs (B, Lq, H, Dh)."""
        B, H, Lq, Dh = q.shape
        if out is None:
            out = torch.empty((B, Lq, H, Dh), dtype=q.dtype, device=q.device)
        ct = torch.cos(self.theta).to(dtype=q.dtype).contiguous()
        st = torch.sin(self.theta).to(dtype=q.dtype).contiguous()
        w = self.head_norm.weight.detach().to(q.dtype).contiguous() if self.head_norm_mode == "full" else None
        d = ops.bounded_attention(
            q=q, rope_cos=rope_cos, rope_sin=rope_sin, rope_interleaved=self.rope_interleaved, theta_cos=ct,
            theta_sin=st, k_prefix=None, v_prefix=None, allowed=None, k_block=k, v_block=v, lam=lam,
            rms_weight=w, eps=self._eps, out=out.permute(0, 2, 1, 3), causal=causal)
        return out

    def forward(self, x: torch.Tensor, *, is_causal: bool = True, attention_mask: Optional[torch.Tensor] = None,
                past_key_value: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
                ) -> Tuple[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
        """x (B, L, D) -> (y, (k_total, v_total)) (baseline.py:95-147)."""
        if self.training:
            raise NotImplementedError("CoDAGQA on MI355X is inference-only (no backward kernels); call .eval()")
        if attention_mask is not None:
            raise NotImplementedError("explicit attention masks are not supported by the MI355X kernels")
        _hip.require_device(x)
        B, L, D = x.shape
        H, Hkv, Dh = self.num_heads, self.num_kv_heads, self.head_dim
        q = self.q_proj(x).view(B, L, H, Dh).permute(0, 2, 1, 3)
        k = self.k_proj(x).view(B, L, Hkv, Dh).permute(0, 2, 1, 3)
        v = self.v_proj(x).view(B, L, Hkv, Dh).permute(0, 2, 1, 3)
        offset = past_key_value[0].size(2) if past_key_value is not None else 0
        cos, sin = self.rope(seq_len=L, offset=offset, device=x.device, dtype=q.dtype)
        cos, sin = cos.contiguous(), sin.contiguous()
        k = apply_rope(k, cos, sin, interleaved=self.rope_interleaved)
        if past_key_value is not None:
            k = torch.cat([past_key_value[0], k], dim=2)
            v = torch.cat([past_key_value[1], v], dim=2)
        else:
            v = v.contiguous()
        lam = torch.sigmoid(self.lambda_proj(x)).permute(0, 2, 1)
        # torch SDPA's is_causal aligns upper-left; with no past it is square
        heads = self.attention_core(q, k, v, lam, cos, sin, causal=2 if is_causal else 0)
        return self.o_proj(heads.view(B, L, D)), (k, v)
