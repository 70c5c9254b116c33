"""Elementwise / per-row primitives of the reference, restated on torch CPU.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the parity checker; never by the product.

Every function keeps the reference's op order so that per-op rounding in
reduced precision (bf16 rounds after every torch op on CPU) is reproduced.
"""

from __future__ import annotations

import torch


def head_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * w over the last dim.

    Follows src/coda_gqa_l/primitives.py:23-27 (HeadwiseRMSNorm.forward).
    """
    ms = x.pow(2).mean(dim=-1, keepdim=True)
    return (x * torch.rsqrt(ms + eps)) * weight


def rope_inv_freq(head_dim: int, base: float) -> torch.Tensor:
    """fp32 inverse frequencies, primitives.py:40 (RotaryEmbedding.__init__).

    The reference registers this as a module buffer, so ``module.to(dtype)``
    casts it; callers pass the cast copy to :func:`rope_tables`.
    """
    return 1.0 / (base ** (torch.arange(0, head_dim, 2).float() / head_dim))


def rope_tables(inv_freq: torch.Tensor, seq_len: int, offset: int, dtype: torch.dtype):
    """cos/sin tables (seq_len, Dh/2), primitives.py:43-55.

    Positions are generated in inv_freq's dtype (bf16 for a bf16 module, a
    reference quirk that rounds positions above 256), the outer product is
    taken in that dtype and cos/sin are cast to ``dtype``.
    """
    t = torch.arange(offset, offset + seq_len, dtype=inv_freq.dtype)
    ang = torch.einsum("i,j->ij", t, inv_freq)
    return ang.cos().to(dtype=dtype), ang.sin().to(dtype=dtype)


def _rotate_pairs(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    ev, od = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = ev * c - od * s
    out[..., 1::2] = ev * s + od * c
    return out


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, interleaved: bool = True) -> torch.Tensor:
    """RoPE on (B, H, L, Dh) with (L, Dh/2) tables, primitives.py:83-113.

    interleaved pairs (2i, 2i+1); otherwise the half-split form
    x*cos_full + rotate_half(x)*sin_full in transformers' op order.
    """
    B, H, L, Dh = x.shape
    half = Dh // 2
    c = cos.view(1, 1, L, half)
    s = sin.view(1, 1, L, half)
    if interleaved:
        return _rotate_pairs(x, c, s)
    c2 = torch.cat([c, c], dim=-1)
    s2 = torch.cat([s, s], dim=-1)
    xr = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * c2 + xr * s2


def noise_rotation(x: torch.Tensor, cos_t: torch.Tensor, sin_t: torch.Tensor) -> torch.Tensor:
    """Per-head pairwise rotation by theta, primitives.py:58-80."""
    B, H, L, Dh = x.shape
    half = Dh // 2
    return _rotate_pairs(x, cos_t.view(1, H, 1, half), sin_t.view(1, H, 1, half))


def expand_kv(x: torch.Tensor, groups: int) -> torch.Tensor:
    """GQA head expansion (B,Hkv,L,Dh)->(B,Hkv*groups,L,Dh), primitives.py:116-127."""
    if groups == 1:
        return x
    B, Hkv, L, Dh = x.shape
    return x[:, :, None].expand(B, Hkv, groups, L, Dh).reshape(B, Hkv * groups, L, Dh)


def unit(x: torch.Tensor) -> torch.Tensor:
    """F.normalize(x, dim=-1, eps=1e-6) as used throughout memory_banks.py."""
    return torch.nn.functional.normalize(x, dim=-1, eps=1e-6)
