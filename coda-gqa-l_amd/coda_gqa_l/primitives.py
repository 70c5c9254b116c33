"""Building blocks shared by the bounded and unbounded layers.

Same public names and semantics as the reference's primitives
(src/coda_gqa_l/primitives.py:15-153).  The hot-path uses of these (RoPE of
keys and queries, the noise rotation, the RMSNorm epilogue) run inside the
HIP kernels; the modules here hold parameters / buffers and build the
angle tables with the reference's op sequence on the device.
"""

from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn

from . import _hip


class HeadwiseRMSNorm(nn.Module):
    """RMSNorm over head_dim (primitives.py:15-27).  The forward runs the HIP
    epilogue with a zero noise stream, so it is exactly the eager norm."""

    def __init__(self, head_dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(head_dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from .ops import diff_epilogue
        zeros = torch.zeros_like(x)
        lam = torch.zeros(x.shape[:-1] + (1,), dtype=x.dtype, device=x.device)
        return diff_epilogue(x, zeros, lam, self.weight, eps=self.eps)


class RotaryEmbedding(nn.Module):
    """RoPE tables (primitives.py:30-55): positions are generated in the
    buffer's dtype and the outer product is taken in it, like the reference."""

    def __init__(self, head_dim: int, base: float = 10_000.0):
        super().__init__()
        if head_dim % 2 != 0:
            raise ValueError("RoPE requires even head_dim.")
        inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2).float() / head_dim))
        self.register_buffer("inv_freq", inv_freq, persistent=False)

    def forward(self, *, seq_len: int, offset: int, device: torch.device,
                dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        t = torch.arange(offset, offset + seq_len, device=device, dtype=self.inv_freq.dtype)
        freqs = torch.einsum("i,j->ij", t, self.inv_freq)
        return freqs.cos().to(dtype=dtype), freqs.sin().to(dtype=dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, interleaved: bool = True,
               out: torch.Tensor = None) -> torch.Tensor:
    """RoPE of (B, H, L, Dh) with (L, Dh/2) tables on the device
    (primitives.py:83-113), one rounding per op in the element type.
    `out` may be any (B, H, L, Dh) view with a unit channel stride."""
    _hip.require_device(x, cos, sin)
    B, H, L, Dh = x.shape
    if out is None:
        out = torch.empty((B, H, L, Dh), dtype=x.dtype, device=x.device)
    xs = x if x.stride(-1) == 1 else x.contiguous()
    cos = cos.reshape(L, Dh // 2).contiguous()
    sin = sin.reshape(L, Dh // 2).contiguous()
    _hip.check(_hip.lib().coda_rope_fwd(
        _hip.dtype_code(x.dtype), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        xs.data_ptr(), xs.stride(0), xs.stride(1), xs.stride(2), cos.data_ptr(), sin.data_ptr(),
        B, H, L, Dh, int(bool(interleaved)), _hip.stream_of(x)))
    return out


def _apply_pairwise_rotation(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Per-head rotation of (2i, 2i+1) pairs by (H, Dh/2) angle tables
    (primitives.py:58-80): the interleaved RoPE kernel with heads on the
    table axis."""
    _hip.require_device(x, cos, sin)
    B, H, L, Dh = x.shape
    xs = x.permute(0, 2, 1, 3)  # (B, L, H, Dh): heads index the table rows
    out = torch.empty((B, L, H, Dh), dtype=x.dtype, device=x.device)
    c = cos.reshape(H, Dh // 2).contiguous()
    s = sin.reshape(H, Dh // 2).contiguous()
    _hip.check(_hip.lib().coda_rope_fwd(
        _hip.dtype_code(x.dtype), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        xs.data_ptr(), xs.stride(0), xs.stride(1), xs.stride(2), c.data_ptr(), s.data_ptr(),
        B, L, H, Dh, 1, _hip.stream_of(x)))
    return out.permute(0, 2, 1, 3)


def repeat_kv(x: torch.Tensor, num_repeat: int) -> torch.Tensor:
    """(B, Hkv, L, Dh) -> (B, Hkv * num_repeat, L, Dh) (primitives.py:116-127).
    The kernels share K/V across the group without this copy."""
    if num_repeat == 1:
        return x
    B, H_kv, L, Dh = x.shape
    return x[:, :, None, :, :].expand(B, H_kv, num_repeat, L, Dh).reshape(B, H_kv * num_repeat, L, Dh)


def compute_lf_start(head_dim: int) -> int:
    """First channel of the low-frequency RoPE band (primitives.py:145-153)."""
    return head_dim // 2
