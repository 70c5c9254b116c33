"""Operator seams of the reference, served by the HIP kernels.

  diff_flash_attn  - fused differential attention
                     (src/coda_gqa_l/triton_diff_flash/__init__.py:86-146)
  diff_epilogue    - sub + RMSNorm + weight
  diff_sub_only    - sub only
                     (kernels/coda_diff_epilogue/torch-ext/coda_kernels/__init__.py:38-103)
  bounded_attention - the bounded-cache form used by the layer: prefix =
                     state cache gated by `allowed`, block = the chunk's
                     keys with a lower-right causal mask, RoPE of q and the
                     noise rotation applied in-kernel.

Errors surface as RuntimeError with the library's message (the reference's
TORCH_CHECK contract, torch_binding.cpp:80-99).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _hip


def is_available() -> bool:
    """True when the HIP library loads and a HIP device is visible."""
    try:
        return _hip.lib().coda_device_count() > 0
    except (OSError, RuntimeError):
        return False


def _strides3(t: torch.Tensor):
    return int(t.stride(0)), int(t.stride(1)), int(t.stride(2))


def _last_dim_contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _run_attn(desc: _hip.AttnDesc, like: torch.Tensor) -> None:
    L = _hip.lib()
    need = __import__("ctypes").c_size_t(0)
    _hip.check(L.coda_attn_workspace_bytes(desc, need))
    ws = None
    if need.value:
        ws = torch.empty(need.value, dtype=torch.uint8, device=like.device)
        desc.workspace = ws.data_ptr()
        desc.workspace_bytes = need.value
    _hip.check(L.coda_diff_attn_fwd(desc, _hip.stream_of(like)))


def diff_flash_attn(q: torch.Tensor, q_noise: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lam: torch.Tensor,
                    rms_weight: Optional[torch.Tensor] = None, eps: float = 1e-6, is_causal: bool = False,
                    sm_scale: Optional[float] = None) -> torch.Tensor:
    """out = RMSNorm(Attn(q,K,V) - lam * Attn(q_noise,K,V)) (same arguments and
    lower-right causal alignment as triton_diff_flash/__init__.py:86-146).

    q, q_noise (B,H,Lq,Dh); k, v (B,Hkv,Lk,Dh); lam (B,H,Lq,1); rms_weight
    (Dh,) or None for the identity norm.
    """
    _hip.require_device(q, q_noise, k, v, lam, rms_weight)
    B, H, Lq, Dh = q.shape
    Bk, Hkv, Lk, Dk = k.shape
    if (Bk, Dk) != (B, Dh) or tuple(v.shape) != tuple(k.shape) or tuple(q_noise.shape) != tuple(q.shape):
        raise RuntimeError(f"diff_flash_attn: shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if H % Hkv:
        raise RuntimeError(f"diff_flash_attn: H={H} not a multiple of Hkv={Hkv}")
    if is_causal and Lk < Lq:
        raise RuntimeError("diff_flash_attn: causal attention needs Lk >= Lq")
    dt = q.dtype
    if not (k.dtype == v.dtype == q_noise.dtype == lam.dtype == dt):
        raise RuntimeError("diff_flash_attn: q, q_noise, k, v, lam must share a dtype")
    q, q_noise, k, v = (_last_dim_contig(t) for t in (q, q_noise, k, v))
    lam3 = lam.reshape(B, H, Lq)
    out = torch.empty((B, H, Lq, Dh), dtype=dt, device=q.device)
    d = _hip.AttnDesc()
    d.dtype = _hip.dtype_code(dt)
    d.B, d.H, d.Hkv, d.Lq, d.Dh = B, H, Hkv, Lq, Dh
    d.q = q.data_ptr(); d.q_sb, d.q_sh, d.q_sl = _strides3(q)
    d.q_noise = q_noise.data_ptr(); d.qn_sb, d.qn_sh, d.qn_sl = _strides3(q_noise)
    d.kb, d.vb, d.Lb = k.data_ptr(), v.data_ptr(), Lk
    if k.stride() != v.stride():
        v = v.contiguous(); k = k.contiguous(); d.kb, d.vb = k.data_ptr(), v.data_ptr()
    d.b_sb, d.b_sh, d.b_sl = _strides3(k)
    d.causal = int(bool(is_causal))
    d.lam = lam3.data_ptr(); d.lam_sb, d.lam_sh, d.lam_sl = _strides3(lam3)
    w = None
    if rms_weight is not None:
        w = rms_weight.to(dt).contiguous()
        d.rms_w = w.data_ptr()
    d.eps = float(eps)
    d.sm_scale = float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(Dh)
    d.out = out.data_ptr(); d.o_sb, d.o_sh, d.o_sl = _strides3(out)
    _run_attn(d, q)
    return out


def attention_desc(*, q: torch.Tensor, rope_cos: Optional[torch.Tensor], rope_sin: Optional[torch.Tensor],
                   rope_interleaved: bool, theta_cos: torch.Tensor, theta_sin: torch.Tensor,
                   k_prefix: Optional[torch.Tensor], v_prefix: Optional[torch.Tensor],
                   allowed: Optional[torch.Tensor], k_block: Optional[torch.Tensor],
                   v_block: Optional[torch.Tensor], lam: torch.Tensor, rms_weight: Optional[torch.Tensor],
                   eps: float, out: torch.Tensor, causal: int = 1):
    """coda_attn_desc of the layer's bounded attention, plus the tensors it
    points to (kept alive by the caller until the launch is enqueued).

    q (B,H,Lq,Dh) pre-RoPE with (Lq, Dh/2) tables (or post-RoPE with
    rope_cos None); prefix = state cache (B,Hkv,Lbuf,Dh) masked by allowed
    (B,Lbuf) or fully visible (allowed None); block keys (B,Hkv,Lb,Dh)
    with causal mode 1 lower-right (the bounded chunk), 2 upper-left
    (torch SDPA is_causal), 0 none; lam (B,H,Lq) view.
    """
    B, H, Lq, Dh = q.shape
    if out.stride(-1) != 1:
        raise RuntimeError("bounded attention: out must have unit stride over head_dim (the kernels write "
                           "whole 16-byte channel runs)")
    q = _last_dim_contig(q)
    keep = [q]
    d = _hip.AttnDesc()
    d.dtype = _hip.dtype_code(q.dtype)
    d.B, d.H, d.Lq, d.Dh = B, H, Lq, Dh
    d.q = q.data_ptr(); d.q_sb, d.q_sh, d.q_sl = _strides3(q)
    d.theta_cos, d.theta_sin = theta_cos.data_ptr(), theta_sin.data_ptr()
    if rope_cos is not None:
        d.rope_cos, d.rope_sin = rope_cos.data_ptr(), rope_sin.data_ptr()
    d.rope_interleaved = int(bool(rope_interleaved))
    Hkv = None
    if k_prefix is not None and (k_prefix.stride() != v_prefix.stride() or k_prefix.stride(-1) != 1):
        k_prefix, v_prefix = k_prefix.contiguous(), v_prefix.contiguous()
        keep += [k_prefix, v_prefix]
    if k_block is not None and (k_block.stride() != v_block.stride() or k_block.stride(-1) != 1):
        k_block, v_block = k_block.contiguous(), v_block.contiguous()
        keep += [k_block, v_block]
    if k_prefix is not None:
        Hkv = k_prefix.shape[1]
        d.kp, d.vp, d.Lp = k_prefix.data_ptr(), v_prefix.data_ptr(), k_prefix.shape[2]
        d.p_sb, d.p_sh, d.p_sl = _strides3(k_prefix)
        if allowed is not None:
            d.allowed = allowed.data_ptr(); d.al_sb = int(allowed.stride(0))
    if k_block is not None:
        Hkv = k_block.shape[1]
        d.kb, d.vb, d.Lb = k_block.data_ptr(), v_block.data_ptr(), k_block.shape[2]
        d.b_sb, d.b_sh, d.b_sl = _strides3(k_block)
        d.causal = int(causal)
    d.Hkv = int(Hkv)
    d.lam = lam.data_ptr(); d.lam_sb, d.lam_sh, d.lam_sl = _strides3(lam)
    if rms_weight is not None:
        d.rms_w = rms_weight.data_ptr()
    d.eps = float(eps)
    d.sm_scale = 1.0 / math.sqrt(Dh)
    d.out = out.data_ptr(); d.o_sb, d.o_sh, d.o_sl = _strides3(out)
    return d, keep


def bounded_attention(**kw) -> torch.Tensor:
    """Attention of the layer's bounded path into `out` (see attention_desc)."""
    d, keep = attention_desc(**kw)
    _run_attn(d, kw["q"])
    return kw["out"]


def _epilogue(out_sig, out_noise, lam, weight, eps, out, norm: bool):
    _hip.require_device(out_sig, out_noise, lam, weight)
    if out_sig.shape != out_noise.shape:
        raise RuntimeError("diff_epilogue: out_sig and out_noise shapes differ")
    Dh = out_sig.shape[-1]
    rows = out_sig.numel() // Dh if Dh else 0
    if lam.numel() != rows:
        raise RuntimeError(f"diff_epilogue: lam has {lam.numel()} elements, expected {rows}")
    dt = out_sig.dtype
    sig, noi = out_sig.contiguous(), out_noise.contiguous()
    lam_flat = lam.reshape(-1).to(dt).contiguous()
    if out is None:
        out = torch.empty_like(sig)
    L = _hip.lib()
    st = _hip.stream_of(sig)
    if norm:
        w = weight.to(dt).contiguous()
        if w.numel() != Dh:
            raise RuntimeError(f"diff_epilogue: weight has {w.numel()} elements, expected {Dh}")
        _hip.check(L.coda_diff_epilogue_fwd(_hip.dtype_code(dt), out.data_ptr(), sig.data_ptr(), noi.data_ptr(),
                                            lam_flat.data_ptr(), w.data_ptr(), rows, Dh, float(eps), st))
    else:
        _hip.check(L.coda_diff_sub_only_fwd(_hip.dtype_code(dt), out.data_ptr(), sig.data_ptr(), noi.data_ptr(),
                                            lam_flat.data_ptr(), rows, Dh, st))
    return out


def diff_epilogue(out_sig: torch.Tensor, out_noise: torch.Tensor, lam: torch.Tensor, weight: torch.Tensor,
                  eps: float = 1e-6, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm(out_sig - lam * out_noise) * weight (coda_kernels/__init__.py:38-71)."""
    return _epilogue(out_sig, out_noise, lam, weight, eps, out, True)


def diff_sub_only(out_sig: torch.Tensor, out_noise: torch.Tensor, lam: torch.Tensor,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out_sig - lam * out_noise (coda_kernels/__init__.py:74-103)."""
    return _epilogue(out_sig, out_noise, lam, None, 0.0, out, False)
