"""Callers of the bounded layer: drop-in attention modules for Llama-family,
Qwen3 and Eve-2 models (reference: llama_adapter.py, qwen3_adapter.py,
eve_adapter.py).  Each holds one CoDAGQALandmarkPerf2 (``bounded=True``,
streaming with a persistent state) or one CoDAGQA (``bounded=False``, plain
causal attention), copies the host model's projection weights and biases
1:1, and keeps the host layer's forward signature.

Everything runs on the HIP path; the modules are inference-only, like the
layers they hold (the reference's training branch, which re-creates a
zero-initialised state on every forward, has no backward kernels here and
raises instead).

Defaults follow the reference: Llama / Qwen3 cold-swap with the contiguous-
half RoPE layout and no head norm (``rope_interleaved=False``,
``head_norm_mode="identity"``), Eve-2 with interleaved RoPE and the full
HeadwiseRMSNorm.  The re-exports in llama_adapter.py, qwen3_adapter.py and
eve_adapter.py keep the reference's import paths.
"""

from __future__ import annotations

import math
import warnings
from typing import List, Optional, Tuple

import torch
import torch.nn as nn

from .attention import CoDAGQALandmarkPerf2
from .baseline import CoDAGQA
from .state import CoDAGQALandmarkStatePerf2

__all__ = ["LlamaCoDAAdapter", "Qwen3CoDAAdapter", "EveCoDAAdapter"]


def _copy_linear(dst_owner: nn.Module, name: str, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> None:
    """Copy ``weight`` (and ``bias``) into ``dst_owner.<name>``, replacing the
    layer by a biased nn.Linear of the same shape when a bias comes along."""
    lin = getattr(dst_owner, name)
    if tuple(lin.weight.shape) != tuple(weight.shape):
        raise ValueError(f"{name}: weight {tuple(weight.shape)} does not fit {tuple(lin.weight.shape)}")
    if bias is not None and lin.bias is None:
        new = nn.Linear(lin.in_features, lin.out_features, bias=True,
                        device=lin.weight.device, dtype=lin.weight.dtype)
        setattr(dst_owner, name, new)
        lin = new
    with torch.no_grad():
        lin.weight.copy_(weight)
        if bias is not None:
            lin.bias.copy_(bias)


class _CoDAAdapter(nn.Module):
    """The bounded / unbounded layer and the streaming state of one
    attention slot of a host model."""

    def __init__(self, *, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int, bounded: bool,
                 rope_theta: float, lambda_init_bias: float, theta_init: float, eps: float, head_norm_mode: str,
                 rope_interleaved: bool, window: int, num_landmarks_exact: int, num_landmarks_summary: int,
                 block_size: int, **coda_kwargs):
        super().__init__()
        if hidden_size != num_heads * head_dim:
            raise ValueError(f"hidden_size {hidden_size} != num_heads {num_heads} * head_dim {head_dim}: "
                             "the layer projects to and from hidden_size")
        self.hidden_size, self.num_heads, self.num_kv_heads = hidden_size, num_heads, num_kv_heads
        self.head_dim, self.bounded, self.block_size = head_dim, bool(bounded), int(block_size)
        common = dict(embed_dim=hidden_size, num_heads=num_heads, num_kv_heads=num_kv_heads, rope_base=rope_theta,
                      lambda_init_bias=lambda_init_bias, theta_init=theta_init, eps=eps,
                      head_norm_mode=head_norm_mode, rope_interleaved=rope_interleaved)
        if self.bounded:
            self.coda = CoDAGQALandmarkPerf2(window=window, num_landmarks_exact=num_landmarks_exact,
                                             num_landmarks_summary=num_landmarks_summary, **common, **coda_kwargs)
        else:
            self.coda = CoDAGQA(**common)
        self._state: Optional[CoDAGQALandmarkStatePerf2] = None

    # ------------------------------------------------------------ forward
    def _attend(self, x: torch.Tensor) -> torch.Tensor:
        if self.training:
            raise NotImplementedError(f"{type(self).__name__} is inference-only on MI355X (no backward kernels); "
                                      "call .eval()")
        if not self.bounded:
            y, _ = self.coda(x, is_causal=True)
            return y
        if self._state is None:
            self._state = self.coda.init_state(batch_size=x.shape[0], device=x.device, dtype=x.dtype)
        if x.shape[1] == 1:
            y, self._state = self.coda.step(x, self._state)
        else:
            y, self._state = self.coda.prefill_chunked(x, self._state, block_size=self.block_size)
        return y

    # ------------------------------------------------------------ state
    def init_inference_state(self, batch_size: int, device: torch.device,
                             dtype: torch.dtype) -> CoDAGQALandmarkStatePerf2:
        if not self.bounded:
            raise RuntimeError("init_inference_state() requires bounded=True")
        self._state = self.coda.init_state(batch_size=batch_size, device=device, dtype=dtype)
        return self._state

    def get_state(self) -> Optional[CoDAGQALandmarkStatePerf2]:
        return self._state

    def set_state(self, state: CoDAGQALandmarkStatePerf2) -> None:
        """Continue from a saved state (see coda_gqa_l.state_io)."""
        self._state = state

    def reset_state(self) -> None:
        self._state = None

    def cache_bytes(self, *, batch_size: int, dtype: torch.dtype) -> int:
        if not self.bounded:
            raise RuntimeError("cache_bytes() requires bounded=True")
        return self.coda.cache_bytes(batch_size=batch_size, dtype=dtype)

    def extra_repr(self) -> str:
        return (f"hidden_size={self.hidden_size}, num_heads={self.num_heads}, num_kv_heads={self.num_kv_heads}, "
                f"head_dim={self.head_dim}, mode={'bounded' if self.bounded else 'unbounded'}")


def _attn_shape(attn: nn.Module) -> Tuple[int, int, int, int]:
    """(hidden, heads, kv heads, head_dim) of a Llama-style attention module,
    from its attributes or, missing those, from the projection shapes."""
    hidden = attn.q_proj.in_features
    q_out, k_out = attn.q_proj.out_features, attn.k_proj.out_features
    cfg = getattr(attn, "config", None)
    heads = getattr(attn, "num_heads", None) or getattr(cfg, "num_attention_heads", None)
    kv = getattr(attn, "num_key_value_heads", None) or getattr(cfg, "num_key_value_heads", None)
    hd = getattr(attn, "head_dim", None)
    if hd is None:
        if heads:
            hd = q_out // heads
        else:
            hd = next((d for d in (128, 64, 96, 256) if q_out % d == 0), None)
            if hd is None:
                raise ValueError(f"cannot infer head_dim from q_proj width {q_out}")
    heads = heads or q_out // hd
    kv = kv or k_out // hd
    return hidden, int(heads), int(kv), int(hd)


def _rope_theta(cfg, default: float) -> float:
    """RoPE base of a HF config: ``rope_theta`` (transformers 4) or
    ``rope_parameters["rope_theta"]`` (transformers 5)."""
    theta = getattr(cfg, "rope_theta", None)
    if theta is None:
        rp = getattr(cfg, "rope_parameters", None)
        theta = rp.get("rope_theta") if isinstance(rp, dict) else None
    return float(theta) if theta is not None else float(default)


class LlamaCoDAAdapter(_CoDAAdapter):
    """Replacement for a Llama-family attention module (LlamaAttention,
    Mistral, SmolLM, ...): ``forward(hidden_states, ...) -> (y,
    past_key_value)``; RoPE and the cache live inside the layer, so position
    ids, masks and HF cache objects are accepted and ignored
    (llama_adapter.py:27-420)."""

    _default_theta = 10_000.0

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int, bounded: bool = False,
                 rope_theta: float = 10_000.0, lambda_init_bias: float = -6.0, theta_init: float = math.pi / 2,
                 eps: float = 1e-6, head_norm_mode: str = "identity", rope_interleaved: bool = False,
                 window: int = 256, num_landmarks_exact: int = 64, num_landmarks_summary: int = 64,
                 block_size: int = 1024, **coda_kwargs):
        super().__init__(hidden_size=hidden_size, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                         bounded=bounded, rope_theta=rope_theta, lambda_init_bias=lambda_init_bias,
                         theta_init=theta_init, eps=eps, head_norm_mode=head_norm_mode,
                         rope_interleaved=rope_interleaved, window=window, num_landmarks_exact=num_landmarks_exact,
                         num_landmarks_summary=num_landmarks_summary, block_size=block_size, **coda_kwargs)

    @classmethod
    def _from_attention(cls, attn: nn.Module, bounded: bool, head_norm_mode: str, rope_interleaved: bool,
                        warn: bool, **coda_kwargs):
        hidden, heads, kv, hd = _attn_shape(attn)
        theta = _rope_theta(getattr(attn, "config", None), cls._default_theta)
        if warn and (rope_interleaved is not True or head_norm_mode != "full"):
            warnings.warn(
                f"{cls.__name__}: rope_interleaved={rope_interleaved}, head_norm_mode={head_norm_mode!r} differ "
                "from the CoDAGQA / CoDAGQALandmarkPerf2 defaults (True, 'full'); weights trained with those "
                "defaults need them passed here, or the outputs diverge", UserWarning, stacklevel=3)
        ad = cls(hidden_size=hidden, num_heads=heads, num_kv_heads=kv, head_dim=hd, bounded=bounded,
                 rope_theta=theta, head_norm_mode=head_norm_mode, rope_interleaved=rope_interleaved, **coda_kwargs)
        ref = next(attn.parameters())
        ad.coda.to(device=ref.device, dtype=ref.dtype)
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            src = getattr(attn, name)
            _copy_linear(ad.coda, name, src.weight.detach(), None if src.bias is None else src.bias.detach())
        return ad

    @classmethod
    def from_llama_attention(cls, llama_attn: nn.Module, bounded: bool = False, head_norm_mode: str = "identity",
                             rope_interleaved: bool = False, **coda_kwargs) -> "LlamaCoDAAdapter":
        """Adapter with the weights (and biases) of ``llama_attn`` copied 1:1;
        ``rope_theta`` from its config when it has one."""
        return cls._from_attention(llama_attn, bounded, head_norm_mode, rope_interleaved, True, **coda_kwargs)

    @classmethod
    def swap_llama_layers(cls, model: nn.Module, bounded: bool = False, head_norm_mode: str = "identity",
                          rope_interleaved: bool = False, **coda_kwargs) -> List["LlamaCoDAAdapter"]:
        """Replace ``model.model.layers[i].self_attn`` by adapters, in place."""
        adapters = []
        for block in model.model.layers:
            ad = cls.from_llama_attention(block.self_attn, bounded=bounded, head_norm_mode=head_norm_mode,
                                          rope_interleaved=rope_interleaved, **coda_kwargs)
            block.self_attn = ad
            adapters.append(ad)
        return adapters

    def forward(self, hidden_states: torch.Tensor, attention_mask: object = None, position_ids: object = None,
                past_key_value: object = None, output_attentions: bool = False, use_cache: bool = False,
                cache_position: object = None, position_embeddings: object = None, **kwargs):
        """Returns ``(y, past_key_value)`` as Llama decoder layers unpack it."""
        return self._attend(hidden_states), past_key_value


class Qwen3CoDAAdapter(LlamaCoDAAdapter):
    """Replacement for Qwen3 attention: the Llama layout with Qwen3's RoPE base
    (1e6) as the default (qwen3_adapter.py:20-219).  Qwen3's per-head q/k
    norms are not part of the layer (cold swap, as in the reference)."""

    _default_theta = 1_000_000.0

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int, bounded: bool = False,
                 rope_theta: float = 1_000_000.0, lambda_init_bias: float = -6.0, theta_init: float = math.pi / 2,
                 eps: float = 1e-6, head_norm_mode: str = "identity", rope_interleaved: bool = False,
                 window: int = 256, num_landmarks_exact: int = 64, num_landmarks_summary: int = 64,
                 block_size: int = 1024, **coda_kwargs):
        super().__init__(hidden_size, num_heads, num_kv_heads, head_dim, bounded=bounded, rope_theta=rope_theta,
                         lambda_init_bias=lambda_init_bias, theta_init=theta_init, eps=eps,
                         head_norm_mode=head_norm_mode, rope_interleaved=rope_interleaved, window=window,
                         num_landmarks_exact=num_landmarks_exact, num_landmarks_summary=num_landmarks_summary,
                         block_size=block_size, **coda_kwargs)

    @classmethod
    def from_qwen3_attention(cls, qwen3_attn: nn.Module, bounded: bool = False, head_norm_mode: str = "identity",
                             rope_interleaved: bool = False, **coda_kwargs) -> "Qwen3CoDAAdapter":
        return cls._from_attention(qwen3_attn, bounded, head_norm_mode, rope_interleaved, False, **coda_kwargs)

    @classmethod
    def swap_qwen3_layers(cls, model: nn.Module, bounded: bool = False, head_norm_mode: str = "identity",
                          rope_interleaved: bool = False, **coda_kwargs) -> List["Qwen3CoDAAdapter"]:
        adapters = []
        for block in model.model.layers:
            ad = cls.from_qwen3_attention(block.self_attn, bounded=bounded, head_norm_mode=head_norm_mode,
                                          rope_interleaved=rope_interleaved, **coda_kwargs)
            block.self_attn = ad
            adapters.append(ad)
        return adapters


class EveCoDAAdapter(_CoDAAdapter):
    """Replacement for Eve-2's CausalSelfAttention: multi-head (as many KV
    heads as query heads), fused ``c_attn`` QKV projection and ``c_proj``
    output, biases on both; ``forward(x, freqs_cis=None) -> y``, the complex
    RoPE table ignored in favour of the layer's own interleaved RoPE with the
    same base (eve_adapter.py:30-465)."""

    def __init__(self, n_embd: int, n_head: int, head_dim: int, bounded: bool = False, rope_theta: float = 10_000.0,
                 lambda_init_bias: float = -6.0, theta_init: float = math.pi / 2, eps: float = 1e-6,
                 head_norm_mode: str = "full", rope_interleaved: bool = True, window: int = 256,
                 num_landmarks_exact: int = 64, num_landmarks_summary: int = 64, block_size: int = 1024,
                 **coda_kwargs):
        super().__init__(hidden_size=n_embd, num_heads=n_head, num_kv_heads=n_head, head_dim=head_dim,
                         bounded=bounded, rope_theta=rope_theta, lambda_init_bias=lambda_init_bias,
                         theta_init=theta_init, eps=eps, head_norm_mode=head_norm_mode,
                         rope_interleaved=rope_interleaved, window=window, num_landmarks_exact=num_landmarks_exact,
                         num_landmarks_summary=num_landmarks_summary, block_size=block_size, **coda_kwargs)
        self.n_embd, self.n_head = n_embd, n_head

    @classmethod
    def from_eve_attention(cls, eve_attn: nn.Module, bounded: bool = False, head_norm_mode: str = "full",
                           rope_interleaved: bool = True, **coda_kwargs) -> "EveCoDAAdapter":
        ad = cls(n_embd=eve_attn.n_embd, n_head=eve_attn.n_head, head_dim=eve_attn.head_dim, bounded=bounded,
                 head_norm_mode=head_norm_mode, rope_interleaved=rope_interleaved, **coda_kwargs)
        ref = eve_attn.c_attn.weight
        ad.coda.to(device=ref.device, dtype=ref.dtype)
        ad.load_eve_weights(c_attn_weight=eve_attn.c_attn.weight.detach(),
                            c_attn_bias=None if eve_attn.c_attn.bias is None else eve_attn.c_attn.bias.detach(),
                            c_proj_weight=eve_attn.c_proj.weight.detach(),
                            c_proj_bias=None if eve_attn.c_proj.bias is None else eve_attn.c_proj.bias.detach())
        return ad

    def load_eve_weights(self, *, c_attn_weight: torch.Tensor, c_attn_bias: Optional[torch.Tensor] = None,
                         c_proj_weight: torch.Tensor, c_proj_bias: Optional[torch.Tensor] = None) -> None:
        """Split the fused QKV weight (3 n_embd, n_embd) and bias (3 n_embd)
        into the layer's q / k / v projections; c_proj into o_proj."""
        n = self.n_embd
        if tuple(c_attn_weight.shape) != (3 * n, n):
            raise ValueError(f"c_attn weight {tuple(c_attn_weight.shape)}, expected {(3 * n, n)}")
        for i, name in enumerate(("q_proj", "k_proj", "v_proj")):
            b = None if c_attn_bias is None else c_attn_bias[i * n:(i + 1) * n]
            _copy_linear(self.coda, name, c_attn_weight[i * n:(i + 1) * n], b)
        _copy_linear(self.coda, "o_proj", c_proj_weight, c_proj_bias)

    def forward(self, x: torch.Tensor, freqs_cis: object = None) -> torch.Tensor:
        return self._attend(x)
