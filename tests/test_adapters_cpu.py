"""Adapters (callers of the bounded layer): weight and bias mapping from the
host modules, shapes and RoPE base taken from HF configs, layer swaps in
tiny random-init HF models, argument checks (CPU only: no kernel runs; the
end-to-end runs are in test_parity_gpu.py)."""

from __future__ import annotations

import warnings

import pytest
import torch
import torch.nn as nn

from coda_gqa_l import EveCoDAAdapter, LlamaCoDAAdapter, Qwen3CoDAAdapter
from coda_gqa_l.llama_adapter import LlamaCoDAAdapter as LlamaFromRefPath

transformers = pytest.importorskip("transformers")


def _tiny_llama(bias: bool = False, layers: int = 2):
    cfg = transformers.LlamaConfig(hidden_size=256, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                                   num_hidden_layers=layers, vocab_size=97, intermediate_size=512,
                                   rope_theta=5e5, attention_bias=bias)
    torch.manual_seed(0)
    return transformers.LlamaForCausalLM(cfg).eval()


class EveAttention(nn.Module):
    """The layout of Eve-2's CausalSelfAttention: fused QKV, biases."""

    def __init__(self, n_embd=512, n_head=8, bias=True):
        super().__init__()
        self.n_embd, self.n_head, self.head_dim = n_embd, n_head, n_embd // n_head
        self.c_attn = nn.Linear(n_embd, 3 * n_embd, bias=bias)
        self.c_proj = nn.Linear(n_embd, n_embd, bias=bias)


def test_reference_import_path():
    assert LlamaFromRefPath is LlamaCoDAAdapter


@pytest.mark.parametrize("bounded", [True, False])
@pytest.mark.parametrize("bias", [False, True])
def test_llama_weights_map_one_to_one(bounded, bias):
    model = _tiny_llama(bias=bias)
    attn = model.model.layers[1].self_attn
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        ad = LlamaCoDAAdapter.from_llama_attention(attn, bounded=bounded, window=32, num_landmarks_exact=8,
                                                   num_landmarks_summary=8)
    assert any("differ from the CoDAGQA" in str(x.message) for x in w)
    assert (ad.num_heads, ad.num_kv_heads, ad.head_dim, ad.hidden_size) == (4, 2, 64, 256)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        src, dst = getattr(attn, name), getattr(ad.coda, name)
        assert torch.equal(src.weight, dst.weight), name
        assert (src.bias is None) == (dst.bias is None), name
        if src.bias is not None:
            assert torch.equal(src.bias, dst.bias), name
    assert ad.coda.head_norm_mode == "identity" and ad.coda.rope_interleaved is False
    assert ad.bounded is bounded


@pytest.mark.filterwarnings("ignore:LlamaCoDAAdapter")
def test_llama_rope_base_from_config():
    model = _tiny_llama()
    ad = LlamaCoDAAdapter.from_llama_attention(model.model.layers[0].self_attn, bounded=True, window=32,
                                               num_landmarks_exact=8, num_landmarks_summary=8)
    cos, _ = ad.coda.rope(seq_len=2, offset=0, device="cpu", dtype=torch.float32)
    inv = 1.0 / (5e5 ** (torch.arange(0, 64, 2, dtype=torch.float64) / 64))
    assert torch.allclose(cos[1].double(), torch.cos(inv), atol=1e-6)


@pytest.mark.filterwarnings("ignore:LlamaCoDAAdapter")
def test_swap_llama_layers_in_place():
    model = _tiny_llama(layers=3)
    adapters = LlamaCoDAAdapter.swap_llama_layers(model, bounded=True, window=32, num_landmarks_exact=8,
                                                  num_landmarks_summary=8, block_size=64)
    assert len(adapters) == 3
    for block, ad in zip(model.model.layers, adapters):
        assert block.self_attn is ad and ad.block_size == 64


def test_qwen3_defaults_and_swap():
    cfg = transformers.Qwen3Config(hidden_size=256, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                                   num_hidden_layers=2, vocab_size=97, intermediate_size=512)
    model = transformers.Qwen3ForCausalLM(cfg).eval()
    ads = Qwen3CoDAAdapter.swap_qwen3_layers(model, bounded=True, window=32, num_landmarks_exact=8,
                                             num_landmarks_summary=8)
    assert len(ads) == 2 and isinstance(ads[0], Qwen3CoDAAdapter)
    ad = Qwen3CoDAAdapter(hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64, bounded=True, window=32,
                          num_landmarks_exact=8, num_landmarks_summary=8)
    cos, _ = ad.coda.rope(seq_len=2, offset=0, device="cpu", dtype=torch.float32)
    assert torch.allclose(cos[1].double(), torch.cos(1.0 / (1e6 ** (torch.arange(0, 64, 2, dtype=torch.float64) / 64))),
                          atol=1e-6)


@pytest.mark.parametrize("bias", [True, False])
def test_eve_fused_qkv_is_split(bias):
    torch.manual_seed(1)
    eve = EveAttention(bias=bias)
    ad = EveCoDAAdapter.from_eve_attention(eve, bounded=True, window=32, num_landmarks_exact=8,
                                           num_landmarks_summary=8)
    n = 512
    assert ad.num_kv_heads == ad.num_heads == 8 and ad.head_dim == 64
    for i, name in enumerate(("q_proj", "k_proj", "v_proj")):
        lin = getattr(ad.coda, name)
        assert torch.equal(lin.weight, eve.c_attn.weight[i * n:(i + 1) * n])
        if bias:
            assert torch.equal(lin.bias, eve.c_attn.bias[i * n:(i + 1) * n])
        else:
            assert lin.bias is None
    assert torch.equal(ad.coda.o_proj.weight, eve.c_proj.weight)
    assert ad.coda.head_norm_mode == "full" and ad.coda.rope_interleaved is True
    with pytest.raises(ValueError):
        ad.load_eve_weights(c_attn_weight=torch.zeros(3 * n, n + 1), c_proj_weight=torch.zeros(n, n))


def test_inference_only_and_device_checks():
    ad = LlamaCoDAAdapter(hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64, bounded=True, window=32,
                          num_landmarks_exact=8, num_landmarks_summary=8)
    ad.train()
    with pytest.raises(NotImplementedError):
        ad(torch.zeros(1, 3, 256))
    ad.eval()
    with pytest.raises(RuntimeError):
        ad(torch.zeros(1, 3, 256))            # CPU tensors: the kernels need a HIP device
    with pytest.raises(ValueError):
        LlamaCoDAAdapter(hidden_size=200, num_heads=4, num_kv_heads=2, head_dim=64)
    with pytest.raises(RuntimeError):
        LlamaCoDAAdapter(hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64).init_inference_state(
            1, torch.device("cpu"), torch.float32)
