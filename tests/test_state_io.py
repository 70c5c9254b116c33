"""State files: the reference's on-disk layout ({"states": {i: state},
"metadata": ...}, neural_db.py:285-308), loaded with weights_only=True, and
the dtype each field keeps when moved to a device (CPU; the GPU round trip
through a decode step is in test_parity_gpu.py)."""

from __future__ import annotations

import pickle

import pytest
import torch

from coda_gqa_l import CoDAGQALandmarkStatePerf2
from coda_gqa_l.state_io import deep_copy_state, load_state, save_state, state_to_cpu, state_to_device


def _state(seed: int, B=2, Hkv=2, W=8, Me=4, Ms=4, Dh=16, dtype=torch.bfloat16, metrics=True):
    g = torch.Generator().manual_seed(seed)
    L = W + Me + Ms
    return CoDAGQALandmarkStatePerf2(
        k_buf=torch.randn(B, Hkv, L, Dh, generator=g).to(dtype),
        v_buf=torch.randn(B, Hkv, L, Dh, generator=g).to(dtype),
        allowed=torch.rand(B, L, generator=g) > 0.3,
        g_recent=torch.rand(B, W, generator=g),
        recent_idx=3, recent_filled=W,
        mem_last_exact=torch.randint(-1, 1000, (B, Me), generator=g),
        pos=1234 + seed, active_exact=Me, active_summary=Ms,
        _exact_v_norm=torch.randn(B, Hkv, Me, Dh, generator=g).to(dtype),
        _sum_lf_k_norm=torch.randn(B, Hkv, Ms, Dh // 2, generator=g).to(dtype),
        metrics={"exact_hits": 5, "exact_fill_ratio": 0.25} if metrics else None,
    )


FIELDS = ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm")
INTS = ("recent_idx", "recent_filled", "pos", "active_exact", "active_summary")


def _same(a, b):
    for f in FIELDS:
        ta, tb = getattr(a, f), getattr(b, f)
        assert ta.dtype == tb.dtype and ta.shape == tb.shape, f
        assert torch.equal(ta, tb), f
    for f in INTS:
        assert getattr(a, f) == getattr(b, f), f
    assert a.metrics == b.metrics


def test_save_load_round_trip(tmp_path):
    states = {0: _state(1), 1: _state(2, metrics=False)}
    meta = {"model_id": "local", "window": 8, "num_tokens": 77, "timestamp": 1.5}
    path = tmp_path / "doc.pt"
    size = save_state({"states": states, "metadata": meta}, path)
    assert size == path.stat().st_size > 0
    loaded = load_state(path)
    assert set(loaded) == {"states", "metadata"} and loaded["metadata"] == meta
    assert set(loaded["states"]) == {0, 1}
    for k, st in states.items():
        got = loaded["states"][k]
        assert type(got) is CoDAGQALandmarkStatePerf2
        _same(st, got)


def test_reference_style_file_loads(tmp_path):
    """A file written like the reference's NeuralDatabase.save_state (one
    torch.save of the dict holding the state dataclass) loads without
    weights_only=False."""
    path = tmp_path / "ref.pt"
    st = _state(3)
    torch.save({"states": {0: st}, "metadata": {"num_landmarks_exact": 4}}, path)
    loaded = load_state(path)
    _same(st, loaded["states"][0])
    with pytest.raises(pickle.UnpicklingError):
        torch.load(path, map_location="cpu", weights_only=True)   # the allow-list is what makes it load


class Foreign:
    """Any class outside the allow-list."""


def test_load_refuses_foreign_objects(tmp_path):
    path = tmp_path / "bad.pt"
    torch.save({"states": {}, "metadata": {"x": Foreign()}}, path)
    with pytest.raises(pickle.UnpicklingError):
        load_state(path)


def test_state_to_device_keeps_norm_caches_in_the_model_dtype():
    st = _state(4)
    st._exact_v_norm = st._exact_v_norm.float()          # as the reference leaves them after a restore
    st._sum_lf_k_norm = st._sum_lf_k_norm.float()
    st.g_recent = st.g_recent.double()
    out = state_to_device(st, "cpu", torch.bfloat16)
    assert out is st
    assert st.k_buf.dtype == st.v_buf.dtype == torch.bfloat16
    assert st._exact_v_norm.dtype == st._sum_lf_k_norm.dtype == torch.bfloat16
    assert st.g_recent.dtype == torch.float32 and st.allowed.dtype == torch.bool
    assert st.mem_last_exact.dtype == torch.int64


def test_copies_are_independent():
    st = _state(5)
    cp = deep_copy_state(st)
    cpu = state_to_cpu(st)
    _same(st, cp)
    _same(st, cpu)
    cp.k_buf.zero_()
    cp.metrics["exact_hits"] = -1
    assert not torch.equal(st.k_buf, cp.k_buf)
    assert st.metrics["exact_hits"] == 5
