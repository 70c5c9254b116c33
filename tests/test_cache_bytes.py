"""cache_bytes (reference attention.py:734-751) against the sizes the
reference publishes: 217.9 KB for the D512 test model with the medium cache
(README.md:133; bf16, batch 1) and 1,771,392 bytes for one 7B-shaped layer
with the medium cache (README.md:195-203: "1.5 MB" of K/V plus the norm
caches and metadata; bf16, batch 1).  The byte count is summed from the
state's own tensors in the GPU test."""

from __future__ import annotations

import pytest
import torch

MEDIUM = dict(window=256, num_landmarks_exact=64, num_landmarks_summary=64)


def _product(**kw):
    from coda_gqa_l import CoDAGQALandmarkPerf2
    with torch.device("meta"):
        return CoDAGQALandmarkPerf2(**kw)


@pytest.mark.parametrize("kw,expect", [
    (dict(embed_dim=512, num_heads=8, num_kv_heads=2, **MEDIUM), 223_104),
    (dict(embed_dim=4096, num_heads=32, num_kv_heads=8, rope_base=1e4, **MEDIUM), 1_771_392),
])
def test_cache_bytes_equals_the_published_sizes(kw, expect):
    m = _product(**kw)
    got = m.cache_bytes(batch_size=1, dtype=torch.bfloat16)
    assert got == expect
    if expect == 223_104:
        assert round(got / 1024, 1) == 217.9   # README.md:133 quotes KiB
    # linear in the batch; fp32 K/V and norm caches double those parts only
    assert m.cache_bytes(batch_size=3, dtype=torch.bfloat16) == 3 * expect
    Hkv, Dh, Lbuf, Me, Ms = kw["num_kv_heads"], kw["embed_dim"] // kw["num_heads"], 384, 64, 64
    tensors_bf16 = 2 * Hkv * Lbuf * Dh * 2 + Hkv * Me * Dh * 2 + Hkv * Ms * (Dh // 2) * 2
    assert m.cache_bytes(batch_size=1, dtype=torch.float32) == expect + tensors_bf16


def test_cache_bytes_matches_the_oracle():
    import sys, os
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", "oracle"))
    from coda_oracle import OracleLayer
    for kw in (dict(embed_dim=512, num_heads=8, num_kv_heads=2, **MEDIUM),
               dict(embed_dim=256, num_heads=4, num_kv_heads=4, window=32, num_landmarks_exact=0,
                    num_landmarks_summary=16)):
        o = OracleLayer(**kw)
        m = _product(**kw)
        for dt in (torch.float32, torch.bfloat16):
            assert m.cache_bytes(batch_size=2, dtype=dt) == o.cache_bytes(batch_size=2, dtype=dt)


@pytest.mark.gpu
def test_cache_bytes_is_the_state_size():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from coda_gqa_l import CoDAGQALandmarkPerf2
    m = CoDAGQALandmarkPerf2(embed_dim=512, num_heads=8, num_kv_heads=2, **MEDIUM).to("cuda:0", torch.bfloat16)
    st = m.init_state(batch_size=2, device="cuda:0", dtype=torch.bfloat16)
    n = sum(t.numel() * t.element_size() for t in (st.k_buf, st.v_buf, st.allowed, st.g_recent,
                                                    st.mem_last_exact, st._exact_v_norm, st._sum_lf_k_norm))
    assert n == m.cache_bytes(batch_size=2, dtype=torch.bfloat16) == 2 * 223_104
