"""The pipelined prefill (bank chain with per-chunk bank snapshots, then one
attention launch per group of chunks) against the CPU oracle and against the
chunk-by-chunk prefill of the same layer.

The chain runs as one library call per group (coda_block_write_chain) when
no per-chunk metrics, expansion flags or decision traces are collected; a
spy on the library counts those calls, so that each case shows which path
it took.  States must be byte-identical to the oracle's and to the
chunk-by-chunk path's; heads agree within the dtype's tolerance (the
grouped launch sums the softmax over the same keys in another order).
"""

from __future__ import annotations

import pytest
import torch

from parity_util import assert_close, compare_states, product_like, to_product_state

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# name: (H, Hkv, Dh, W, Me, Ms, B, L, block, gates, group chunks)
CASES = {
    # the 7B layer's per-KV-head geometry, one group
    "g4_b4_blk256": (8, 2, 128, 256, 64, 64, 4, 1536, 256, "random", None),
    # blocks of 128, a ragged last chunk and groups of 3 chunks
    "g4_b4_blk128_groups3": (8, 2, 128, 256, 64, 64, 4, 1189, 128, "random", 3),
    # the 70B layer's per-KV-head geometry
    "g8_b4_blk256": (16, 2, 128, 512, 128, 128, 4, 2048, 256, "random", None),
    # head_dim 64, G = 2, gates all tied, groups of 4
    "dh64_g2_ties": (4, 2, 64, 128, 32, 32, 8, 700, 64, "const", 4),
}


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _gates(kind, B, L, g):
    if kind == "const":
        v = torch.sigmoid(torch.tensor(-2.0, dtype=torch.bfloat16)).float()
        return v.expand(B, L).contiguous()
    return torch.sigmoid(torch.randn(B, L, generator=g) * 1.5 - 2.0)


def _inputs(m, B, L, kind, g, dtype=torch.bfloat16):
    H, Hkv, Dh = m.num_heads, m.num_kv_heads, m.head_dim
    q = torch.randn(B, H, L, Dh, generator=g).to(dtype)
    k = torch.randn(B, Hkv, L, Dh, generator=g).to(dtype)
    v = torch.randn(B, Hkv, L, Dh, generator=g).to(dtype)
    lam = torch.sigmoid(torch.randn(B, H, L, 1, generator=g) - 1.0).to(dtype)
    return q, k, v, _gates(kind, B, L, g), lam


class _ChainSpy:
    """The library with coda_block_write_chain counted."""

    def __init__(self, real):
        self._real = real
        self.chains = 0

    def __getattr__(self, name):
        return getattr(self._real, name)

    def coda_block_write_chain(self, *args):
        self.chains += 1
        return self._real.coda_block_write_chain(*args)


def _spy(monkeypatch):
    from coda_gqa_l import _hip
    spy = _ChainSpy(_hip.lib())
    monkeypatch.setattr(_hip, "lib", lambda: spy)
    return spy


def _layers(name, dtype=torch.bfloat16):
    from coda_oracle import OracleLayer
    H, Hkv, Dh, W, Me, Ms, B, L, block, kind, group = CASES[name]
    kw = dict(embed_dim=H * Dh, num_heads=H, num_kv_heads=Hkv, window=W, num_landmarks_exact=Me,
              num_landmarks_summary=Ms, rope_base=1e4)
    torch.manual_seed(51)
    m = OracleLayer(**kw).to(dtype).eval()
    p = product_like(m, {"kw": kw}, dtype, DEV)
    p.pipelined_group_chunks = group
    torch.manual_seed(52)
    st_o = m.init_state(batch_size=B, dtype=dtype)
    return m, p, st_o


def _run(p, st, q, k, v, gate, lam, c, s, block):
    return p.prefill_core(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV), lam.squeeze(-1).to(DEV), c.to(DEV),
                          s.to(DEV), st, block_size=block)


@pytest.mark.parametrize("name", list(CASES))
@torch.no_grad()
def test_pipelined_chain_matches_oracle(name, monkeypatch):
    """A fresh call (the ring fills inside it) and a ragged second call (the
    ring full at entry: its first chunks run one by one, the rest as a
    chain): heads and the whole state against the oracle after each."""
    _need_gpu()
    from coda_oracle import prims
    H, Hkv, Dh, W, Me, Ms, B, L, block, kind, group = CASES[name]
    print(f"[pipelined chain] {name}: H{H} Hkv{Hkv} Dh{Dh} W{W} Me{Me} Ms{Ms} B{B} L{L} block {block} "
          f"groups {group}", flush=True)
    dtype = torch.bfloat16
    m, p, st_o = _layers(name)
    st_p = to_product_state(st_o, DEV)
    spy = _spy(monkeypatch)
    g = torch.Generator().manual_seed(53)
    for call, Lc in enumerate((L, block * 3 + block // 2 + 5)):
        q, k, v, gate, lam = _inputs(m, B, Lc, kind, g)
        c, s = m.rope_tables(Lc, st_o.pos, dtype)
        before = spy.chains
        heads_o = m.prefill_core(prims.rope(q, c, s, m.rope_interleaved), k, v, gate, lam, st_o, block_size=block)
        heads_p = _run(p, st_p, q, k, v, gate, lam, c, s, block)
        torch.cuda.synchronize()
        assert spy.chains > before, f"{name} call {call}: the chain call did not run"
        assert_close(heads_p.permute(0, 2, 1, 3), heads_o, dtype, f"{name} call {call} heads")
        compare_states(st_p, st_o, dtype, W, Me, f"{name} call {call}")
    p.check_bank_status()


@pytest.mark.parametrize("name", ["g4_b4_blk128_groups3", "dh64_g2_ties"])
@torch.no_grad()
def test_pipelined_paths_equal_chunk_by_chunk(name, monkeypatch):
    """The chain call, the per-chunk snapshot path (forced by collecting
    metrics) and the chunk-by-chunk prefill leave byte-identical states;
    their heads agree within the tolerance."""
    _need_gpu()
    H, Hkv, Dh, W, Me, Ms, B, L, block, kind, group = CASES[name]
    print(f"[pipelined paths] {name}: B{B} L{L} block {block} groups {group}", flush=True)
    dtype = torch.bfloat16
    m, p, st0 = _layers(name)
    spy = _spy(monkeypatch)
    g = torch.Generator().manual_seed(54)
    q, k, v, gate, lam = _inputs(m, B, L, kind, g)
    c, s = m.rope_tables(L, 0, dtype)
    out = {}
    for mode in ("chain", "per_chunk_snapshots", "chunk_by_chunk"):
        st = to_product_state(st0, DEV)
        p.pipelined_prefill = mode != "chunk_by_chunk"
        if mode == "per_chunk_snapshots":
            from coda_gqa_l.memory_banks import METRIC_KEYS, DeviceMetrics
            st.metrics = DeviceMetrics({k: (0.0 if k.endswith("ratio") else 0) for k in METRIC_KEYS})
        before = spy.chains
        heads = _run(p, st, q, k, v, gate, lam, c, s, block)
        torch.cuda.synchronize()
        assert (spy.chains > before) == (mode == "chain"), f"{name} {mode}: chain calls {spy.chains - before}"
        out[mode] = (heads.cpu(), st)
    p.pipelined_prefill = True
    h_ref, st_ref = out["chunk_by_chunk"]
    from test_bench_shapes_gpu import _cpu_copy
    for mode in ("chain", "per_chunk_snapshots"):
        h, st = out[mode]
        assert_close(h, h_ref, dtype, f"{name} {mode}: heads")
        compare_states(st, _cpu_copy(st_ref), dtype, W, Me, f"{name} {mode} vs chunk by chunk")
    p.check_bank_status()


@pytest.mark.parametrize("case", ["four_launch_fallback", "short_calls"])
@torch.no_grad()
def test_pipelined_prefill_fallbacks_match_oracle(case, monkeypatch):
    """Where the chain cannot run, the layer falls back without losing
    state: with the one-launch update switched off (CODA_BLOCK_FUSED=0) the
    chain call returns CODA_EUNSUP before enqueueing anything and the call
    continues chunk by chunk on the four-launch update; calls shorter than
    one block, and calls of exactly one block, take the ordinary paths.
    Heads and the whole state against the oracle after every call."""
    _need_gpu()
    from coda_oracle import prims
    name = "g4_b4_blk128_groups3"
    H, Hkv, Dh, W, Me, Ms, B, L, block, kind, _ = CASES[name]
    print(f"[pipelined fallbacks] {case}", flush=True)
    dtype = torch.bfloat16
    m, p, st_o = _layers(name)
    st_p = to_product_state(st_o, DEV)
    if case == "four_launch_fallback":
        monkeypatch.setenv("CODA_BLOCK_FUSED", "0")
        lengths = (L, block * 2 + 17)
    else:
        lengths = (100, block, 3, block * 3 + 1, 57)
    g = torch.Generator().manual_seed(56)
    for call, Lc in enumerate(lengths):
        q, k, v, gate, lam = _inputs(m, B, Lc, kind, g)
        c, s = m.rope_tables(Lc, st_o.pos, dtype)
        heads_o = m.prefill_core(prims.rope(q, c, s, m.rope_interleaved), k, v, gate, lam, st_o, block_size=block)
        heads_p = _run(p, st_p, q, k, v, gate, lam, c, s, block)
        torch.cuda.synchronize()
        assert_close(heads_p.permute(0, 2, 1, 3), heads_o, dtype, f"{case} call {call} ({Lc} tokens) heads")
        compare_states(st_p, st_o, dtype, W, Me, f"{case} call {call} ({Lc} tokens)")
    p.check_bank_status()
