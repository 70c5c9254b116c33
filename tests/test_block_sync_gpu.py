"""The one-launch chunk update's cross-workgroup waits (coda_block_write):

- replayed from a captured HIP graph, whose launch arguments (the host's
  epoch included) are fixed, every replay meets its own sync words: the
  state after each replay equals the eager call's, byte for byte;
- a wait that gives up (forced from the host with a negative spin limit, so
  every kernel still exits normally) is reported: the workspace's status
  word counts it and the layer raises instead of returning a state that is
  silently wrong.

Reference path: the bank update of prefill_chunked
(memory_banks.py:438-564, 570-950), which has no cross-workgroup wait."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF16 = torch.bfloat16

# give-ups this module forces on purpose (test_block_write_sync_never_gave_up
# discounts them)
FORCED = {"n": 0}


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _layer_with_full_ring(B, seed):
    import coda_gqa_l
    torch.manual_seed(seed)
    m = coda_gqa_l.CoDAGQALandmarkPerf2(embed_dim=1024, num_heads=8, num_kv_heads=2, window=64,
                                        num_landmarks_exact=32, num_landmarks_summary=32).to(BF16).to(DEV).eval()
    st = m.init_state(batch_size=B, device=DEV, dtype=BF16)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    with torch.no_grad():
        m.prefill_chunked(torch.randn(B, 200, 1024, generator=g, device=DEV, dtype=BF16), st, block_size=64,
                          return_outputs=False)
    torch.cuda.synchronize()
    m.check_bank_status()
    return m, st, g


def _snapshot(st):
    f = ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm")
    return {k: getattr(st, k).clone() for k in f}


def _restore(st, snap):
    for k, t in snap.items():
        getattr(st, k).copy_(t)


@torch.no_grad()
def test_block_write_replays_from_a_captured_graph_match_eager():
    _need_gpu()
    from coda_gqa_l import _hip
    B, blk = 6, 96
    print(f"[graph replay] B{B} block {blk}", flush=True)
    m, st, g = _layer_with_full_ring(B, seed=21)
    Hkv, Dh, W = m.num_kv_heads, m.head_dim, m.window
    k = torch.randn(B, Hkv, blk, Dh, generator=g, device=DEV, dtype=BF16)
    v = torch.randn(B, Hkv, blk, Dh, generator=g, device=DEV, dtype=BF16)
    gate = torch.sigmoid(torch.randn(B, blk, generator=g, device=DEV) * 1.5 - 2.0).contiguous()
    plan, kmax, do_e, do_s = m._plan_candidates(st, gate, blk, blk)
    Te = min(m.exact_candidates_per_block, blk) if do_e else 0
    Ts = min(m.summary_candidates_per_block, blk) if do_s else 0
    assert Te > 0 and Ts > 0
    eta = m._eta_f32(DEV, BF16)
    ws = m._block_workspace(st, kmax)
    L = _hip.lib()
    d = m._bank_desc(st, eta, None, None)
    pos0 = int(st.pos)

    def chunk():
        _hip.check(L.coda_block_write(d, k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
                                      gate.data_ptr(), gate.stride(0), blk, 0, W, pos0, plan[0].data_ptr(), kmax,
                                      Te, Ts, ws.data_ptr(), ws.numel(), _hip.stream_of(k)))

    start = _snapshot(st)
    # eager: the chunk applied once, then once more on the result
    chunk()
    torch.cuda.synchronize()
    eager1 = _snapshot(st)
    chunk()
    torch.cuda.synchronize()
    eager2 = _snapshot(st)
    assert any(not torch.equal(eager1[f], eager2[f]) for f in eager1), "the second application changes nothing"
    # captured once, replayed three times from the start state, with eager
    # work and syncs between the replays
    _restore(st, start)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            chunk()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        _restore(st, start)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for f, want in eager1.items():
            assert torch.equal(getattr(st, f), want), f"replay {rep}: {f} differs from the eager chunk"
        graph.replay()
        torch.cuda.synchronize()
        for f, want in eager2.items():
            assert torch.equal(getattr(st, f), want), f"replay {rep} (applied twice): {f} differs from eager"
        # eager work between replays
        chunk()
        torch.cuda.synchronize()
    status = int(m._status_word(ws).item())
    assert status == 0, f"status word {status}: a wait gave up"


@torch.no_grad()
def test_forced_give_up_makes_the_layer_raise():
    _need_gpu()
    import ctypes
    from coda_gqa_l import _hip
    print("[forced give-up] B4 prefill with spin limit -1", flush=True)
    m, st, g = _layer_with_full_ring(4, seed=33)
    L = _hip.lib()
    n0 = ctypes.c_uint(0)
    _hip.check(L.coda_block_sync_timeouts(ctypes.byref(n0)))
    prev = L.coda_block_sync_spin_limit(-1)
    try:
        m.prefill_chunked(torch.randn(4, 128, 1024, generator=g, device=DEV, dtype=BF16), st, block_size=64,
                          return_outputs=False)
        torch.cuda.synchronize()
    finally:
        L.coda_block_sync_spin_limit(prev)
    n1 = ctypes.c_uint(0)
    _hip.check(L.coda_block_sync_timeouts(ctypes.byref(n1)))
    FORCED["n"] += n1.value - n0.value
    assert n1.value > n0.value, "no wait gave up with a spin limit of -1"
    with pytest.raises(RuntimeError, match="gave up waiting"):
        m.check_bank_status()
    # reported once; the layer then runs again (on a new state)
    m.check_bank_status()
    st = m.init_state(batch_size=4, device=DEV, dtype=BF16)
    m.prefill_chunked(torch.randn(4, 200, 1024, generator=g, device=DEV, dtype=BF16), st, block_size=64,
                      return_outputs=False)
    torch.cuda.synchronize()
    m.check_bank_status()
