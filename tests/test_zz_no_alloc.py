"""coda_block_write_noalloc, the bank update of a prefill chunk that
allocates nothing (its scratch is a static per-GPU array of the library),
against coda_block_write with a caller workspace, through the C ABI: two
chunks in a row on the same GPU, the second with a smaller input (fewer
sequences, a shorter block), so the second call finds the first one's stale
scratch.  The bank state after each call must be byte-identical."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF16 = torch.bfloat16


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _clone_state(st):
    from coda_gqa_l import CoDAGQALandmarkStatePerf2
    c = lambda t: None if t is None else t.clone()
    return CoDAGQALandmarkStatePerf2(
        k_buf=c(st.k_buf), v_buf=c(st.v_buf), allowed=c(st.allowed), g_recent=c(st.g_recent),
        recent_idx=st.recent_idx, recent_filled=st.recent_filled, mem_last_exact=c(st.mem_last_exact),
        pos=st.pos, active_exact=st.active_exact, active_summary=st.active_summary,
        _exact_v_norm=c(st._exact_v_norm), _sum_lf_k_norm=c(st._sum_lf_k_norm))


def _one_chunk_both_ways(B, blk, seed):
    """A layer and a state with a full ring, then one chunk of `blk` new
    tokens written through both entry points into two copies of the state."""
    import coda_gqa_l
    from coda_gqa_l import _hip
    print(f"[no-alloc] B{B} block {blk} seed {seed}", flush=True)
    torch.manual_seed(seed)
    m = coda_gqa_l.CoDAGQALandmarkPerf2(embed_dim=1024, num_heads=8, num_kv_heads=2, window=64,
                                        num_landmarks_exact=32, num_landmarks_summary=32).to(BF16).to(DEV).eval()
    st = m.init_state(batch_size=B, device=DEV, dtype=BF16)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    with torch.no_grad():
        m.prefill_chunked(torch.randn(B, 200, 1024, generator=g, device=DEV, dtype=BF16), st, block_size=64,
                          return_outputs=False)
    Hkv, Dh, W = m.num_kv_heads, m.head_dim, m.window
    k = torch.randn(B, Hkv, blk, Dh, generator=g, device=DEV, dtype=BF16)
    v = torch.randn(B, Hkv, blk, Dh, generator=g, device=DEV, dtype=BF16)
    gate = torch.sigmoid(torch.randn(B, blk, generator=g, device=DEV) * 1.5 - 2.0).contiguous()
    assert st.recent_filled == W and st.recent_idx == 0
    plan, kmax, do_e, do_s = m._plan_candidates(st, gate, blk, blk)
    n_ev = blk
    Te = min(m.exact_candidates_per_block, n_ev) if do_e else 0
    Ts = min(m.summary_candidates_per_block, n_ev) if do_s else 0
    eta = m._eta_f32(DEV, BF16)
    L = _hip.lib()
    stream = _hip.stream_of(k)
    out = []
    for noalloc in (False, True):
        sx = _clone_state(st)
        d = m._bank_desc(sx, eta, None, None)
        args = (d, k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2), gate.data_ptr(),
                gate.stride(0), blk, 0, W, int(sx.pos), plan[0].data_ptr(), kmax, Te, Ts)
        if noalloc:
            _hip.check(L.coda_block_write_noalloc(*args, stream))
        else:
            ws = m._block_workspace(sx, kmax)
            _hip.check(L.coda_block_write(*args, ws.data_ptr(), ws.numel(), stream))
        torch.cuda.synchronize()
        out.append(sx)
    return out


def _assert_same(a, b, what):
    for f in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm"):
        x, y = getattr(a, f), getattr(b, f)
        assert torch.equal(x, y), f"{what}: {f} differs between coda_block_write and coda_block_write_noalloc"


@torch.no_grad()
def test_noalloc_block_write_equals_workspace_entry_point_twice_in_a_row():
    _need_gpu()
    from coda_gqa_l import _hip
    assert _hip.lib().coda_block_write_noalloc_max_bytes() == 16 << 20
    a, b = _one_chunk_both_ways(B=12, blk=96, seed=3)
    _assert_same(a, b, "first call (B12, block 96)")
    a, b = _one_chunk_both_ways(B=3, blk=40, seed=4)
    _assert_same(a, b, "second call (B3, block 40)")
