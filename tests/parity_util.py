"""Shared helpers of the GPU parity tests: tolerance metric, oracle <-> product
state transfer, seeded oracle inputs at the post-projection boundary."""

from __future__ import annotations

import torch

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b| over the whole tensor (0 for an all-zero b)."""
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    if b.numel() == 0:
        return 0.0
    den = b.abs().max().item()
    err = (a - b).abs().max().item() if a.numel() else 0.0
    return err / den if den > 0 else err


def assert_close(a, b, dtype, what, tol=None):
    t = TOL[dtype] if tol is None else tol
    r = max_rel(a, b)
    assert r <= t, f"{what}: max rel err {r:.3e} > {t:.1e}"


def to_product_state(st, device):
    from coda_gqa_l import CoDAGQALandmarkStatePerf2
    mv = lambda t: None if t is None else t.clone().to(device)
    return CoDAGQALandmarkStatePerf2(
        k_buf=mv(st.k_buf), v_buf=mv(st.v_buf), allowed=mv(st.allowed), g_recent=mv(st.g_recent),
        recent_idx=st.recent_idx, recent_filled=st.recent_filled, mem_last_exact=mv(st.mem_last_exact),
        pos=st.pos, active_exact=st.active_exact, active_summary=st.active_summary,
        _exact_v_norm=mv(st._exact_v_norm), _sum_lf_k_norm=mv(st._sum_lf_k_norm),
        metrics=None if st.metrics is None else dict(st.metrics))


def product_like(oracle, case, dtype, device):
    """Product layer with the oracle's weights (same constructor kwargs)."""
    import coda_gqa_l
    m = coda_gqa_l.CoDAGQALandmarkPerf2(**case["kw"]).to(dtype=dtype)
    m.load_state_dict(oracle.state_dict())
    return m.to(device).eval()


def compare_states(sp, so, dtype, W, Me, what):
    """Ring and exact bank byte-exact, decisions exact, summary bank and norm
    caches to rounding (summary EMA uses sigmoid(eta), fp32 normalisation
    sums in a different order)."""
    so_k, so_v = so.k_buf, so.v_buf
    sp_k, sp_v = sp.k_buf.cpu(), sp.v_buf.cpu()
    assert torch.equal(sp.allowed.cpu(), so.allowed), f"{what}: allowed differs"
    assert torch.equal(sp.mem_last_exact.cpu(), so.mem_last_exact), f"{what}: LRU stamps differ"
    assert torch.equal(sp.g_recent.cpu(), so.g_recent), f"{what}: ring gates differ"
    ints_p = [sp.recent_idx, sp.recent_filled, sp.pos, sp.active_exact, sp.active_summary]
    ints_o = [so.recent_idx, so.recent_filled, so.pos, so.active_exact, so.active_summary]
    assert ints_p == ints_o, f"{what}: ring ints {ints_p} != {ints_o}"
    E = W + Me
    assert torch.equal(sp_k[:, :, :E], so_k[:, :, :E]), f"{what}: ring/exact K differ"
    assert torch.equal(sp_v[:, :, :E], so_v[:, :, :E]), f"{what}: ring/exact V differ"
    st = 1e-5 if dtype == torch.float32 else 8e-3
    assert_close(sp_k[:, :, E:], so_k[:, :, E:], dtype, f"{what}: summary K", st)
    assert_close(sp_v[:, :, E:], so_v[:, :, E:], dtype, f"{what}: summary V", st)
    for f in ("_exact_v_norm", "_sum_lf_k_norm"):
        a, b = getattr(sp, f), getattr(so, f)
        if b is None:
            assert a is None
        else:
            assert_close(a, b, dtype, f"{what}: {f}", st)
