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


def _two_stream_fp32(self, q, q_noise, k, v, mask, lam, is_causal=False):
    """The oracle's two-stream attention and head norm (OracleLayer.two_stream)
    evaluated in fp32 on its bf16 operands, rounded once at the end: the fp32
    reference of the attention op over the same state."""
    import torch.nn.functional as F
    from coda_oracle.layer import expand_kv
    g = self.num_heads // self.num_kv_heads
    ke, ve = expand_kv(k, g).float(), expand_kv(v, g).float()
    o_s = F.scaled_dot_product_attention(q.float(), ke, ve, attn_mask=mask, is_causal=is_causal)
    o_n = F.scaled_dot_product_attention(q_noise.float(), ke, ve, attn_mask=mask, is_causal=is_causal)
    y = o_s - lam.float() * o_n
    if self.head_norm_mode == "full":
        y = y * torch.rsqrt(y.pow(2).mean(dim=-1, keepdim=True) + self.head_norm.eps) * self.head_norm.weight.float()
    return y.to(q.dtype)


class fp32_attention:
    """Within the block, `oracle.two_stream` runs in fp32 (the heads it returns
    feed no bank decision, so the state trajectory is unchanged)."""

    def __init__(self, oracle):
        self.m = oracle

    def __enter__(self):
        import types
        self.m.two_stream = types.MethodType(_two_stream_fp32, self.m)
        return self.m

    def __exit__(self, *exc):
        del self.m.two_stream
        return False


def assert_heads(hp, h_ref, h_f32, dtype, what):
    """Heads of the HIP path against (1) the oracle's attention evaluated in
    fp32 on the same state, within the dtype's tolerance, and (2) the oracle's
    own dtype path, within the tolerance plus that path's distance from (1):
    at the 7B shape the bf16 reference's per-op roundings (SDPA outputs,
    lambda * noise, the difference, the norm) put it up to ~2.2e-2 from its
    own fp32 evaluation, where the HIP path stays within ~1.1e-2 of it."""
    assert_close(hp, h_f32, dtype, f"{what} (vs the fp32 evaluation)")
    e_ref = max_rel(h_ref, h_f32)
    assert_close(hp, h_ref, dtype, f"{what} (vs the oracle; its own distance from fp32 {e_ref:.2e})",
                 tol=TOL[dtype] + e_ref)


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


def _diff_summary(a: torch.Tensor, b: torch.Tensor) -> str:
    a, b = a.float(), b.float()
    n = int((a != b).sum().item())
    return f"{n} of {b.numel()} elements differ, max abs diff {(a - b).abs().max().item():.3e}"


def compare_states(sp, so, dtype, W, Me, what):
    """Every state field byte-exact: ring, both banks, both norm caches,
    visibility bytes, LRU stamps, ring gates and the host ints."""
    assert torch.equal(sp.allowed.cpu(), so.allowed), f"{what}: allowed differs"
    assert torch.equal(sp.mem_last_exact.cpu(), so.mem_last_exact), f"{what}: LRU stamps differ"
    assert torch.equal(sp.g_recent.cpu(), so.g_recent), f"{what}: ring gates differ"
    ints_p = [sp.recent_idx, sp.recent_filled, sp.pos, sp.active_exact, sp.active_summary]
    ints_o = [so.recent_idx, so.recent_filled, so.pos, so.active_exact, so.active_summary]
    assert ints_p == ints_o, f"{what}: ring ints {ints_p} != {ints_o}"
    E = W + Me
    for f in ("k_buf", "v_buf"):
        a, b = getattr(sp, f).cpu(), getattr(so, f)
        for part, sl in (("ring", slice(0, W)), ("exact bank", slice(W, E)), ("summary bank", slice(E, None))):
            assert torch.equal(a[:, :, sl], b[:, :, sl]), f"{what}: {f} {part}: {_diff_summary(a[:, :, sl], b[:, :, sl])}"
    for f in ("_exact_v_norm", "_sum_lf_k_norm"):
        a, b = getattr(sp, f), getattr(so, f)
        if b is None:
            assert a is None
        else:
            a = a.cpu()
            assert torch.equal(a, b), f"{what}: {f}: {_diff_summary(a, b)}"


def _margin(tag, sc, where, m):
    """Oracle margin of the decision at `where` (tuple index into the
    decision tensor) from its masked score row."""
    row = sc[where].float()
    top = torch.topk(row, k=min(2, row.numel())).values
    gap = (top[0] - top[1]).item() if top.numel() > 1 else float("inf")
    msg = f"best {top[0].item():.6g}, gap to second {gap:.3e}"
    if tag.startswith("exact"):
        d = min(abs(top[0].item() - m.exact_novelty_threshold), abs(top[0].item() - m.exact_match_threshold))
        msg += f", distance to a cosine threshold {d:.3e}"
    return msg


def compare_traces(tp, to, m, what):
    """Decision events of the HIP path (layer.decision_trace) against the
    oracle's trace: same events in the same order, every decision field
    equal.  On a difference the message gives the oracle's margin there
    (score gap between the best two slots, distance to the thresholds)."""
    tags_p, tags_o = [e[0] for e in tp], [e[0] for e in to]
    assert tags_p == tags_o, f"{what}: decision events {tags_p[:8]}... != {tags_o[:8]}..."
    for i, (ep, eo) in enumerate(zip(tp, to)):
        tag = eo[0]
        for j in range(1, len(ep)):
            a, b = ep[j].cpu(), eo[j]
            if a.shape != b.shape or not torch.equal(a.to(b.dtype), b):
                msg = f"{what}: event {i} ({tag}) field {j} differs from the oracle"
                if a.shape == b.shape and tag != "select":
                    bad = (a.to(b.dtype) != b).nonzero()
                    where = tuple(bad[0].tolist())
                    msg += f" at {where} (HIP {a[where].item()}, oracle {b[where].item()}); oracle margin: " + \
                        _margin(tag, eo[-1], where, m)
                raise AssertionError(msg)
    return len(tp)
