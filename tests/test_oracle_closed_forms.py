"""Pin the oracle's operator-level functions where the golden trajectories
do not reach them: closed forms, textbook routines and invariants.

  - diff_attention (the checker of the fused attention kernel) against a
    float64 brute-force softmax written with explicit loops, for plain,
    lower-right causal and GQA-shared inputs, with and without RMSNorm;
  - diff_epilogue / diff_sub_only against their float64 formulas;
  - RoPE against complex multiplication (interleaved) and against the
    rotate-half formula (half-split); the noise rotation at theta = pi/2;
  - HeadwiseRMSNorm: the output's RMS equals the weight (closed form);
  - OracleUnbounded against the golden-pinned OracleLayer with W >= L
    (no eviction: bounded == unbounded, the reference README's equivalence,
    README.md:263-269);
  - exact_route / summary_update (operator seams S3 / S4) against the
    golden-pinned block bank functions on identical inputs;
  - zero-initialised summary bank: every candidate routes to slot 0
    (first-occurrence argmax of all-zero scores).
Each check is chosen so that a plausible slip (dropped term, sign, index,
transposed operand) fails it; the planted-mistake tests at the end show
that for the attention checker.
"""

from __future__ import annotations

import math

import pytest
import torch

from coda_oracle import (OracleLayer, OracleState, OracleUnbounded, banks, diff_attention, diff_epilogue,
                         diff_sub_only, exact_route, lower_right_mask, prims, summary_update)


def _brute_attention(q, k, v, mask):
    """float64 softmax attention, one query row at a time."""
    B, H, Lq, Dh = q.shape
    Hkv = k.shape[1]
    g = H // Hkv
    out = torch.zeros(B, H, Lq, Dh, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            kk, vv = k[b, h // g].double(), v[b, h // g].double()
            for i in range(Lq):
                s = [float((q[b, h, i].double() * kk[j]).sum()) / math.sqrt(Dh)
                     if mask is None or mask[i, j] else -math.inf for j in range(kk.shape[0])]
                mx = max(s)
                if mx == -math.inf:
                    continue
                p = [math.exp(x - mx) for x in s]
                z = sum(p)
                for j, pj in enumerate(p):
                    out[b, h, i] += (pj / z) * vv[j]
    return out


def _brute_diff(q, qn, k, v, lam, w, mask, eps=1e-6):
    d = _brute_attention(q, k, v, mask) - lam.double() * _brute_attention(qn, k, v, mask)
    if w is None:
        return d
    rms = torch.sqrt((d * d).mean(dim=-1, keepdim=True) + eps)
    return d / rms * w.double()


@pytest.mark.parametrize("B,H,Hkv,Lq,Lk,Dh,causal,norm", [
    (1, 2, 2, 3, 5, 8, False, True),
    (2, 4, 2, 4, 7, 8, True, True),
    (1, 8, 2, 1, 9, 16, False, False),
    (1, 4, 1, 6, 6, 8, True, False),
])
def test_diff_attention_equals_brute_force(B, H, Hkv, Lq, Lk, Dh, causal, norm):
    g = torch.Generator().manual_seed(B * 100 + Lq * 10 + Lk)
    q, qn = torch.randn(B, H, Lq, Dh, generator=g), torch.randn(B, H, Lq, Dh, generator=g)
    k, v = torch.randn(B, Hkv, Lk, Dh, generator=g), torch.randn(B, Hkv, Lk, Dh, generator=g)
    lam = torch.rand(B, H, Lq, 1, generator=g)
    w = 1 + 0.2 * torch.randn(Dh, generator=g) if norm else None
    got = diff_attention(q, qn, k, v, lam, w, is_causal=causal)
    mask = lower_right_mask(Lq, Lk) if causal else None
    ref = _brute_diff(q, qn, k, v, lam, w, mask)
    assert torch.allclose(got.double(), ref, atol=2e-5, rtol=1e-5), (got.double() - ref).abs().max()


def test_lower_right_mask_alignment():
    """Query i of Lq sees keys [0, Lk - Lq + i] (the last query sees all)."""
    m = lower_right_mask(3, 5)
    assert m.tolist() == [[True, True, True, False, False], [True, True, True, True, False], [True] * 5]


def test_epilogue_formulas():
    g = torch.Generator().manual_seed(3)
    s, n = torch.randn(5, 16, generator=g), torch.randn(5, 16, generator=g)
    lam, w = torch.rand(5, 1, generator=g), torch.randn(16, generator=g)
    d = s.double() - lam.double() * n.double()
    ref = d / torch.sqrt((d * d).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert torch.allclose(diff_epilogue(s, n, lam, w).double(), ref, atol=1e-6)
    assert torch.allclose(diff_sub_only(s, n, lam).double(), d, atol=1e-6)


def test_rope_interleaved_is_complex_rotation():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 2, 7, 16, generator=g, dtype=torch.float64)
    inv = prims.rope_inv_freq(16, 10000.0).double()
    c, s = prims.rope_tables(inv, 7, 11, torch.float64)
    got = prims.rope(x, c, s, True)
    z = torch.complex(x[..., 0::2], x[..., 1::2])
    pos = torch.arange(11, 18, dtype=torch.float64).view(7, 1)
    rot = torch.polar(torch.ones(7, 8, dtype=torch.float64), pos * inv.view(1, 8))
    zr = z * rot
    ref = torch.stack([zr.real, zr.imag], dim=-1).flatten(-2)
    assert torch.allclose(got, ref, atol=1e-12)


def test_rope_half_split_is_rotate_half():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 1, 4, 8, generator=g, dtype=torch.float64)
    inv = prims.rope_inv_freq(8, 10000.0).double()
    c, s = prims.rope_tables(inv, 4, 0, torch.float64)
    got = prims.rope(x, c, s, False)
    half = 4
    for i in range(half):
        a, b = x[..., i], x[..., i + half]
        assert torch.allclose(got[..., i], a * c[:, i] - b * s[:, i], atol=1e-12)
        assert torch.allclose(got[..., i + half], b * c[:, i] + a * s[:, i], atol=1e-12)


def test_noise_rotation_at_half_pi_and_norm_preserved():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 3, 2, 8, generator=g, dtype=torch.float64)
    th = torch.full((3, 4), math.pi / 2, dtype=torch.float64)
    y = prims.noise_rotation(x, torch.cos(th), torch.sin(th))
    assert torch.allclose(y[..., 0::2], -x[..., 1::2], atol=1e-12)
    assert torch.allclose(y[..., 1::2], x[..., 0::2], atol=1e-12)
    th = torch.rand(3, 4, generator=g, dtype=torch.float64) * 6.28
    y = prims.noise_rotation(x, torch.cos(th), torch.sin(th))
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), atol=1e-12)


def test_head_rms_norm_output_rms_is_weight():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4, 32, generator=g, dtype=torch.float64) * 3
    w = torch.full((32,), 2.5, dtype=torch.float64)
    y = prims.head_rms_norm(x, w, 0.0)
    assert torch.allclose(y.pow(2).mean(-1).sqrt(), torch.full((4,), 2.5, dtype=torch.float64), atol=1e-12)


@torch.no_grad()
def test_unbounded_equals_bounded_without_eviction():
    """W >= L: the banks never receive a token and are masked, so the bounded
    layer's prefill equals plain causal differential attention."""
    kw = dict(embed_dim=128, num_heads=4, num_kv_heads=2)
    torch.manual_seed(21)
    bnd = OracleLayer(**kw, window=64, num_landmarks_exact=8, num_landmarks_summary=8).eval()
    unb = OracleUnbounded(**kw)
    sd = {k: v for k, v in bnd.state_dict().items() if k in unb.state_dict()}
    unb.load_state_dict(sd)
    x = torch.randn(2, 40, 128, generator=torch.Generator().manual_seed(22))
    st = bnd.init_state(batch_size=2, dtype=torch.float32)
    y_b, _ = bnd.prefill_chunked(x, st, block_size=40)
    y_u, _ = unb(x)
    assert (y_b - y_u).abs().max().item() < 1e-5


def _bank_layer(seed, **kw):
    torch.manual_seed(seed)
    m = OracleLayer(embed_dim=128, num_heads=4, num_kv_heads=2, window=16, num_landmarks_exact=8,
                    num_landmarks_summary=8, **kw).eval()
    st = m.init_state(batch_size=2, dtype=torch.float32)
    g = torch.Generator().manual_seed(seed + 1)
    m.prefill_chunked(torch.randn(2, 60, 128, generator=g), st, block_size=20, return_outputs=False)
    return m, st, g


def _clone(st):
    c = lambda t: None if t is None else t.clone()
    return OracleState(k_buf=c(st.k_buf), v_buf=c(st.v_buf), allowed=c(st.allowed), g_recent=c(st.g_recent),
                       recent_idx=st.recent_idx, recent_filled=st.recent_filled,
                       mem_last_exact=c(st.mem_last_exact), pos=st.pos, active_exact=st.active_exact,
                       active_summary=st.active_summary, _exact_v_norm=c(st._exact_v_norm),
                       _sum_lf_k_norm=c(st._sum_lf_k_norm))


@torch.no_grad()
def test_exact_route_seam_equals_block_function():
    m, st, g = _bank_layer(31)
    T, Dh, W, Me = 6, 32, m.window, m.Me
    k_sel, v_sel = torch.randn(2, 2, T, Dh, generator=g), torch.randn(2, 2, T, Dh, generator=g)
    # reuse two bank rows so hits and matches occur
    v_sel[:, :, 0] = st.v_buf[:, :, W + 1]
    pos_sel = torch.arange(T).repeat(2, 1) + 100
    gate = torch.tensor([[0.5, 0.05, 0.5, 0.5, 0.5, 0.5], [0.5] * T])
    used0, last0 = st.allowed[:, W:W + Me].clone(), st.mem_last_exact.clone()
    idx, ow, touch, last = exact_route(prims.unit(v_sel), st._exact_v_norm, used0, last0, gate, pos_sel,
                                       tau_gate=m.write_gate_threshold_exact, tau_match=m.exact_match_threshold,
                                       tau_novel=m.exact_novelty_threshold, active_exact=st.active_exact)
    s2 = _clone(st)
    trace = []
    banks.exact_block(m, s2, k_sel, v_sel, pos_sel, gate, trace=trace)
    _, idx_b, ow_b, touch_b = trace[-1][:4]
    assert torch.equal(idx, idx_b) and torch.equal(ow, ow_b) and torch.equal(touch, touch_b)
    assert torch.equal(last, s2.mem_last_exact)


@torch.no_grad()
def test_summary_update_seam_equals_block_function():
    m, st, g = _bank_layer(41)
    T, Dh, s0 = 10, 32, m.window + m.Me
    k_sel, v_sel = torch.randn(2, 2, T, Dh, generator=g), torch.randn(2, 2, T, Dh, generator=g)
    w_tok = torch.rand(2, T, generator=g)
    nk, nv, used, idx = summary_update(k_sel, v_sel, w_tok, st.k_buf[:, :, s0:].clone(),
                                       st.v_buf[:, :, s0:].clone(), st.allowed[:, s0:].clone(),
                                       st._sum_lf_k_norm, eta_logit=m.summary_eta_logit.detach(),
                                       energy_scale=m.energy_scale, lf_start=m.lf_start,
                                       overwrite_on_insert=m.summary_overwrite_on_insert,
                                       active_summary=st.active_summary)
    s2 = _clone(st)
    trace = []
    banks.summary_block(m, s2, k_sel, v_sel, None, w_tok, trace=trace)
    assert torch.equal(idx.long(), trace[-1][1])
    assert torch.equal(nk, s2.k_buf[:, :, s0:]) and torch.equal(nv, s2.v_buf[:, :, s0:])
    assert torch.equal(used, s2.allowed[:, s0:])


@torch.no_grad()
def test_zero_init_summary_routes_everything_to_slot_zero():
    torch.manual_seed(51)
    m = OracleLayer(embed_dim=128, num_heads=4, num_kv_heads=2, window=8, num_landmarks_exact=4,
                    num_landmarks_summary=4).eval()
    st = m.init_state(batch_size=1, dtype=torch.float32, mem_init="zeros")
    trace = []
    m.prefill_chunked(torch.randn(1, 24, 128, generator=torch.Generator().manual_seed(52)), st, block_size=24,
                      trace=trace)
    routes = [ev[1] for ev in trace if ev[0] == "summary_block"]
    assert routes and all(bool((r == 0).all()) for r in routes)


# ---------------------------------------------------------------- planted mistakes
def test_brute_force_catches_planted_mistakes():
    """The brute-force pin rejects a dropped lambda, a sign flip and a
    transposed GQA head mapping in the checker."""
    g = torch.Generator().manual_seed(61)
    q, qn = torch.randn(1, 4, 3, 8, generator=g), torch.randn(1, 4, 3, 8, generator=g)
    k, v = torch.randn(1, 2, 5, 8, generator=g), torch.randn(1, 2, 5, 8, generator=g)
    lam = torch.rand(1, 4, 3, 1, generator=g) + 0.2
    ref = _brute_diff(q, qn, k, v, lam, None, None)
    ok = diff_attention(q, qn, k, v, lam)
    assert torch.allclose(ok.double(), ref, atol=1e-5)
    no_lam = diff_attention(q, qn, k, v, torch.ones_like(lam))
    sign = diff_attention(q, qn, k, v, -lam)
    swapped = diff_attention(q, qn, k.flip(1), v.flip(1), lam)
    for bad in (no_lam, sign, swapped):
        assert not torch.allclose(bad.double(), ref, atol=1e-3)
