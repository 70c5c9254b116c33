"""The decode-shaped projection front end (coda_project: one MFMA GEMM over
the packed q / k / v / lambda / write-gate weights with the RoPE and sigmoid
epilogues, at most 64 token rows), against a torch float32 reference of the
same ops on the device and against the CPU oracle's project() + RoPE
(reference attention.py:396-410, 516-547), within the bf16 tolerance; the
layer's step() takes it, and the step's state and heads equal those of the
torch-projection path up to GEMM rounding."""

from __future__ import annotations

import pytest
import torch

from parity_util import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


# name: (D, H, Hkv, B, L, rope_interleaved, write_policy, qkv bias)
SHAPES = {
    "7b_decode_b64": (4096, 32, 8, 64, 1, True, "gated", False),
    "7b_decode_b1": (4096, 32, 8, 1, 1, True, "gated", False),
    "c1_decode_b3_half_split_bias": (512, 8, 2, 3, 1, False, "gated", True),
    "mha_no_gate_b5": (256, 4, 4, 5, 1, True, "none", False),
    "70b_decode_b8": (8192, 64, 8, 8, 1, True, "gated", False),
    "7b_two_tokens_b32": (4096, 32, 8, 32, 2, True, "gated", False),
}


def _layer(D, H, Hkv, inter, policy, bias):
    import coda_gqa_l
    torch.manual_seed(D + H + Hkv)
    m = coda_gqa_l.CoDAGQALandmarkPerf2(embed_dim=D, num_heads=H, num_kv_heads=Hkv, window=64, num_landmarks_exact=16,
                                        num_landmarks_summary=16, rope_interleaved=inter, write_policy=policy)
    with torch.no_grad():
        # non-trivial gate weights and biases (the layer inits them to zero)
        m.write_proj.weight.normal_(0, 0.05)
        m.lambda_proj.bias.uniform_(-1, 1)
        if bias:
            for lin in (m.q_proj, m.k_proj, m.v_proj):
                lin.bias = torch.nn.Parameter(torch.randn(lin.out_features) * 0.1)
    return m.to(DEV, torch.bfloat16).eval()


def _reference(m, x, p0):
    """float32 GEMMs on the device, then the eager ops' roundings."""
    from coda_gqa_l.primitives import apply_rope
    B, L, D = x.shape
    H, Hkv, Dh = m.num_heads, m.num_kv_heads, m.head_dim
    xf = x.float()

    def lin(l):
        y = xf @ l.weight.float().t()
        return (y + l.bias.float() if l.bias is not None else y).to(torch.bfloat16)

    q = lin(m.q_proj).view(B, L, H, Dh).permute(0, 2, 1, 3)
    k_raw = lin(m.k_proj).view(B, L, Hkv, Dh).permute(0, 2, 1, 3)
    v = lin(m.v_proj).view(B, L, Hkv, Dh).permute(0, 2, 1, 3)
    cos, sin = m.rope(seq_len=L, offset=p0, device=x.device, dtype=x.dtype)
    k = apply_rope(k_raw, cos, sin, interleaved=m.rope_interleaved)
    lam = torch.sigmoid(lin(m.lambda_proj)).permute(0, 2, 1)
    g = torch.sigmoid(lin(m.write_proj)).squeeze(-1).float() if m.write_policy != "none" else \
        torch.ones(B, L, device=x.device)
    return q, k, v, g, lam


@pytest.mark.parametrize("name", list(SHAPES))
@torch.no_grad()
def test_front_end_matches_float32_reference(name):
    _need_gpu()
    D, H, Hkv, B, L, inter, policy, bias = SHAPES[name]
    print(f"[proj] {name}: D{D} H{H} Hkv{Hkv} B{B} L{L} interleaved={inter} {policy} bias={bias}", flush=True)
    m = _layer(D, H, Hkv, inter, policy, bias)
    g_ = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(B, L, D, generator=g_, device=DEV, dtype=torch.bfloat16)
    p0 = 37
    got = m._front(x, p0, fused=True)
    ref = _reference(m, x, p0)
    torch.cuda.synchronize()
    for what, a, r in zip(("q", "k", "v", "g", "lam"), got[:5], ref):
        assert a.shape == r.shape, (what, a.shape, r.shape)
        assert_close(a, r, torch.bfloat16, f"{name} {what}")
        # fp32 accumulation in another order: the bf16 results are the
        # reference's in all but a few roundings
        same = (a.float() == r.float()).float().mean().item()
        assert same > 0.97, f"{name} {what}: only {same:.4f} of the elements equal the float32 reference's rounding"


@pytest.mark.parametrize("inter", [True, False])
@torch.no_grad()
def test_front_end_matches_oracle_project(inter):
    _need_gpu()
    from coda_oracle import OracleLayer, prims
    from parity_util import product_like
    kw = dict(embed_dim=512, num_heads=8, num_kv_heads=2, window=256, num_landmarks_exact=64, num_landmarks_summary=64,
              rope_interleaved=inter)
    torch.manual_seed(3)
    m = OracleLayer(**kw).to(torch.bfloat16).eval()
    with torch.no_grad():
        m.write_proj.weight.normal_(0, 0.05)
    p = product_like(m, {"kw": kw}, torch.bfloat16, DEV)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(6, 1, 512, generator=g).to(torch.bfloat16)
    q, k, v, gate, lam = m.project(x)
    got = p._front(x.to(DEV), 11, fused=True)
    # k roped with the product's own tables: a bf16 layer takes positions
    # and angles in bf16 (the buffer's dtype, as the reference), and torch's
    # device and CPU outer products round a few large angles differently
    k = prims.rope(k, got[5].cpu(), got[6].cpu(), inter)
    for what, a, r in zip(("q", "k", "v", "g", "lam"), got[:5], (q, k, v, gate, lam.squeeze(-1))):
        assert_close(a, r, torch.bfloat16, f"oracle project {what}")


@torch.no_grad()
def test_cached_step_equals_general_step():
    """The layer's cached steady-state step (descriptors and buffers kept
    per state) and its general step give bit-identical outputs and states
    over 40 decode tokens at the 7B shape, including tokens after an
    in-place edit of the state (which must rebuild the cache)."""
    _need_gpu()
    import coda_gqa_l
    from coda_gqa_l.state_io import deep_copy_state
    print("[cached step] 7B shape B8: 40 steps cached vs general", flush=True)
    torch.manual_seed(7)
    m = coda_gqa_l.CoDAGQALandmarkPerf2(embed_dim=4096, num_heads=32, num_kv_heads=8, window=256,
                                        num_landmarks_exact=64, num_landmarks_summary=64,
                                        rope_base=1e4).to(DEV, torch.bfloat16).eval()
    g = torch.Generator(device=DEV).manual_seed(8)
    B = 8
    st_a = m.init_state(batch_size=B, device=DEV, dtype=torch.bfloat16)
    m.prefill_chunked(torch.randn(B, 600, 4096, generator=g, device=DEV, dtype=torch.bfloat16), st_a,
                      block_size=256, return_outputs=False)
    st_b = deep_copy_state(st_a)
    xs = torch.randn(40, B, 1, 4096, generator=g, device=DEV, dtype=torch.bfloat16)
    ya, yb = [], []
    for t in range(40):
        if t == 20:
            st_a.v_buf[:, :, 300].mul_(0.5)  # an in-place edit through torch
        ya.append(m.step(xs[t], st_a)[0])
        assert m.__dict__.get("_fast") is not None, "the cached path did not run"
    fast = m._step_fast
    m._step_fast = lambda *args: None
    try:
        for t in range(40):
            if t == 20:
                st_b.v_buf[:, :, 300].mul_(0.5)
            yb.append(m.step(xs[t], st_b)[0])
    finally:
        m._step_fast = fast
    torch.cuda.synchronize()
    for t in range(40):
        assert torch.equal(ya[t], yb[t]), f"step {t}: outputs differ"
    for f in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm"):
        assert torch.equal(getattr(st_a, f), getattr(st_b, f)), f"state field {f} differs"
    assert (st_a.pos, st_a.recent_idx) == (st_b.pos, st_b.recent_idx)


@pytest.mark.parametrize("name", ["7b_decode_b64", "7b_decode_b1", "c1_decode_b3_half_split_bias", "70b_decode_b8"])
@torch.no_grad()
def test_tiled_weights_equal_row_major(name):
    """coda_project_pack's fragment tiles hold the packed weights in the
    documented order (untiled with torch they equal the row-major packing,
    k rows paired for half-split RoPE), and coda_project over the tiles
    equals coda_project over the row-major copy bit for bit (same products,
    same summation order)."""
    _need_gpu()
    D, H, Hkv, B, L, inter, policy, bias = SHAPES[name]
    print(f"[proj tiles] {name}: D{D} B{B}", flush=True)
    m = _layer(D, H, Hkv, inter, policy, bias)
    wt, b, layout = m._proj_pack(torch.bfloat16)
    assert layout == 1, "the row kernel's D must take the tiled weights"
    Dh = D // H
    wk = m.k_proj.weight
    if not inter:
        half = Dh // 2
        pair = torch.stack([torch.arange(half), torch.arange(half) + half], 1).reshape(-1)
        wk = wk[(torch.arange(Hkv)[:, None] * Dh + pair[None]).reshape(-1).to(DEV)]
    rows = [m.q_proj.weight, wk, m.v_proj.weight, m.lambda_proj.weight]
    if policy != "none":
        rows.append(m.write_proj.weight)
    w_rm = torch.cat([r.detach() for r in rows]).to(torch.bfloat16).contiguous()
    n_feat = w_rm.shape[0]
    nf64 = wt.shape[0]
    assert nf64 % 64 == 0 and nf64 >= n_feat
    # tile (fb, ks): element 8 (r + 16 q) + e holds W[16 fb + r][32 ks + 8 q + e]
    untiled = wt.view(nf64 // 16, D // 32, 4, 16, 8).permute(0, 3, 1, 2, 4).reshape(nf64, D)
    assert torch.equal(untiled[:n_feat], w_rm), "tiles differ from the row-major packing"
    assert not untiled[n_feat:].any(), "padding rows are not zero"
    g_ = torch.Generator(device=DEV).manual_seed(2)
    x = torch.randn(B, L, D, generator=g_, device=DEV, dtype=torch.bfloat16)
    got_t = [t.clone() for t in m._front(x, 5, fused=True)[:5]]
    cache = m.__dict__["_derived_cache"]
    tag, _ = cache[("proj", torch.bfloat16)]
    cache[("proj", torch.bfloat16)] = (tag, (w_rm, b, 0))
    try:
        got_r = m._front(x, 5, fused=True)[:5]
    finally:
        del cache[("proj", torch.bfloat16)]
    torch.cuda.synchronize()
    for what, a, r in zip(("q", "k", "v", "g", "lam"), got_t, got_r):
        assert torch.equal(a, r), f"{name} {what}: tiled and row-major weights give different results"
