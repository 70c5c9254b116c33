"""Parity of the HIP path with the CPU oracle at the benchmark's own shapes.

Head_dim 128 with the per-KV-head geometry of the 7B layer (G = 4, W256 /
Me64 / Ms64, Lbuf 384) and of the 70B layer (G = 8, W512 / Me128 / Ms128,
Lbuf 768), blocks of 256 and 128, and batches large enough that the bank
kernels run one workgroup per (sequence, KV head) (B * Hkv >= 512).

Free-running: the oracle and the HIP path each keep their own state through
a chunked prefill, a second ragged prefill call and then decode steps (the
HIP decode carries its routing record from step to step, as in the bench);
the states are compared after every call and every step.  Inputs are seeded
on the CPU at the post-projection boundary and copied to the device.
"""

from __future__ import annotations

import pytest
import torch

from parity_util import (assert_close, assert_heads, compare_states, compare_traces, fp32_attention, product_like,
                         to_product_state)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# name: (H, Hkv, Dh, W, Me, Ms, B, L, block, gates, decode steps, dtype)
SHAPES = {
    # configs[1] / configs[2] per-KV-head shape (7B: 32 / 8 heads -> G = 4)
    "c2_g4_b4_blk256": (8, 2, 128, 256, 64, 64, 4, 1536, 256, "random", 6, torch.bfloat16),
    "c2_g4_b4_blk128": (8, 2, 128, 256, 64, 64, 4, 1152, 128, "const", 6, torch.bfloat16),
    "c2_g4_b64_blk256": (8, 2, 128, 256, 64, 64, 64, 1024, 256, "random", 4, torch.bfloat16),
    "c2_g4_b4_f32": (8, 2, 128, 256, 64, 64, 4, 768, 256, "random", 4, torch.float32),
    # the 7B layer itself at the decode bench's batch: B * Hkv = 512, so the
    # routing and write-back kernels run one workgroup per (sequence, head)
    "c2_full_b64_blk256": (32, 8, 128, 256, 64, 64, 64, 640, 256, "const", 4, torch.bfloat16),
    # the 7B layer at configs[1]'s other decode batches (B = 1: 8 workgroups
    # for 256 CUs; B = 16: 128)
    "c1_full_b1_blk256": (32, 8, 128, 256, 64, 64, 1, 896, 256, "random", 8, torch.bfloat16),
    "c1_full_b16_blk256": (32, 8, 128, 256, 64, 64, 16, 640, 256, "random", 6, torch.bfloat16),
    # configs[2]'s layer at B = 4: the second call's first chunks run one by
    # one, 256 eight-wave attention workgroups (the 8-wave, four-stage kernel)
    "c2_full_b4_blk256": (32, 8, 128, 256, 64, 64, 4, 1024, 256, "random", 4, torch.bfloat16),
    # configs[4] per-KV-head shape (70B: 64 / 8 heads -> G = 8), large cache
    "c5_g8_b4_blk256": (16, 2, 128, 512, 128, 128, 4, 2048, 256, "random", 4, torch.bfloat16),
    "c5_full_b2_blk256": (64, 8, 128, 512, 128, 128, 2, 1280, 256, "const", 4, torch.bfloat16),
    # small rows, B * Hkv = 512 (one workgroup per (sequence, head) again)
    "tiny_b256": (4, 2, 32, 32, 16, 16, 256, 200, 48, "random", 6, torch.bfloat16),
}


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")


def _gates(kind, B, L, g):
    if kind == "const":
        # the layer's own gate at init: sigmoid(write_proj(x)) with zero
        # weights and bias -2, in bf16 -> one value for every token (all ties)
        v = torch.sigmoid(torch.tensor(-2.0, dtype=torch.bfloat16)).float()
        return v.expand(B, L).contiguous()
    return torch.sigmoid(torch.randn(B, L, generator=g) * 1.5 - 2.0)


def _inputs(m, B, L, dtype, kind, g):
    H, Hkv, Dh = m.num_heads, m.num_kv_heads, m.head_dim
    q = torch.randn(B, H, L, Dh, generator=g).to(dtype)
    k = torch.randn(B, Hkv, L, Dh, generator=g).to(dtype)
    v = torch.randn(B, Hkv, L, Dh, generator=g).to(dtype)
    lam = torch.sigmoid(torch.randn(B, H, L, 1, generator=g) - 1.0).to(dtype)
    return q, k, v, _gates(kind, B, L, g), lam


def _prefill_both(m, p, st_o, st_p, q, k, v, gate, lam, block, dtype, what):
    """One prefill call on each side; heads (against the oracle and against
    its attention evaluated in fp32 on a copy of the same state), slot
    decisions (every chunk's candidates, exact and summary routing) and the
    whole state compared."""
    import copy
    from coda_oracle import prims
    L = q.shape[2]
    c, s = m.rope_tables(L, st_o.pos, dtype)
    q_r = prims.rope(q, c, s, m.rope_interleaved)
    st_f = copy.deepcopy(st_o)
    with fp32_attention(m):
        heads_f = m.prefill_core(q_r, k, v, gate, lam, st_f, block_size=block)
    del st_f
    tr_o = []
    p.decision_trace = []
    heads_o = m.prefill_core(q_r, k, v, gate, lam, st_o, block_size=block, trace=tr_o)
    heads_p = p.prefill_core(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV), lam.squeeze(-1).to(DEV), c.to(DEV),
                             s.to(DEV), st_p, block_size=block)
    torch.cuda.synchronize()
    n = compare_traces(p.decision_trace, tr_o, m, f"{what} decisions")
    p.decision_trace = None
    assert_heads(heads_p.permute(0, 2, 1, 3), heads_o, heads_f, dtype, f"{what} heads")
    del heads_o, heads_p, heads_f
    compare_states(st_p, st_o, dtype, m.window, m.Me, what)
    return n


@pytest.mark.parametrize("name", list(SHAPES))
@torch.no_grad()
def test_bench_shape_trajectory_matches_oracle(name):
    _need_gpu()
    from coda_oracle import OracleLayer, banks
    H, Hkv, Dh, W, Me, Ms, B, L, block, kind, steps, dtype = SHAPES[name]
    print(f"[bench shape] {name}: H{H} Hkv{Hkv} Dh{Dh} W{W} Me{Me} Ms{Ms} B{B} L{L} block {block} "
          f"gates {kind} {dtype}", flush=True)
    kw = dict(embed_dim=H * Dh, num_heads=H, num_kv_heads=Hkv, window=W, num_landmarks_exact=Me,
              num_landmarks_summary=Ms, rope_base=1e4)
    torch.manual_seed(31)
    m = OracleLayer(**kw).to(dtype).eval()
    p = product_like(m, {"kw": kw}, dtype, DEV)
    torch.manual_seed(32)
    st_o = m.init_state(batch_size=B, dtype=dtype)
    st_p = to_product_state(st_o, DEV)
    g = torch.Generator().manual_seed(33)
    # ---- prefill: the whole sequence in one call, then a ragged second call
    q, k, v, gate, lam = _inputs(m, B, L, dtype, kind, g)
    _prefill_both(m, p, st_o, st_p, q, k, v, gate, lam, block, dtype, f"{name} prefill")
    L2 = block + block // 2 + 3
    q, k, v, gate, lam = _inputs(m, B, L2, dtype, kind, g)
    _prefill_both(m, p, st_o, st_p, q, k, v, gate, lam, block, dtype, f"{name} second prefill ({L2} tokens)")
    del q, k, v, gate, lam
    # ---- decode, free-running: the HIP side keeps its state (and routing
    # record) from step to step; even steps record their decisions (the
    # uncached launch path), odd steps run through the cached descriptors;
    # steps 1, 2 (mod 4) hand the kernel the raw k projection (it ropes k
    # itself), the others k roped as the oracle gets it
    from coda_oracle import prims
    for t in range(steps):
        traced = t % 2 == 0
        tr_o = [] if traced else None
        p.decision_trace = [] if traced else None
        qp = int(st_o.pos)
        qt = torch.randn(B, H, 1, Dh, generator=g).to(dtype)
        kn = torch.randn(B, Hkv, 1, Dh, generator=g).to(dtype)
        vn = torch.randn(B, Hkv, 1, Dh, generator=g).to(dtype)
        gn = _gates(kind, B, 1, g)
        lamt = torch.sigmoid(torch.randn(B, H, 1, 1, generator=g) - 1.0).to(dtype)
        ct, sn = m.rope_tables(1, qp, dtype)
        raw = t % 4 in (1, 2)
        banks.write_one(m, st_o, prims.rope(kn, ct, sn, m.rope_interleaved) if raw else kn, vn, gn, tr_o)
        ho = m.attend_core(qt, lamt, st_o, qp)
        with fp32_attention(m):
            hf = m.attend_core(qt, lamt, st_o, qp)
        hp = p.decode_step_core(qt.to(DEV), kn.to(DEV), vn.to(DEV), gn.reshape(B).to(DEV), lamt.squeeze(-1).to(DEV),
                                st_p, ct.to(DEV), sn.to(DEV), k_roped=not raw)
        torch.cuda.synchronize()
        if traced:
            compare_traces(p.decision_trace, tr_o, m, f"{name} decode step {t} decisions")
        p.decision_trace = None
        assert_heads(hp.permute(0, 2, 1, 3), ho, hf, dtype, f"{name} decode step {t} heads")
        compare_states(st_p, st_o, dtype, W, Me, f"{name} decode step {t}")


def _cpu_copy(st):
    from types import SimpleNamespace
    f = lambda t: None if t is None else t.detach().cpu()
    return SimpleNamespace(
        k_buf=f(st.k_buf), v_buf=f(st.v_buf), allowed=f(st.allowed), g_recent=f(st.g_recent),
        recent_idx=st.recent_idx, recent_filled=st.recent_filled, mem_last_exact=f(st.mem_last_exact), pos=st.pos,
        active_exact=st.active_exact, active_summary=st.active_summary, _exact_v_norm=f(st._exact_v_norm),
        _sum_lf_k_norm=f(st._sum_lf_k_norm))


@pytest.mark.parametrize("name", ["c2_g4_b4_blk256", "c2_g4_b4_f32", "c5_g8_b4_blk256", "tiny_b256"])
@torch.no_grad()
def test_one_launch_block_write_equals_four_launch_path(name, monkeypatch):
    """The one-launch chunk update (heads of a sequence meeting at a sync
    word) and the four-launch pipeline (route, decide, apply, ring) leave
    byte-identical states and decision traces after a chunked prefill; the
    heads agree within the tolerance (the one-launch path attends from bank
    snapshots in one launch per group of chunks)."""
    _need_gpu()
    from coda_oracle import OracleLayer
    H, Hkv, Dh, W, Me, Ms, B, L, block, kind, _, dtype = SHAPES[name]
    print(f"[one launch vs four] {name}: B{B} L{L} block {block} {dtype}", flush=True)
    kw = dict(embed_dim=H * Dh, num_heads=H, num_kv_heads=Hkv, window=W, num_landmarks_exact=Me,
              num_landmarks_summary=Ms, rope_base=1e4)
    torch.manual_seed(41)
    m = OracleLayer(**kw).to(dtype).eval()
    p = product_like(m, {"kw": kw}, dtype, DEV)
    st0 = m.init_state(batch_size=B, dtype=dtype)
    g = torch.Generator().manual_seed(42)
    q, k, v, gate, lam = _inputs(m, B, L, dtype, kind, g)
    c, s = m.rope_tables(L, 0, dtype)
    out = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("CODA_BLOCK_FUSED", mode)
        st = to_product_state(st0, DEV)
        p.decision_trace = []
        heads = p.prefill_core(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV), lam.squeeze(-1).to(DEV), c.to(DEV),
                               s.to(DEV), st, block_size=block)
        torch.cuda.synchronize()
        trace = [tuple(x.cpu() if torch.is_tensor(x) else x for x in ev) for ev in p.decision_trace]
        p.decision_trace = None
        out[mode] = (heads.cpu(), st, trace)
    h0, s0, t0 = out["0"]
    h1, s1, t1 = out["1"]
    # (the four-launch update has no bank snapshots, so its chunks attend
    # chunk by chunk to the live state: the same keys, other sum orders)
    assert_close(h0, h1, dtype, f"{name}: heads")
    assert len(t0) == len(t1), f"{name}: {len(t0)} vs {len(t1)} trace events"
    for i, (a, b) in enumerate(zip(t0, t1)):
        assert a[0] == b[0] and all(torch.equal(x, y) for x, y in zip(a[1:], b[1:])), f"{name}: trace event {i} differs"
    compare_states(s1, _cpu_copy(s0), dtype, W, Me, f"{name} one launch vs four")


def test_block_write_sync_never_gave_up():
    """No workgroup of the one-launch block write gave up its bounded wait
    for the other heads of its sequence in any run of this process (other
    than the give-ups test_block_sync_gpu forces on purpose)."""
    _need_gpu()
    import ctypes
    import sys
    from coda_gqa_l import _hip
    n = ctypes.c_uint(0)
    _hip.check(_hip.lib().coda_block_sync_timeouts(ctypes.byref(n)))
    mod = sys.modules.get("test_block_sync_gpu")
    forced = mod.FORCED["n"] if mod is not None else 0
    assert n.value == forced, f"{n.value - forced} workgroups gave up waiting at a block-write sync word"


@torch.no_grad()
def test_many_candidates_split_path_matches_oracle_and_is_batch_independent():
    """Every evicted token of a 256-block a candidate of both banks (Te = Ts
    = 256, past the one-launch kernel's 64) at the large cache (Me = Ms =
    128): the four-launch path, whose route and apply kernels take more
    workgroups per (sequence, head) where one's LDS would not fit.  B = 4
    against the oracle; at B = 64 (B * Hkv = 512, one route workgroup would
    need ~300 KB) the first four sequences equal the B = 4 run bit for bit."""
    _need_gpu()
    from coda_oracle import OracleLayer
    H, Hkv, Dh, W, Me, Ms, L, block, dtype = 16, 8, 128, 256, 128, 128, 768, 256, torch.bfloat16
    print(f"[many candidates] H{H} Hkv{Hkv} Me{Me} Ms{Ms} Te=Ts=256 L{L}", flush=True)
    kw = dict(embed_dim=H * Dh, num_heads=H, num_kv_heads=Hkv, window=W, num_landmarks_exact=Me,
              num_landmarks_summary=Ms, rope_base=1e4, exact_candidates_per_block=256,
              summary_candidates_per_block=256)
    torch.manual_seed(51)
    m = OracleLayer(**kw).to(dtype).eval()
    p = product_like(m, {"kw": kw}, dtype, DEV)
    torch.manual_seed(52)
    st_big = m.init_state(batch_size=64, dtype=dtype)
    g = torch.Generator().manual_seed(53)
    q, k, v, gate, lam = _inputs(m, 64, L, dtype, "random", g)
    # B = 4 against the oracle
    import dataclasses
    first4 = lambda st: dataclasses.replace(st, **{f.name: getattr(st, f.name)[:4].clone() for f in
                                                   dataclasses.fields(st) if torch.is_tensor(getattr(st, f.name))})
    st_o = first4(st_big)
    st_p4 = to_product_state(st_o, DEV)
    _prefill_both(m, p, st_o, st_p4, q[:4], k[:4], v[:4], gate[:4], lam[:4], block, dtype, "many candidates B4")
    # B = 64 and B = 4 on the device from the same initial state
    c, s = m.rope_tables(L, 0, dtype)
    st_p64 = to_product_state(st_big, DEV)
    h64 = p.prefill_core(q.to(DEV), k.to(DEV), v.to(DEV), gate.to(DEV), lam.squeeze(-1).to(DEV), c.to(DEV),
                         s.to(DEV), st_p64, block_size=block)
    st_p4b = to_product_state(first4(st_big), DEV)
    h4 = p.prefill_core(q[:4].to(DEV), k[:4].to(DEV), v[:4].to(DEV), gate[:4].to(DEV),
                        lam[:4].squeeze(-1).to(DEV), c.to(DEV), s.to(DEV), st_p4b, block_size=block)
    torch.cuda.synchronize()
    assert torch.equal(h64[:4].cpu(), h4.cpu()), "heads of sequences 0-3 depend on the batch"
    for f in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm"):
        a, b = getattr(st_p64, f), getattr(st_p4b, f)
        if a is None:
            continue
        assert torch.equal(a[:4].cpu(), b.cpu()), f"state field {f} of sequences 0-3 depends on the batch"


@pytest.mark.parametrize("Dh,inter", [(128, True), (128, False), (64, True), (64, False)])
@torch.no_grad()
def test_raw_k_decode_equals_roped_k(Dh, inter, monkeypatch):
    """The decode step handed the raw k projection (coda_decode_step_raw_k:
    the kernels rope it) leaves the same state bytes and head outputs as the
    step handed k roped by the RoPE kernel, from an empty ring through its
    filling (decode write kernel) into eviction, on the one-launch path and
    on the two-launch path (CODA_DECODE_FUSED=0), for both RoPE pairings."""
    _need_gpu()
    import coda_gqa_l
    H, Hkv, W, Me, Ms, B, n = 8, 2, 16, 8, 8, 3, 40
    print(f"[raw k] Dh{Dh} interleaved {inter}", flush=True)
    torch.manual_seed(61)
    p = coda_gqa_l.CoDAGQALandmarkPerf2(embed_dim=H * Dh, num_heads=H, num_kv_heads=Hkv, window=W,
                                        num_landmarks_exact=Me, num_landmarks_summary=Ms, rope_base=1e4,
                                        rope_interleaved=inter).to(DEV, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(62)
    seq = [(torch.randn(B, H, 1, Dh, generator=g), torch.randn(B, Hkv, 1, Dh, generator=g),
            torch.randn(B, Hkv, 1, Dh, generator=g), torch.sigmoid(torch.randn(B, generator=g) * 2),
            torch.sigmoid(torch.randn(B, H, 1, generator=g))) for _ in range(n)]
    runs = {}
    for fused in ("1", "0"):
        monkeypatch.setenv("CODA_DECODE_FUSED", fused)
        for raw in (False, True):
            torch.manual_seed(63)
            st = p.init_state(batch_size=B, device=DEV, dtype=torch.bfloat16)
            heads = []
            for q, k, v, gt, lam in seq:
                pos = int(st.pos)
                c, s_ = p.rope(seq_len=1, offset=pos, device=DEV, dtype=torch.bfloat16)
                c, s_ = c.contiguous(), s_.contiguous()
                kd = k.to(DEV, torch.bfloat16)
                if not raw:
                    kd = coda_gqa_l.apply_rope(kd, c, s_, interleaved=inter)
                h = p.decode_step_core(q.to(DEV, torch.bfloat16), kd, v.to(DEV, torch.bfloat16), gt.to(DEV),
                                       lam.to(DEV, torch.bfloat16), st, c, s_, k_roped=not raw)
                heads.append(h.cpu())
            torch.cuda.synchronize()
            runs[(fused, raw)] = (torch.stack(heads), _cpu_copy(st))
    for fused in ("1", "0"):
        h0, s0 = runs[(fused, False)]
        h1, s1 = runs[(fused, True)]
        assert torch.equal(h0, h1), f"fused={fused}: heads differ between raw and roped k"
        for f in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm"):
            assert torch.equal(getattr(s0, f), getattr(s1, f)), f"fused={fused}: state field {f} differs"


@pytest.mark.parametrize("G,Dh", [(2, 128), (4, 128), (8, 128), (4, 64)])
@torch.no_grad()
def test_decode_heads_do_not_depend_on_batch(G, Dh):
    """A batch of 32 (Hkv x B = 256 workgroups, one per CU) gives its first
    sequences exactly the head outputs and state bytes they get in a batch of
    4 from the same initial state, steps into eviction included: nothing in
    the step couples the sequences of a batch."""
    _need_gpu()
    import dataclasses
    from coda_oracle import OracleLayer
    Hkv, W, Me, Ms, n = 8, 16, 8, 8, 28
    H, Bbig, Bs = G * Hkv, 32, 4
    print(f"[batch independence] G{G} Dh{Dh}", flush=True)
    kw = dict(embed_dim=H * Dh, num_heads=H, num_kv_heads=Hkv, window=W, num_landmarks_exact=Me,
              num_landmarks_summary=Ms, rope_base=1e4, rope_interleaved=True)
    torch.manual_seed(71)
    m = OracleLayer(**kw).to(torch.bfloat16).eval()
    p = product_like(m, {"kw": kw}, torch.bfloat16, DEV)
    torch.manual_seed(72)
    st_big = m.init_state(batch_size=Bbig, dtype=torch.bfloat16)
    first = lambda st: dataclasses.replace(st, **{f.name: getattr(st, f.name)[:Bs].clone() for f in
                                                  dataclasses.fields(st) if torch.is_tensor(getattr(st, f.name))})
    g = torch.Generator().manual_seed(73)
    seq = [(torch.randn(Bbig, H, 1, Dh, generator=g), torch.randn(Bbig, Hkv, 1, Dh, generator=g),
            torch.randn(Bbig, Hkv, 1, Dh, generator=g), torch.sigmoid(torch.randn(Bbig, generator=g) * 2),
            torch.sigmoid(torch.randn(Bbig, H, 1, generator=g))) for _ in range(n)]
    runs = {}
    for B, st0 in ((Bbig, st_big), (Bs, first(st_big))):
        st = to_product_state(st0, DEV)
        heads = []
        for q, k, v, gt, lam in seq:
            pos = int(st.pos)
            c, s_ = p.rope(seq_len=1, offset=pos, device=DEV, dtype=torch.bfloat16)
            h = p.decode_step_core(q[:B].to(DEV, torch.bfloat16), k[:B].to(DEV, torch.bfloat16),
                                   v[:B].to(DEV, torch.bfloat16), gt[:B].to(DEV), lam[:B].to(DEV, torch.bfloat16),
                                   st, c.contiguous(), s_.contiguous(), k_roped=False)
            heads.append(h[:Bs].cpu())
        torch.cuda.synchronize()
        runs[B] = (torch.stack(heads), _cpu_copy(st))
    hb, sb = runs[Bbig]
    hs, ss = runs[Bs]
    assert torch.equal(hb, hs), f"G{G} Dh{Dh}: heads of sequences 0-3 depend on the batch"
    for f in ("k_buf", "v_buf", "allowed", "g_recent", "mem_last_exact", "_exact_v_norm", "_sum_lf_k_norm"):
        a, b = getattr(sb, f), getattr(ss, f)
        if a is None:
            continue
        assert torch.equal(a[:Bs], b), f"G{G} Dh{Dh}: state field {f} of sequences 0-3 depends on the batch"
