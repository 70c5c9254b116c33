"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, its ctypes mirrors match the C struct layout, argument
validation fails cleanly before any HIP call, the selection order equals
torch's CPU topk, and the product refuses host tensors (no host path)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "coda_mi355x.h")


def _hip():
    from coda_gqa_l import _hip
    return _hip


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(coda_\w+|diff_\w+_forward_\w+)\s*\(", src,
                                 flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    L = _hip().lib()
    names = _declared_functions()
    assert len(names) >= 15, names
    typed = ["diff_%s_forward_%s" % (k, t) for k in ("epilogue", "sub_only") for t in ("bf16", "fp16", "fp32")]
    assert set(typed) <= set(names), "the reference's typed epilogue symbols must be declared"
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert L.coda_abi_version() == 1
    assert set(names) <= set(_hip()._SIGS), "ctypes signatures missing for: %s" % (set(names) - set(_hip()._SIGS))


def test_library_is_built_from_the_sources_beside_it():
    from coda_gqa_l import _srchash
    H = _hip()
    want = _srchash.source_hash()
    assert want is not None and len(want) == 16
    assert H.lib().coda_source_hash().decode() == want


def test_loader_refuses_a_library_built_from_other_sources(monkeypatch):
    H = _hip()
    H.lib()
    monkeypatch.setattr(H, "_lib", None)
    monkeypatch.setattr(H, "source_hash", lambda: "0123456789abcdef")
    with pytest.raises(RuntimeError, match="built from other sources"):
        H.lib()
    monkeypatch.undo()
    assert H.lib() is not None


def _c_layout(struct, fields, tmp_path):
    prog = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){",
            f'printf("%zu\\n", sizeof({struct}));']
    for f in fields:
        prog.append(f'printf("%zu\\n", offsetof({struct}, {f}));')
    prog.append("return 0;}")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(prog))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-O0", str(c), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    return [int(v) for v in out]


@pytest.mark.parametrize("cls,cname", [("AttnDesc", "coda_attn_desc"), ("BankDesc", "coda_bank_desc"),
                                       ("ProjDesc", "coda_proj_desc")])
def test_ctypes_structs_match_c_layout(cls, cname, tmp_path):
    S = getattr(_hip(), cls)
    fields = [f for f, _ in S._fields_]
    got = [ctypes.sizeof(S)] + [getattr(S, f).offset for f in fields]
    assert got == _c_layout(cname, fields, tmp_path)


def test_validation_fails_before_any_hip_call():
    H = _hip()
    L = H.lib()
    d = H.AttnDesc()
    d.dtype = 7
    assert L.coda_diff_attn_fwd(d, None) == 1
    assert b"dtype" in L.coda_last_error()
    d.dtype = H.CODA_BF16
    d.B, d.H, d.Hkv, d.Lq, d.Dh = 1, 6, 4, 1, 64
    assert L.coda_diff_attn_fwd(d, None) == 1
    assert b"multiple" in L.coda_last_error()
    d.H, d.Dh = 8, 96
    assert L.coda_diff_attn_fwd(d, None) == 1
    assert b"head_dim" in L.coda_last_error()
    b = H.BankDesc()
    b.dtype, b.B, b.Hkv, b.Dh, b.W, b.Me, b.Ms, b.lf = H.CODA_F32, 1, 2, 64, 8, 4, 4, 16
    assert L.coda_decode_write(b, None, None, 0, 0, None, 0, 0, 0, None) == 1
    assert b"lf" in L.coda_last_error()
    b.lf = 32
    assert L.coda_decode_write(b, None, None, 0, 0, None, 0, 0, 0, None) == 1
    assert b"buffers" in L.coda_last_error()
    assert L.coda_block_plan(None, 0, 3, 8, None, 0, 1, 10, 4, 8, 64, 1, 1, None, 64, None) == 1
    assert L.coda_diff_epilogue_fwd(0, None, None, None, None, None, 4, 64, 1e-6, None) == 1
    assert L.coda_rope_fwd(1, None, 0, 0, 0, None, 0, 0, 0, None, None, 1, 1, 1, 63, 1, None) == 1


def test_noalloc_block_write_rejects_chunks_beyond_its_scratch():
    """coda_block_write_noalloc refuses, before any HIP call, a chunk whose
    scratch exceeds the library's per-GPU array (16 MiB), naming the limit."""
    H = _hip()
    L = H.lib()
    limit = L.coda_block_write_noalloc_max_bytes()
    assert limit == 16 << 20
    b = H.BankDesc()
    b.dtype, b.B, b.Hkv, b.Dh, b.W, b.Me, b.Ms, b.lf = H.CODA_BF16, 4096, 8, 128, 256, 64, 64, 64
    b.active_exact, b.active_summary = 64, 64
    fake = 256  # never dereferenced: the size check comes first
    b.k_buf = b.v_buf = b.allowed = b.g_recent = b.mem_last = b.exact_v_norm = b.sum_lf_k_norm = b.eta = fake
    rc = L.coda_block_write_noalloc(b, fake, fake, 0, 0, 0, fake, 0, 256, 0, 256, 0, fake, 64, 8, 64, None)
    assert rc == 1
    msg = L.coda_last_error()
    assert b"16777216" in msg and b"coda_block_write with a workspace" in msg, msg


def _topk_host(vals, k, largest, sorted_):
    L = _hip().lib()
    out = np.zeros(k, np.int64)
    if vals.dtype == torch.int64:
        a = np.ascontiguousarray(vals.numpy())
        rc = L.coda_topk_order_host_i64(a.ctypes.data, a.size, k, int(largest), int(sorted_), out.ctypes.data)
    else:
        a = np.ascontiguousarray(vals.numpy().astype(np.float32))
        rc = L.coda_topk_order_host(a.ctypes.data, a.size, k, int(largest), int(sorted_), out.ctypes.data)
    assert rc == 0
    return out


@pytest.mark.parametrize("seed", range(4))
def test_selection_order_equals_torch_cpu_topk(seed):
    """The device selection code, run on the host, reproduces torch.topk's
    CPU output order (nth_element / partial_sort / sort paths, ties)."""
    g = torch.Generator().manual_seed(seed)
    for trial in range(400):
        n = int(torch.randint(1, 300, (1,), generator=g))
        k = int(torch.randint(0, n + 1, (1,), generator=g))
        mode = trial % 5
        if mode == 0:
            v = torch.full((n,), 0.11920292)            # constant write gate at init
        elif mode == 1:
            v = torch.randint(0, 3, (n,), generator=g).float()
        elif mode == 2:
            v = torch.rand(n, generator=g)
        elif mode == 3:
            v = torch.randint(-4, 4, (n,), generator=g).to(torch.int64)
        else:
            v = torch.where(torch.rand(n, generator=g) < 0.5, torch.tensor(-(2 ** 62)),
                            torch.randint(0, 50, (n,), generator=g))
        largest, srt = bool(trial % 3), bool((trial // 3) % 2)
        ref = torch.topk(v, k, largest=largest, sorted=srt).indices.numpy()
        np.testing.assert_array_equal(_topk_host(v, k, largest, srt), ref, err_msg=f"n={n} k={k} mode={mode}")


def test_known_tie_orders():
    """Orders probed from torch on the reference's constant-gate evictions."""
    g = torch.full((256,), 0.11920292)
    assert list(_topk_host(g, 8, True, False)) == list(torch.topk(g, 8, sorted=False).indices)
    assert list(_topk_host(g, 64, True, False)[:4]) == [160, 191, 190, 189]
    rk = torch.full((64,), -(2 ** 62), dtype=torch.int64)
    assert list(_topk_host(rk, 8, False, True)) == [44, 41, 42, 43, 46, 47, 40, 45]


def test_product_has_no_host_path():
    import coda_gqa_l
    m = coda_gqa_l.CoDAGQALandmarkPerf2(embed_dim=64, num_heads=2, num_kv_heads=1, window=4,
                                        num_landmarks_exact=2, num_landmarks_summary=2)
    with pytest.raises(RuntimeError, match="HIP device"):
        m.init_state(batch_size=1, device="cpu", dtype=torch.float32)
    q = torch.zeros(1, 2, 1, 32)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        coda_gqa_l.diff_flash_attn(q, q, torch.zeros(1, 1, 4, 32), torch.zeros(1, 1, 4, 32), torch.zeros(1, 2, 1, 1))
    with pytest.raises(RuntimeError, match="HIP devices only"):
        coda_gqa_l.diff_epilogue(q, q, torch.zeros(1, 2, 1, 1), torch.ones(32))


def test_product_weights_equal_reference_init():
    """Seeded construction yields the reference's parameters (pinned by the
    golden weight checksums through the oracle)."""
    import coda_gqa_l
    from golden_util import build_oracle, checksum, load
    for name in ("tiny_f32", "tiny_llama", "c1_f32"):
        case, dtype, _ = build_oracle(name)
        torch.manual_seed(case["seed_model"])
        m = coda_gqa_l.CoDAGQALandmarkPerf2(**case["kw"]).to(dtype=dtype)
        ck = np.array([checksum(p) for _, p in sorted(m.state_dict().items())])
        np.testing.assert_array_equal(ck, load(name)["weights_ck"])


def _sizes_desc(Me, Ms, Dh=128, Hkv=8, B=0, dt=None):
    H = _hip()
    d = H.BankDesc()
    d.dtype = H.CODA_BF16 if dt is None else dt
    d.B, d.Hkv, d.Dh, d.W, d.Me, d.Ms, d.lf = B, Hkv, Dh, 256, Me, Ms, Dh // 2
    d.active_exact, d.active_summary = Me, Ms
    return d


@pytest.mark.parametrize("Me,Ms,Te,Ts,ok", [
    (64, 64, 8, 64, True),        # configs[1] / [2] (medium cache)
    (128, 128, 8, 64, True),      # configs[4] (large cache)
    (128, 128, 64, 64, True),
    (128, 128, 256, 256, True),   # every token of a 256-block a candidate (four-kernel path)
    (160, 160, 8, 64, True),
    (256, 256, 1, 1, False),      # one head's norm caches alone exceed a workgroup's LDS
    (1024, 0, 8, 0, False),
])
def test_block_write_check_bounds_the_bank_sizes(Me, Ms, Te, Ts, ok):
    H = _hip()
    rc = H.lib().coda_block_write_check(_sizes_desc(Me, Ms), Te, Ts)
    assert (rc == 0) == ok, H.lib().coda_last_error()
    if not ok:
        assert b"LDS" in H.lib().coda_last_error()


def test_layer_rejects_bank_sizes_beyond_the_kernels_at_construction():
    import coda_gqa_l
    kw = dict(embed_dim=1024, num_heads=8, num_kv_heads=2, window=64, num_landmarks_summary=8)
    coda_gqa_l.CoDAGQALandmarkPerf2(num_landmarks_exact=128, **kw)
    with pytest.raises(ValueError, match="LDS"):
        coda_gqa_l.CoDAGQALandmarkPerf2(num_landmarks_exact=512, **kw)
