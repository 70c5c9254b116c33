"""The two summation orders the bank kernels follow so that their norm caches
and routing dots equal torch's CPU results bit for bit, pinned against torch
itself on this host:

- F.normalize's last-dim 2-norm (x86 ATen kernel): eight fp32 accumulators,
  channel k to accumulator k % 8 with fused multiply-adds over the vector
  part (8 fp32 / 16 bf16 elements per vector), the accumulators added in
  order, then the tail's rounded squares one by one;
- bf16 matmul (oneDNN on AVX512-BF16 hosts without AMX, the VDPBF16PS
  accumulation): channel pairs in increasing order, the odd channel's exact
  product added first.

The first holds on every x86 host torch runs on here (CPU test).  The second
depends on the host's matrix unit: it is what the GPU box's CPU does (the
oracle there is the parity reference of the GPU tests), so that test runs
with them (marker gpu); on a host with AMX tiles the order differs and the
routing dots differ in about 1 of 10^5 roundings.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

F = torch.nn.functional


def _norm_rule(x: torch.Tensor) -> torch.Tensor:
    xf = x.float().numpy().astype(np.float64)
    N, n = xf.shape
    vw = 16 if x.dtype == torch.bfloat16 else 8
    nv = n - n % vw
    acc = np.zeros((N, 8), np.float32)
    for k in range(nv):
        acc[:, k % 8] = (acc[:, k % 8].astype(np.float64) + xf[:, k] ** 2).astype(np.float32)   # fused
    ss = acc[:, 0].copy()
    for j in range(1, 8):
        ss = (ss + acc[:, j]).astype(np.float32)
    for k in range(nv, n):
        sq = (xf[:, k].astype(np.float32) * xf[:, k].astype(np.float32)).astype(np.float32)        # rounded
        ss = (ss + sq).astype(np.float32)
    nrm = torch.from_numpy(np.sqrt(ss, dtype=np.float32)).to(x.dtype)
    den = torch.maximum(nrm, torch.tensor(1e-6, dtype=x.dtype)).float()
    return (x.float() / den.unsqueeze(-1)).to(x.dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [16, 20, 32, 64, 128])
def test_normalize_order_rule_equals_torch(dtype, n):
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(20000, n, generator=g) * torch.rand(20000, 1, generator=g) * 3).to(dtype)
    assert torch.equal(_norm_rule(x), F.normalize(x, dim=-1, eps=1e-6))


def test_normalize_rule_rejects_a_planted_order():
    """A 16-accumulator order (the AVX512 register width) is not torch's:
    the pin can tell the two apart."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2000, 64, generator=g)
    xf = x.numpy().astype(np.float64)
    acc = np.zeros((2000, 16), np.float32)
    for k in range(64):
        acc[:, k % 16] = (acc[:, k % 16].astype(np.float64) + xf[:, k] ** 2).astype(np.float32)
    ss = acc[:, 0].copy()
    for j in range(1, 16):
        ss = (ss + acc[:, j]).astype(np.float32)
    wrong = x / torch.from_numpy(np.sqrt(ss, dtype=np.float32)).clamp_min(1e-6).unsqueeze(-1)
    assert not torch.equal(wrong, F.normalize(x, dim=-1, eps=1e-6))


def _pair_dots(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a [N, T, D], b [N, M, D] bf16 -> a @ b^T with the pair rule, bf16."""
    a64, b64 = a.double(), b.double()
    N, T, D = a.shape
    M = b.shape[1]
    acc = torch.zeros(N, T, M, dtype=torch.float32)
    for k in range(0, D, 2):
        for kk in (k + 1, k):
            acc = (acc.double() + a64[:, :, kk:kk + 1] * b64[:, None, :, kk]).float()
    return acc.to(torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("D,T", [(128, 64), (128, 8), (128, 1), (64, 64), (64, 1), (32, 16)])
def test_bf16_matmul_pair_order_equals_torch_on_this_host(D, T):
    g = torch.Generator().manual_seed(D + T)
    a = F.normalize(torch.randn(128, T, D, generator=g), dim=-1, eps=1e-6).to(torch.bfloat16)
    b = F.normalize(torch.randn(128, 64, D, generator=g), dim=-1, eps=1e-6).to(torch.bfloat16)
    ref = torch.matmul(a, b.transpose(1, 2))
    got = _pair_dots(a, b)
    n_bad = int((got != ref).sum().item())
    assert n_bad == 0, f"{n_bad} of {ref.numel()} bf16 dots differ from torch's CPU matmul on this host"
