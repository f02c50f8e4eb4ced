"""The order of the fp32 sum of squares that makes the gfx950 norm kernels bit-exact
against the oracle's rmsnorm (emberserve/model/ops.py:51-55: `xf.pow(2).mean(-1)` on the
CPU) for rows of at most 512 elements: the emulation in tests/sum_order.py against torch on
this host, the whole normalised row through it, and a check that a different order is
caught."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_ops as ref
from tests.sum_order import emulated_sumsq, pairwise_sumsq, torch_order_holds


@pytest.mark.parametrize("d", [32, 64, 128, 256, 512])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_emulated_order_is_torchs(d, dtype):
    g = torch.Generator().manual_seed(d)
    x = (torch.randn(3000, d, generator=g) * 3).to(dtype).float()
    want = x.pow(2).sum(-1).numpy()
    assert (emulated_sumsq(x.numpy()) == want).all()
    # mean = sum / d exactly (d a power of two here), as the kernels divide
    assert (x.pow(2).mean(-1).numpy() == (want / np.float32(d)).astype(np.float32)).all()


def test_other_order_is_caught():
    """The check discriminates: a butterfly order differs from torch's on many rows."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3000, 128, generator=g).to(torch.bfloat16).float()
    want = x.pow(2).sum(-1).numpy()
    assert (pairwise_sumsq(x.numpy()) != want).mean() > 0.2


@pytest.mark.parametrize("d", [64, 128, 512])
def test_rmsnorm_through_emulated_order_is_bitexact(d):
    """The whole normalised row (1/sqrt of the mean plus eps, two roundings, weight) built
    on the emulated sum equals the oracle's rmsnorm bit for bit."""
    g = torch.Generator().manual_seed(100 + d)
    x = torch.randn(4000, d, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    want = ref.rmsnorm(x, w, 1e-6)
    xf = x.float().numpy()
    var = (emulated_sumsq(xf) / np.float32(d)).astype(np.float32)
    inv = (np.float32(1) / np.sqrt((var + np.float32(1e-6)).astype(np.float32))).astype(np.float32)
    y = torch.from_numpy((xf * inv[:, None]).astype(np.float32)).to(torch.bfloat16)
    got = (y.float() * w.float()).to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_host_check():
    assert torch_order_holds(128)
