"""A numpy emulation of the summation order the gfx950 norm kernels use for rows of at most
64 packs of 8 elements (the `torch_order_sumsq` device helper): eight-wide vectors, four
interleaved accumulators that each add their vectors left to right, the four accumulators
added in order, then the eight lanes left to right. That is the order of PyTorch's CPU fp32
sum over a contiguous last dimension for such rows (aten/src/ATen/native/cpu/SumKernel.cpp,
`vectorized_inner_sum` -> `row_sum` -> `multi_row_sum`). `torch_order_holds()` checks the
claim on the running host, so a GPU test can require bit-exact normed values only where the
oracle's own sum really runs in that order.
"""

from __future__ import annotations

import functools

import numpy as np
import torch


def emulated_sumsq(rows: np.ndarray) -> np.ndarray:
    """Sum of squares of each row of a float32 [N, D] array (D a multiple of 32, D <= 512) in
    the kernels' order, every operation rounded to float32."""
    rows = np.asarray(rows, dtype=np.float32)
    n, d = rows.shape
    assert d % 32 == 0 and d <= 512, d
    sq = (rows * rows).astype(np.float32)
    vec = sq.reshape(n, d // 8, 8)
    acc = [vec[:, k].copy() for k in range(4)]
    for r in range(1, d // 32):
        for k in range(4):
            acc[k] = (acc[k] + vec[:, 4 * r + k]).astype(np.float32)
    p = acc[0]
    for k in range(1, 4):
        p = (p + acc[k]).astype(np.float32)
    tot = np.zeros(n, dtype=np.float32)
    for e in range(8):
        tot = (tot + p[:, e]).astype(np.float32)
    return tot


def pairwise_sumsq(rows: np.ndarray) -> np.ndarray:
    """A plausible other order (a butterfly over the row, as a wave reduction would do):
    used to show the checks can tell orders apart."""
    sq = (np.asarray(rows, dtype=np.float32) ** 2).astype(np.float32)
    while sq.shape[1] > 1:
        h = sq.shape[1] // 2
        sq = (sq[:, :h] + sq[:, h:]).astype(np.float32)
    return sq[:, 0]


@functools.lru_cache(maxsize=None)
def torch_order_holds(d: int = 128, rows: int = 4096, seed: int = 11) -> bool:
    """True when this host's torch sums fp32 rows of width d in the emulated order."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, d, generator=g).to(torch.bfloat16).float()
    want = x.pow(2).sum(-1).numpy()
    return bool((emulated_sumsq(x.numpy()) == want).all())
