"""Host-side checks of the piecewise runner's orchestration (emberserve_amd.piecewise), with
CPU tensors, where the pieces run eagerly instead of from graphs."""

from __future__ import annotations

import pytest
import torch

from emberserve_amd import ops
from emberserve_amd.eager import PAD_SLOT
from emberserve_amd.piecewise import DEFAULT_TOKEN_BUCKETS, PiecewiseGraphs, stage_rows, token_buckets


def test_token_buckets():
    assert token_buckets(8192) == DEFAULT_TOKEN_BUCKETS
    assert token_buckets(1024, 256) == (16, 32, 64, 128, 256, 512, 768, 1024)


def test_stage_rows_marks_padding():
    pos = torch.full((16,), 7, dtype=torch.int64)
    slots = torch.full((16,), 7, dtype=torch.int64)
    stage_rows(3, 8, pos, slots, torch.tensor([5, 6, 7]), torch.tensor([10, 11, 12]))
    assert pos.tolist() == [5, 6, 7, 0, 0, 0, 0, 0] + [7] * 8
    assert slots.tolist() == [10, 11, 12] + [PAD_SLOT] * 5 + [7] * 8
    with pytest.raises(ValueError):
        stage_rows(9, 8, pos, slots, torch.zeros(9, dtype=torch.int64), torch.zeros(9, dtype=torch.int64))


def test_run_orders_pieces_and_picks_buckets():
    calls = []
    pw = PiecewiseGraphs(2, (16, 64), lambda i, t: calls.append(("pre", i, t)),
                         lambda i, t: calls.append(("post", i, t)), device="cpu")
    with pytest.raises(RuntimeError):
        pw.run(4, lambda i, n: None)
    pw.capture()
    calls.clear()
    assert pw.run(5, lambda i, n: calls.append(("attend", i, n))) == 16
    assert calls == [("pre", 0, 16), ("attend", 0, 5), ("post", 0, 16),
                     ("pre", 1, 16), ("attend", 1, 5), ("post", 1, 16)]
    calls.clear()
    assert pw.run(64, lambda i, n: None) == 64
    calls.clear()
    assert pw.run(65, lambda i, n: None) is None  # above the largest bucket: eager at n rows
    assert calls == [("pre", 0, 65), ("post", 0, 65), ("pre", 1, 65), ("post", 1, 65)]


def test_eager_cache_writes_skip_padding_slots():
    k = torch.randn(4, 2, 8)
    v = torch.randn(4, 2, 8)
    kc = torch.zeros(2, 4, 2, 8)
    vc = torch.zeros(2, 4, 2, 8)
    ops.kv_cache_write(k, v, torch.tensor([3, PAD_SLOT, 0, PAD_SLOT]), kc, vc)
    flat = kc.view(-1, 2, 8)
    assert torch.equal(flat[3], k[0]) and torch.equal(flat[0], k[2]) and not bool(flat[1:3].any())
    with pytest.raises(IndexError):
        ops.kv_cache_write(k, v, torch.tensor([3, -2, 0, 1]), kc, vc)
