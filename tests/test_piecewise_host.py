"""Host-side checks of the piecewise runner's orchestration (emberserve_amd.piecewise.SegmentGraphs), with
CPU tensors, where the pieces run eagerly instead of from graphs."""

from __future__ import annotations

import pytest
import torch

from emberserve_amd import ops
from emberserve_amd.eager import PAD_SLOT
from emberserve_amd.piecewise import DEFAULT_TOKEN_BUCKETS, SegmentGraphs, bucket_ladder, stage_rows


def test_bucket_ladder():
    assert DEFAULT_TOKEN_BUCKETS == (16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192)
    assert bucket_ladder(8192) == DEFAULT_TOKEN_BUCKETS
    assert bucket_ladder(1024, 256) == (16, 32, 64, 128, 256, 512, 768, 1024)
    assert bucket_ladder(5000) == (16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 5000)
    assert bucket_ladder(10) == (16,)
    assert bucket_ladder(1000, 300, smallest=64) == (64, 128, 256, 556, 856, 1156)
    with pytest.raises(ValueError):
        bucket_ladder(0)


def test_stage_rows_marks_padding():
    pos = torch.full((16,), 7, dtype=torch.int64)
    slots = torch.full((16,), 7, dtype=torch.int64)
    stage_rows(3, 8, pos, slots, torch.tensor([5, 6, 7]), torch.tensor([10, 11, 12]))
    assert pos.tolist() == [5, 6, 7, 0, 0, 0, 0, 0] + [7] * 8
    assert slots.tolist() == [10, 11, 12] + [PAD_SLOT] * 5 + [7] * 8
    with pytest.raises(ValueError):
        stage_rows(9, 8, pos, slots, torch.zeros(9, dtype=torch.int64), torch.zeros(9, dtype=torch.int64))


def test_segments_share_post_and_next_pre():
    """L layers give L + 1 segments: pre(0) | post(l-1) + pre(l) | post(L-1), with one
    attention call between consecutive segments, all at the step's bucket."""
    calls = []
    sg = SegmentGraphs(3, (64, 16), lambda i, t: calls.append(("pre", i, t)),
                       lambda i, t: calls.append(("post", i, t)), device="cpu")
    assert sg.buckets == (16, 64) and sg.num_segments == 4
    with pytest.raises(RuntimeError):
        sg.step(4, lambda i, n: None)
    sg.capture()
    assert sg.captured
    calls.clear()
    assert sg.step(5, lambda i, n: calls.append(("attend", i, n))) == 16
    assert calls == [("pre", 0, 16), ("attend", 0, 5), ("post", 0, 16), ("pre", 1, 16), ("attend", 1, 5),
                     ("post", 1, 16), ("pre", 2, 16), ("attend", 2, 5), ("post", 2, 16)]
    calls.clear()
    assert sg.step(64, lambda i, n: None) == 64
    assert {c[2] for c in calls} == {64}
    calls.clear()
    assert sg.step(65, lambda i, n: calls.append(("attend", i, n))) is None  # eager at n rows
    assert calls == [("pre", 0, 65), ("attend", 0, 65), ("post", 0, 65), ("pre", 1, 65), ("attend", 1, 65),
                     ("post", 1, 65), ("pre", 2, 65), ("attend", 2, 65), ("post", 2, 65)]
    assert sg.bucket(1) == 16 and sg.bucket(17) == 64 and sg.bucket(65) is None
    sg.release()
    assert not sg.captured


def test_step_stages_the_runner_rows():
    sg = SegmentGraphs(1, (8,), lambda i, t: None, lambda i, t: None, device="cpu")
    assert sg.rows.slots.tolist() == [PAD_SLOT] * 8  # nothing is written before a step is staged
    sg.capture()
    sg.step(3, lambda i, n: None, torch.tensor([4, 5, 6]), torch.tensor([1, 2, 3]))
    assert sg.rows.positions.tolist() == [4, 5, 6, 0, 0, 0, 0, 0]
    assert sg.rows.slots.tolist() == [1, 2, 3] + [PAD_SLOT] * 5
    with pytest.raises(ValueError):
        sg.step(3, lambda i, n: None, torch.tensor([4, 5, 6]))
    with pytest.raises(ValueError):
        SegmentGraphs(0, (8,), lambda i, t: None, lambda i, t: None, device="cpu")


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
