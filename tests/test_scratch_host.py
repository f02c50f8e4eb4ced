"""Host-side checks of the split-K workspace cache (no GPU): one buffer per (shape, device,
stream), counters verified and re-zeroed when left non-zero, and the MLA decode error word
mapped to exceptions."""

from __future__ import annotations

import pytest
import torch

from emberserve_amd import _lib, _scratch, mla_decode


def test_two_streams_get_different_workspaces(monkeypatch):
    cache = _scratch.ScratchCache("t")
    stream = {"id": 1}
    monkeypatch.setattr(_scratch, "_stream_key", lambda device: stream["id"])
    dev = torch.device("cpu")
    a = cache.get((2, 4), lambda: 1024, dev)
    assert cache.get((2, 4), lambda: 1024, dev) is a  # same stream, same shape: reused
    stream["id"] = 2
    b = cache.get((2, 4), lambda: 1024, dev)
    assert b is not a and b.data_ptr() != a.data_ptr()
    assert len(cache) == 2
    assert not bool(a.any()) and not bool(b.any())  # zero-filled


def test_workspace_size_floor_and_invalid(monkeypatch):
    monkeypatch.setattr(_scratch, "_stream_key", lambda device: 0)
    cache = _scratch.ScratchCache("t", min_bytes=256)
    assert cache.get((1,), lambda: 16, torch.device("cpu")).numel() * 4 == 256
    with pytest.raises(ValueError):
        cache.get((2,), lambda: -1, torch.device("cpu"))


def test_verify_counters_rezeroes_and_raises():
    cache = _scratch.ScratchCache("t")
    buf = torch.zeros(64, dtype=torch.float32)
    cache.verify_counters(buf, 128, 192)  # all zero: passes
    buf.view(torch.int32)[40] = 3  # a counter left at 3 by an aborted launch
    buf[0] = 1.5  # partials outside the region are not counters
    with pytest.raises(RuntimeError, match="non-zero"):
        cache.verify_counters(buf, 128, 192)
    assert int(buf.view(torch.int32)[32:48].abs().sum()) == 0
    assert float(buf[0]) == 1.5
    cache.verify_counters(buf, 128, 192)


def test_mla_decode_error_word_mapping():
    mla_decode.raise_decode_errors(0)
    with pytest.raises(RuntimeError, match="handshake"):
        mla_decode.raise_decode_errors(_lib.ERR_SYNC)
    with pytest.raises(IndexError, match="block id"):
        mla_decode.raise_decode_errors(_lib.ERR_BLOCK_ID)
    with pytest.raises(IndexError, match="context length"):
        mla_decode.raise_decode_errors(_lib.ERR_DECODE_CTX | _lib.ERR_SYNC)


def test_round_up():
    assert _scratch.round_up(0, 16) == 0 and _scratch.round_up(17, 16) == 32 and _scratch.round_up(256, 256) == 256
