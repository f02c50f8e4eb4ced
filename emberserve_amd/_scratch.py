"""Workspace cache shared by the split-K kernels (paged decode, MLA decode, the fused
gate_up + silu kernels).

Each of those kernels keeps arrival counters at the end of its workspace: every launch
bumps them and the last arrival returns them to zero, so a buffer is zero-filled once and
then reused. Two launches that overlap on one buffer would interfere (a counter reset by
one launch can erase another's increment), so a buffer belongs to one stream: the cache
key holds the launch stream beside the shape and device. During torch.cuda.graph capture
the current stream is the capture stream, so graphs captured on one capture stream share
buffers and must be replayed one after another on a single stream; graphs that replay
concurrently need distinct capture streams.

With `EMBERSERVE_CHECK_INDICES=1` the caller verifies after each launch that the counter
region is back at zero (`verify_counters`). A non-zero counter (an aborted launch, or an
overlap the rule above forbids) would otherwise leave some rows unmerged on every later
call; the check re-zeroes the region with a fill kernel (never a memset, so it is safe
inside a captured graph) and raises.
"""

from __future__ import annotations

from typing import Callable

import torch
from torch import Tensor


def _stream_key(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


class ScratchCache:
    """Zero-filled workspaces keyed by (shape key, device, current stream)."""

    def __init__(self, what: str, min_bytes: int = 256) -> None:
        self.what = what
        self.min_bytes = min_bytes
        self._bufs: dict[tuple, Tensor] = {}

    def get(self, key: tuple, nbytes: Callable[[], int], device: torch.device) -> Tensor:
        full = (*key, str(device), _stream_key(device))
        buf = self._bufs.get(full)
        if buf is None:
            n = int(nbytes())
            if n < 0:
                raise ValueError(f"{self.what}: no workspace for {key}")
            buf = torch.zeros(max(n, self.min_bytes) // 4, dtype=torch.float32, device=device)
            self._bufs[full] = buf
        return buf

    def __len__(self) -> int:
        return len(self._bufs)

    def verify_counters(self, buf: Tensor, start_bytes: int, end_bytes: int) -> None:
        """Raises RuntimeError (after re-zeroing them) when the counters in
        [start_bytes, end_bytes) of `buf` are not all zero. Synchronises."""
        region = buf.view(torch.int32)[start_bytes // 4:end_bytes // 4]
        if bool(region.any()):
            region.zero_()
            raise RuntimeError(f"{self.what}: split-K arrival counters were left non-zero (an aborted "
                               "launch, or two overlapping launches on one workspace); re-zeroed")


def round_up(n: int, m: int) -> int:
    return (n + m - 1) // m * m
