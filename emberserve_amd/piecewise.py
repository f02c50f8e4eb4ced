"""Piecewise hipGraph replay of the per-layer ops at padded token buckets: the role of
emberserve/attn/piecewise_graphs.py (PiecewiseGraphRunner) for this library's kernels.

A prefill or mixed step has a variable token count, so one graph per step shape is not
possible; attention also needs per-step metadata. The pieces around attention are
row-wise, so they can be captured once per token bucket T and replayed for any step of
n <= T tokens, with the n real rows at the front of static buffers and T - n padding rows
behind them (piecewise_graphs.py:12-15). Per layer l and bucket T:

    pre graph  [l, T]: pre(l, T)    e.g. add + RMSNorm, qk-norm + rope + paged KV write
    eager            : attend(l, n) attention on the n real rows, with the step's metadata
    post graph [l, T]: post(l, T)   e.g. add + RMSNorm, silu_and_mul

The padding rows compute on whatever the static buffers hold and nothing reads their
results. What they must not do is write shared state: the fused paged-cache writes get
slot -1 (PAD_SLOT) for every padding row, which the kernels skip (`stage_rows`), so the KV
cache changes only at the real rows' slots.

Every kernel of this library launches on the current stream with no host sync and no
memset, so the pieces capture as they are. All graphs of one runner share a memory pool
and one capture stream, and replay one after another on the caller's stream; the split-K
workspaces of the decode kernels are keyed by that capture stream.
"""

from __future__ import annotations

from typing import Callable

import torch

from .eager import PAD_SLOT

DEFAULT_TOKEN_BUCKETS = (16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192)


def token_buckets(max_tokens: int, step: int = 0) -> tuple[int, ...]:
    """Capture buckets, the reference's choice (piecewise_graphs.py:49-60): powers of two
    from 16 (`step` 0), or powers of two up to `step` and then every `step` tokens up to
    `max_tokens`."""
    if step <= 0:
        return DEFAULT_TOKEN_BUCKETS
    out = [b for b in DEFAULT_TOKEN_BUCKETS if b <= step]
    out += list(range(2 * step, max_tokens + 1, step))
    return tuple(out)


def stage_rows(n: int, bucket: int, positions: torch.Tensor, slots: torch.Tensor,
               step_positions: torch.Tensor, step_slots: torch.Tensor) -> None:
    """Writes a step's n positions and cache slots into the front of the static buffers
    and marks the padding rows [n, bucket) with slot PAD_SLOT (position 0), so that a
    replay at `bucket` stores nothing for them. Device-side copies and fills only."""
    if not 0 <= n <= bucket <= positions.shape[0]:
        raise ValueError(f"stage_rows: need 0 <= n ({n}) <= bucket ({bucket}) <= {positions.shape[0]}")
    positions[:n].copy_(step_positions)
    slots[:n].copy_(step_slots)
    if bucket > n:
        positions[n:bucket].zero_()
        slots[n:bucket].fill_(PAD_SLOT)


class _Eager:
    """A replayable that runs the piece directly (CPU tensors, where there is no graph)."""

    def __init__(self, fn: Callable[[], None]) -> None:
        self.fn = fn

    def replay(self) -> None:
        self.fn()


class PiecewiseGraphs:
    """Per-layer pre/post pieces captured at each token bucket.

    pre(layer, t) and post(layer, t) run one layer's pieces on rows [:t] of the caller's
    static buffers (allocated at the largest bucket). `capture()` warms every piece up on
    a side stream, then records one graph per (layer, bucket) and piece, largest bucket
    first. `run(n, attend)` replays the pieces of every layer at the smallest bucket >= n
    with attend(layer, n) launched eagerly in between; steps above the largest bucket run
    every piece eagerly at n rows."""

    def __init__(self, num_layers: int, buckets: tuple[int, ...], pre: Callable[[int, int], None],
                 post: Callable[[int, int], None], device: torch.device | str = "cuda",
                 max_tokens: int | None = None) -> None:
        if num_layers < 1:
            raise ValueError("PiecewiseGraphs: at least one layer")
        top = max(buckets) if max_tokens is None else max_tokens
        bs = sorted({b for b in buckets if 0 < b <= top} | ({max_tokens} if max_tokens else set()))
        if not bs:
            raise ValueError("PiecewiseGraphs: no bucket")
        self.num_layers = num_layers
        self.buckets: list[int] = bs
        self.max_bucket = bs[-1]
        self.pre, self.post = pre, post
        self.device = torch.device(device)
        self.graphs_pre: dict[tuple[int, int], object] = {}
        self.graphs_post: dict[tuple[int, int], object] = {}
        self._pool = None
        self._stream = None
        self._captured = False

    def _record(self, fn: Callable[[], None]):
        if self.device.type != "cuda":
            return _Eager(fn)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=self._pool, stream=self._stream):
            fn()
        return g

    @torch.inference_mode()
    def capture(self, warmup_iters: int = 1) -> None:
        if self.device.type == "cuda":
            self._pool = torch.cuda.graph_pool_handle()
            self._stream = torch.cuda.Stream(self.device)
            side = torch.cuda.Stream(self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                for t in reversed(self.buckets):
                    for _ in range(warmup_iters):
                        for i in range(self.num_layers):
                            self.pre(i, t)
                            self.post(i, t)
            torch.cuda.current_stream(self.device).wait_stream(side)
            torch.cuda.synchronize(self.device)
        for t in reversed(self.buckets):
            for i in range(self.num_layers):
                self.graphs_pre[i, t] = self._record(lambda i=i, t=t: self.pre(i, t))
                self.graphs_post[i, t] = self._record(lambda i=i, t=t: self.post(i, t))
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        self._captured = True

    def bucket_for(self, n: int) -> int | None:
        for b in self.buckets:
            if b >= n:
                return b
        return None

    def run(self, n: int, attend: Callable[[int, int], None]) -> int | None:
        """One step of n tokens over every layer; returns the bucket replayed (None: ran
        eagerly at n rows). The caller has staged the step's rows (`stage_rows`)."""
        if not self._captured:
            raise RuntimeError("PiecewiseGraphs.run: call capture() first")
        t = self.bucket_for(n)
        for i in range(self.num_layers):
            if t is None:
                self.pre(i, n)
            else:
                self.graphs_pre[i, t].replay()
            attend(i, n)
            if t is None:
                self.post(i, n)
            else:
                self.graphs_post[i, t].replay()
        return t

    @torch.inference_mode()
    def release(self) -> None:
        for g in list(self.graphs_pre.values()) + list(self.graphs_post.values()):
            if hasattr(g, "reset"):
                g.reset()
        self.graphs_pre.clear()
        self.graphs_post.clear()
        self._captured = False

    def __repr__(self) -> str:
        return f"PiecewiseGraphs(buckets={self.buckets}, layers={self.num_layers}, captured={self._captured})"
