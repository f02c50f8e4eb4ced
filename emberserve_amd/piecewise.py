"""Segment graphs: hipGraph replay of the row-wise ops between attention calls, at padded
token buckets (the role emberserve/attn/piecewise_graphs.py plays for the reference's
model: a prefill or mixed step of any token count replays captured launches for
everything except attention).

Design. A decoder stack of L layers, each `pre(l) -> attention(l) -> post(l)`, is cut at
the attention calls only, which gives L + 1 segments:

    segment 0      : pre(0)
    segment l      : post(l - 1), then pre(l)        (1 <= l < L)
    segment L      : post(L - 1)

Each segment is one graph per bucket T, so a step replays L + 1 graphs with L eager
attention calls between them (not 2 L graphs: the post of one layer and the pre of the
next have no attention between them, so they share a graph). The step's n real rows sit
at the front of static buffers sized for the largest bucket; rows [n, T) are padding and
their results are never read (the padded-bucket contract of piecewise_graphs.py:12-15).

Padding rows must not write shared state. The runner owns the step's per-row metadata
(positions and paged-cache slots, `StepRows`); staging a step fills the padding rows'
slots with PAD_SLOT (-1), which every cache-writing kernel of this library skips, so the
KV cache changes at the real rows' slots only.

Every kernel of this library launches on the current stream with no host sync and no
memset, so a segment captures as it is. All graphs share one memory pool and are captured
on one stream owned by the runner, largest bucket first (its allocations size the pool;
smaller buckets then reuse it).
"""

from __future__ import annotations

import bisect
from typing import Callable

import torch

from .eager import PAD_SLOT

Piece = Callable[[int, int], None]  # (layer, rows) -> None


def bucket_ladder(max_tokens: int, linear_step: int = 0, smallest: int = 16) -> tuple[int, ...]:
    """Token buckets for capture: doubling from `smallest`; with `linear_step` > 0 the
    doubling stops at `linear_step` and the ladder continues in steps of `linear_step`
    (finer buckets waste less padded compute at 7B sizes, at the price of more graphs).
    The ladder ends at the first bucket >= max_tokens."""
    if max_tokens < 1 or smallest < 1:
        raise ValueError("bucket_ladder: max_tokens and smallest must be positive")
    out = []
    b = smallest
    cap = linear_step if linear_step > 0 else max_tokens
    while True:
        out.append(b)
        if b >= max_tokens:
            return tuple(out)
        if b * 2 > cap:
            break
        b *= 2
    # linear part (linear_step > 0, or a max_tokens between two powers of two)
    step = linear_step if linear_step > 0 else max_tokens - b
    while b < max_tokens:
        b += step
        out.append(b)
    return tuple(out)


DEFAULT_TOKEN_BUCKETS = bucket_ladder(8192)


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


class StepRows:
    """The per-row metadata of a step, held by the runner at the largest bucket: int64
    `positions` and `slots`. The pieces read rows [:T] of them."""

    def __init__(self, rows: int, device: torch.device) -> None:
        self.positions = torch.zeros(rows, dtype=torch.int64, device=device)
        self.slots = torch.full((rows,), PAD_SLOT, dtype=torch.int64, device=device)

    def stage(self, n: int, bucket: int, positions: torch.Tensor, slots: torch.Tensor) -> None:
        stage_rows(n, bucket, self.positions, self.slots, positions, slots)


class SegmentGraphs:
    """Graphs of the L + 1 attention-free segments of an L-layer stack, per token bucket.

    `pre(l, t)` / `post(l, t)` run layer l's pieces on rows [:t] of the caller's static
    buffers (and of `rows.positions` / `rows.slots`). `capture()` records every segment at
    every bucket. `step(n, attend, positions, slots)` stages the step's metadata, then
    replays segment 0, attend(0, n), segment 1, ..., attend(L - 1, n), segment L at the
    smallest bucket >= n and returns that bucket; a step above the largest bucket runs the
    same sequence eagerly at n rows and returns None. On a CPU device the segments run
    eagerly (no graphs), which keeps the orchestration testable without a GPU."""

    def __init__(self, num_layers: int, buckets, pre: Piece, post: Piece,
                 device: torch.device | str = "cuda") -> None:
        if num_layers < 1:
            raise ValueError("SegmentGraphs: at least one layer")
        bs = sorted({int(b) for b in buckets if int(b) > 0})
        if not bs:
            raise ValueError("SegmentGraphs: no bucket")
        self.num_layers = num_layers
        self.buckets = tuple(bs)
        self.pre, self.post = pre, post
        self.device = torch.device(device)
        self.rows = StepRows(bs[-1], self.device)
        self._graphs: dict[int, list] = {}  # bucket -> one replayable per segment
        self._pool = None
        self._stream = None

    # --------------------------------------------------------------------- segments
    def _segment(self, s: int, t: int) -> None:
        if s > 0:
            self.post(s - 1, t)
        if s < self.num_layers:
            self.pre(s, t)

    @property
    def num_segments(self) -> int:
        return self.num_layers + 1

    @property
    def captured(self) -> bool:
        return bool(self._graphs)

    # --------------------------------------------------------------------- capture
    def capture(self, warmup: int = 1) -> None:
        """Records every (bucket, segment) graph, largest bucket first. Each bucket's
        segments run `warmup` times eagerly on the capture stream before they are
        recorded (first-call work such as library handle set-up stays out of the graph).
        Runs in the caller's grad mode: call it under `torch.inference_mode()` when the
        pieces need it (capturing inside inference mode makes torch's graph RNG state an
        inference tensor, which a later capture outside it cannot update)."""
        if self.device.type != "cuda":
            for t in self.buckets:
                self._graphs[t] = [(lambda s=s, t=t: self._segment(s, t)) for s in range(self.num_segments)]
            return
        self._pool = torch.cuda.graph_pool_handle()
        self._stream = torch.cuda.Stream(self.device)
        self._stream.wait_stream(torch.cuda.current_stream(self.device))
        for t in reversed(self.buckets):
            with torch.cuda.stream(self._stream):
                for _ in range(warmup):
                    for s in range(self.num_segments):
                        self._segment(s, t)
            self._stream.synchronize()
            seg_graphs = []
            for s in range(self.num_segments):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=self._pool, stream=self._stream):
                    self._segment(s, t)
                seg_graphs.append(g.replay)
            self._graphs[t] = seg_graphs
        torch.cuda.current_stream(self.device).wait_stream(self._stream)
        torch.cuda.synchronize(self.device)

    # --------------------------------------------------------------------- replay
    def bucket(self, n: int) -> int | None:
        """The smallest bucket holding n rows, or None above the largest."""
        i = bisect.bisect_left(self.buckets, n)
        return self.buckets[i] if i < len(self.buckets) else None

    def step(self, n: int, attend: Piece, positions: torch.Tensor | None = None,
             slots: torch.Tensor | None = None) -> int | None:
        """One step of n tokens through every layer. `positions` / `slots` (n entries each)
        are staged into `rows` first when given; otherwise the caller staged them."""
        if not self._graphs:
            raise RuntimeError("SegmentGraphs.step: call capture() first")
        t = self.bucket(n)
        if positions is not None or slots is not None:
            if positions is None or slots is None:
                raise ValueError("SegmentGraphs.step: pass positions and slots together")
            self.rows.stage(n, n if t is None else t, positions, slots)
        if t is None:
            for s in range(self.num_segments):
                self._segment(s, n)
                if s < self.num_layers:
                    attend(s, n)
            return None
        graphs = self._graphs[t]
        for s in range(self.num_segments):
            graphs[s]()
            if s < self.num_layers:
                attend(s, n)
        return t

    def release(self) -> None:
        """Drops every graph (and with them the pool's memory)."""
        self._graphs.clear()
        self._pool = None
        self._stream = None

    def __repr__(self) -> str:
        return (f"SegmentGraphs(layers={self.num_layers}, segments={self.num_segments}, "
                f"buckets={self.buckets}, captured={self.captured})")
