"""The query pack and output unpack of a mixed prefill + decode attention step.

Reference: `PagedFlashAttentionBackend._prefill_kvcache` (emberserve/attn/paged_flash.py:
242-289) with its per-step `MixedPlan` (:99-150). In a step where some sequences attend with
query_len > 1 next to many single-query decode rows, every layer runs:

    q.index_select(0, dec_tokens)                       the decode rows, packed
    q.new_zeros((P, max_q, H, D)) + P slice copies       the prefill rows, left-padded
    out.index_copy_(0, dec_tokens, o)                   the decode outputs back
    out[start:start + n] = o_pad[i, max_q - n:]  (P x)  the prefill outputs back

(about 3 + 2P launches per layer: the fill, gather, index_copy and copy rows of the
reference's 7B mixed-step profile, results/tail/profile_mixed_39x300.txt). Here the same
data movement is two bit-exact kernels per layer, driven by one index tensor built once
per step: `ember_gather_rows` packs `[decode rows | P x max_q padded prefill rows]` (padding
written as zeros) and `ember_scatter_rows2` puts both attention outputs back.

`MixedRows` keeps the reference plan's row order: decode rows in batch order, then each
prefill sequence's rows left-padded to max_q (flash's bottom-right causal alignment:
padded slot r holds query `n - max_q + r`).
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch
from torch import Tensor

from . import _lib
from .ops import _check_indices, _launch, _raise_index_errors, _require_device

__all__ = ["MixedRows", "pack_queries", "unpack_outputs", "prefill_kvcache"]


def _index_tensor(values: Sequence[int], device: torch.device) -> Tensor:
    """int64 tensor on `device` without a stream synchronisation: built in pinned host
    memory and copied asynchronously (the reference's devutil.index_tensor contract)."""
    host = torch.tensor(list(values), dtype=torch.int64)
    if device.type != "cuda":
        return host.to(device)
    return host.pin_memory().to(device, non_blocking=True)


class MixedRows:
    """Row plan of one mixed step, shared by every layer (MixedPlan.build,
    paged_flash.py:127-150, restricted to the row bookkeeping).

    `query_lens[i]` is sequence i's query length this step (its packed rows are
    consecutive, in batch order). Sequences with query_len == 1 are decode rows; the
    others are prefill rows. `rows[t]` is the packed token held by slot t of the pack
    buffer, -1 for padding: slots [0, num_dec) are the decode rows, then prefill sequence
    p owns slots num_dec + p * max_q + [0, max_q)."""

    def __init__(self, query_lens: Sequence[int], device: torch.device | str) -> None:
        device = torch.device(device)
        dec: list[int] = []
        pre: list[tuple[int, int]] = []
        start = 0
        for n in query_lens:
            n = int(n)
            if n < 1:
                raise ValueError(f"emberserve_amd.mixed: query length {n} < 1")
            if n == 1:
                dec.append(start)
            else:
                pre.append((start, n))
            start += n
        self.num_tokens = start
        self.num_dec = len(dec)
        self.pre_rows = pre
        self.num_pre = len(pre)
        self.max_q = max((n for _, n in pre), default=0)
        slots = list(dec)
        for s, n in pre:
            slots += [-1] * (self.max_q - n) + list(range(s, s + n))
        self.num_slots = len(slots)
        self.rows = _index_tensor(slots, device)
        self.dec_tokens = self.rows[:self.num_dec]  # the reference plan's dec_tokens


def _row_view(t: Tensor, name: str) -> tuple[int, int]:
    """(rows, row stride) of a tensor whose trailing dims are one contiguous row per
    leading index (every dim but the first is packed)."""
    row = 1
    for d in range(t.dim() - 1, 0, -1):
        if t.shape[d] != 1 and t.stride(d) != row:
            raise ValueError(f"emberserve_amd.mixed: {name} must be contiguous inside a row "
                             f"(shape {tuple(t.shape)}, stride {t.stride()})")
        row *= t.shape[d]
    return t.shape[0], t.stride(0)


def pack_queries(q: Tensor, plan: MixedRows) -> tuple[Tensor | None, Tensor | None]:
    """q [T, H, D] (any token stride; heads and head_dim packed) -> (q_dec [num_dec, H, D],
    q_pad [P, max_q, H, D]), one launch. Equals q.index_select(0, dec_tokens) and the
    zero-padded copies of paged_flash.py:263-272 bit for bit. Either is None when that
    group is empty."""
    _require_device("emberserve_amd.mixed.pack_queries", q, plan.rows)
    if q.shape[0] != plan.num_tokens:
        raise ValueError(f"emberserve_amd.mixed: q has {q.shape[0]} tokens, the plan {plan.num_tokens}")
    n_rows, stride = _row_view(q, "q")
    row_elems = q[0].numel() if n_rows else 0
    buf = q.new_empty((plan.num_slots,) + tuple(q.shape[1:]))
    if plan.num_slots:
        _launch("ember_gather_rows", _lib.load().ember_gather_rows, q.device, q.data_ptr(), n_rows, stride,
                plan.rows.data_ptr(), plan.num_slots, buf.data_ptr(), buf.stride(0), row_elems, q.element_size())
        if _check_indices():
            _raise_index_errors()
    q_dec = buf[:plan.num_dec] if plan.num_dec else None
    q_pad = buf[plan.num_dec:].view((plan.num_pre, plan.max_q) + tuple(q.shape[1:])) if plan.num_pre else None
    return q_dec, q_pad


def unpack_outputs(out: Tensor, o_dec: Tensor | None, o_pad: Tensor | None, plan: MixedRows) -> Tensor:
    """Writes the decode outputs (o_dec [num_dec, ..., H, D]) and the padded prefill outputs
    (o_pad [P, max_q, H, D]) into out [T, H, D] in one launch: out.index_copy_(0,
    dec_tokens, o_dec) and out[start:start + n] = o_pad[p, max_q - n:] (paged_flash.py:267,
    276-277), bit for bit. Returns out."""
    _require_device("emberserve_amd.mixed.unpack_outputs", out, plan.rows,
                    *[t for t in (o_dec, o_pad) if t is not None])
    if out.shape[0] != plan.num_tokens:
        raise ValueError(f"emberserve_amd.mixed: out has {out.shape[0]} tokens, the plan {plan.num_tokens}")
    if (o_dec is None) != (plan.num_dec == 0) or (o_pad is None) != (plan.num_pre == 0):
        raise ValueError("emberserve_amd.mixed: o_dec / o_pad must be given exactly for the non-empty groups")
    n_out, out_stride = _row_view(out, "out")
    row_elems = out[0].numel()
    s0 = s1 = 0
    n0 = n1 = 0
    p0 = p1 = None
    if o_dec is not None:
        o = o_dec
        n0, s0 = _row_view(o, "o_dec")
        if n0 != plan.num_dec or o[0].numel() != row_elems or o.dtype != out.dtype:
            raise ValueError(f"emberserve_amd.mixed: o_dec shape {tuple(o_dec.shape)} does not match the plan")
        p0 = o.data_ptr()
    if o_pad is not None:
        if o_pad.shape[:2] != (plan.num_pre, plan.max_q) or o_pad.dtype != out.dtype:
            raise ValueError(f"emberserve_amd.mixed: o_pad shape {tuple(o_pad.shape)} does not match the plan")
        if o_pad.stride(0) != plan.max_q * o_pad.stride(1):
            raise ValueError("emberserve_amd.mixed: o_pad's first two dims must be packed")
        o = o_pad.reshape((plan.num_pre * plan.max_q,) + tuple(o_pad.shape[2:]))
        n1, s1 = _row_view(o, "o_pad")
        if o[0].numel() != row_elems:
            raise ValueError(f"emberserve_amd.mixed: o_pad row of {o[0].numel()} elements, out rows {row_elems}")
        p1 = o.data_ptr()
    _launch("ember_scatter_rows2", _lib.load().ember_scatter_rows2, out.device, p0, n0, s0, p1, n1, s1,
            plan.rows.data_ptr(), out.data_ptr(), n_out, out_stride, row_elems, out.element_size())
    if _check_indices():
        _raise_index_errors()
    return out


def prefill_kvcache(q: Tensor, plan: MixedRows,
                    decode_attn: Callable[[Tensor], Tensor] | None,
                    prefill_attn: Callable[[Tensor], Tensor] | None) -> Tensor:
    """The data movement of `_prefill_kvcache` (paged_flash.py:242-289) around the two
    attention calls, which the caller supplies: `decode_attn(q_dec [num_dec, 1, H, D])` and
    `prefill_attn(q_pad [P, max_q, H, D])` (flash_attn_with_kvcache with the plan's
    context lengths and block tables in the reference; `paged_attention_decode` serves the
    decode rows). Two pack/unpack launches replace the reference's 3 + 2P copies."""
    q_dec, q_pad = pack_queries(q, plan)
    out = q.new_empty(q.shape)
    o_dec = decode_attn(q_dec.view((plan.num_dec, 1) + tuple(q.shape[1:]))) if q_dec is not None else None
    o_pad = prefill_attn(q_pad) if q_pad is not None else None
    return unpack_outputs(out, o_dec, o_pad, plan)
