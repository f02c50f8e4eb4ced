"""The routed experts' gate_up projection with silu_and_mul as its epilogue: the first
grouped GEMM of fused_moe_forward plus the activation (emberserve/model/moe_triton.py:
332-345) as one launch of `ember_moe_gate_up_silu` (libember_ops.so), over the reference's
block-aligned expert layout (`moe_align`, moe_triton.py:215-254).

    x [N, H], topk_ids [N, k] -> moe_align -> (sorted_ids, block_expert, num_valid)
    moe_gate_up_silu(x, w_gate_up [E, 2I, H], sorted_ids, block_expert, num_valid, k)
        -> act [N * k, I],  act[t * k + c] = silu_and_mul(x[t] @ w_gate_up[topk_ids[t, c]].T)

with the linear layer's output rounded to the activation dtype before the activation, as
`_grouped_gemm` stores it. The down projection and the routed-weight sum stay the
caller's (moe_triton.py:341-345).

CPU tensors, or `EMBERSERVE_FUSED_OPS=0`, take an eager per-block form.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib, ops
from ._scratch import ScratchCache, round_up
from .ops import _check_indices, _launch, _require_device, fused_enabled
from .paged_decode import num_sms

BLOCK_M = 16  # assignments per block (moe_triton.py:38)
SUPPORTED_DTYPES = (torch.float16, torch.bfloat16)


def moe_align_torch(topk_ids: Tensor, num_experts: int, block_m: int = BLOCK_M) -> tuple[Tensor, Tensor, int]:
    """Eager form of the layout for CPU tensors: one pass per expert over the flat
    assignment list (nonzero gives each expert's ids in ascending order)."""
    flat = topk_ids.reshape(-1)
    num_valid = flat.numel()
    max_padded = -(-(num_valid + num_experts * (block_m - 1)) // block_m) * block_m
    sorted_ids = torch.full((max_padded,), num_valid, dtype=torch.int32, device=flat.device)
    block_expert = torch.full((max_padded // block_m,), num_experts, dtype=torch.int32, device=flat.device)
    at = 0
    for e in range(num_experts):
        mine = (flat == e).nonzero().view(-1)
        n = mine.numel()
        if n == 0:
            continue
        sorted_ids[at:at + n] = mine.to(torch.int32)
        nb = -(-n // block_m)
        block_expert[at // block_m:at // block_m + nb] = e
        at += nb * block_m
    return sorted_ids, block_expert, num_valid


def moe_align(topk_ids: Tensor, num_experts: int, block_m: int = BLOCK_M, *,
              grid: bool = True) -> tuple[Tensor, Tensor, int]:
    """The block-aligned expert layout of moe_triton.py:215-254 (the single-launch form of
    :97-160): `ember_moe_align` on the GPU, no host sync. Past 3072 assignments it runs as a
    count launch and a placement launch over up to 64 workgroups with a small count-table
    workspace (grid=False keeps the one-workgroup form, the same layout).
    Returns (sorted_ids [max_padded] int32, block_expert [max_blocks] int32, num_valid):
    assignments id = token * k + choice grouped by expert in ascending id order, each
    expert's run padded to a multiple of block_m with num_valid, and the expert of every
    block (num_experts past the last used block). CPU tensors take `moe_align_torch`."""
    flat = topk_ids.reshape(-1)
    if not flat.is_cuda:
        return moe_align_torch(topk_ids, num_experts, block_m)
    if flat.dtype not in (torch.int32, torch.int64):
        flat = flat.long()
    flat = flat.contiguous()
    num_valid = flat.numel()
    lib = _lib.load()
    max_padded = lib.ember_moe_align_padded_size(num_valid, num_experts, block_m)
    if max_padded < 0:
        raise ValueError(f"moe_align: bad sizes (num_valid {num_valid}, num_experts {num_experts}, "
                         f"block_m {block_m})")
    sorted_ids = torch.empty((max_padded,), dtype=torch.int32, device=flat.device)
    block_expert = torch.empty((max_padded // block_m,), dtype=torch.int32, device=flat.device)
    ws_bytes = lib.ember_moe_align_workspace_bytes(num_valid, num_experts) if grid else 0
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=flat.device) if ws_bytes > 0 else None
    _launch("ember_moe_align", lib.ember_moe_align, flat.device, flat.data_ptr(), flat.element_size(), num_valid,
            num_experts, block_m, sorted_ids.data_ptr(), max_padded, block_expert.data_ptr(), max_padded // block_m,
            None if ws is None else ws.data_ptr(), 0 if ws is None else ws_bytes)
    if _check_indices() and _lib.read_errors(clear=True) & _lib.ERR_EXPERT_ID:
        raise IndexError(f"emberserve_amd.moe_align: expert id outside [0, {num_experts})")
    return sorted_ids, block_expert, num_valid


def _busy(num_valid: int, num_experts: int, inter: int) -> int:
    """Workgroups over the blocks that can hold assignments (at most min(num_valid,
    num_experts) experts are used) and the 64-column slabs, for one k split."""
    return min(num_valid, num_experts) * max(1, inter // 64)


def moe_num_splits(num_valid: int, num_experts: int, hidden: int, inter: int, device: torch.device,
                   packed: bool = False) -> int:
    """k splits from shapes only (>= 2 k steps per split). Row kernel: 1 while the busy
    workgroups number under the CUs, else 2. Packed kernel: 1. Measured at Moonlight's
    geometry with the weights rotated past the Infinity Cache (µs at 1 / 2 / 4 splits;
    row | packed): 1 token 18.0 / 20.0 / 19.9 | 15.4 / 20.3 / 19.0;  2 tokens 37.3 / 32.5 /
    31.8 | 32.3 / 31.0 / 30.3;  3 tokens 43.0 / 41.1 / 41.4 | 34.7 / 35.6 / 37.9;  4 tokens
    52.2 / 48.0 / 52.3 | 40.1 / 44.6 / 47.5;  8 tokens 86.2 / 70.9 / 75.0 | 57.7 / 65.1 /
    68.3;  64 tokens 147.0 / 137.2 / 155.5 | 112.6 / 137.9 / 154.9."""
    steps = hidden // 64
    if packed or steps % 2 or steps // 2 < 2:
        return 1
    return 1 if _busy(num_valid, num_experts, inter) < num_sms(device) else 2


def moe_half_slabs(num_valid: int, num_experts: int, inter: int, device: torch.device) -> bool:
    """Packed weights, one split: two-wave half-slab workgroups while the four-wave ones
    (used blocks x slabs) number from one to 1.5 times the CUs. Measured at Moonlight's
    geometry (µs, four-wave / half-slab): 1 token 15.3 / 15.9, 2 tokens 32.3 / 28.8 (30.2 at
    the best split), 3 tokens 34.4 / 32.5, 4 tokens 40.1 / 41.3, 8 tokens 57.6 / 60.7."""
    busy, cus = _busy(num_valid, num_experts, inter), num_sms(device)
    return cus <= busy < 1.5 * cus


# fused_moe_gate_up over packed experts: the direct path (no alignment) up to this many
# tokens. Measured at Moonlight's geometry (µs, align + packed kernel | direct at the
# moe_direct_half_slabs choice): 1 token 20.3 | 15.5, 2: 26.5 | 21.8, 3: 39.8 | 31.4,
# 4: 42.3 | 43.1, 8: 74.1 | 65.8, 12: 94.9 | 86.7, 16: 98.8 | 107.5, 32: 115.8 | 120.8.
DIRECT_MAX_TOKENS = 12
# The direct kernel holds at most this many routing ids (4 per lane of one wave); larger
# routings (top_k > 21 at 12 tokens) take the aligned path.
DIRECT_MAX_ASSIGNMENTS = 256


def moe_direct_half_slabs(num_assignments: int, num_experts: int, inter: int, device: torch.device) -> bool:
    """The direct path's workgroup shape: two-wave half-slab workgroups while the four-wave
    ones over the experts that can be used (min(assignments, experts) x slabs) number from
    one to five times the CUs. Measured (µs, four-wave | half-slab): 1 token 15.5 | 16.1,
    2: 31.5 | 28.0 (21.9 | 21.8 on another routing), 3: 33.4 | 31.4, 4: 46.1 | 43.1, 8: 75.4 |
    65.8, 12: 86.7 | 89.5."""
    busy, cus = min(num_assignments, num_experts) * max(1, inter // 64), num_sms(device)
    return cus <= busy < 5 * cus


def _workspace_bytes(splits: int, num_valid: int, inter: int, num_blocks: int) -> int:
    return _lib.load().ember_moe_gate_up_silu_workspace_bytes(num_valid, inter, num_blocks, splits)


# Split partials and counters, zero-filled once per (splits, num_valid, inter, num_blocks,
# device, stream), so graph replays see captured addresses and two streams never share
# counters.
_SCRATCH = ScratchCache("moe_gate_up_silu")


def moe_gate_up_silu_torch(x: Tensor, w_gate_up: Tensor, sorted_ids: Tensor, block_expert: Tensor,
                           num_valid: int, top_k: int) -> Tensor:
    """Eager form: per used block, silu_and_mul(F.linear(rows, w_gate_up[e])), stored at
    the blocks' assignment rows."""
    inter = w_gate_up.shape[1] // 2
    act = torch.empty((num_valid, inter), dtype=x.dtype, device=x.device)
    ids = sorted_ids.view(-1, BLOCK_M).tolist()
    for b, e in enumerate(block_expert.tolist()):
        if e >= w_gate_up.shape[0]:
            continue
        rows = [i for i in ids[b] if i < num_valid]
        if rows:
            r = torch.tensor(rows, dtype=torch.long, device=x.device)
            act[r] = ops.silu_and_mul(F.linear(x[r // top_k], w_gate_up[e]))
    return act


class PackedExperts:
    """The routed experts' gate_up weights [E, 2I, H] rearranged for
    `ember_moe_gate_up_silu_packed`: per expert, 16 KiB units of MFMA operand fragments in
    k-major order, so the workgroups of one expert read adjacent units. Made once per weight
    by `pack_moe_gate_up_weight`; the same bytes as the weight."""

    def __init__(self, packed: Tensor, num_experts: int, hidden: int, inter: int) -> None:
        self.packed, self.num_experts, self.hidden, self.inter = packed, num_experts, hidden, inter

    @property
    def dtype(self) -> torch.dtype:
        return self.packed.dtype

    @property
    def device(self) -> torch.device:
        return self.packed.device


def pack_moe_gate_up_weight(w_gate_up: Tensor) -> PackedExperts:
    """The packed copy of w_gate_up [E, 2I, H] (fp16/bf16 on the GPU, H and I multiples of 64)."""
    if w_gate_up.dim() != 3 or w_gate_up.shape[1] % 2 or w_gate_up.dtype not in SUPPORTED_DTYPES:
        raise ValueError(f"pack_moe_gate_up_weight: an [E, 2I, H] fp16/bf16 weight expected, got "
                         f"{tuple(w_gate_up.shape)} {w_gate_up.dtype}")
    _require_device("pack_moe_gate_up_weight", w_gate_up)
    E, two_i, H = w_gate_up.shape
    if (H % 64 or (two_i // 2) % 64 or w_gate_up.stride(2) != 1 or w_gate_up.stride(1) % 8
            or w_gate_up.stride(0) % 8 or w_gate_up.data_ptr() % 16):
        raise ValueError("pack_moe_gate_up_weight: H and I must be multiples of 64, rows unit-stride and 16-byte "
                         "aligned")
    packed = torch.empty(E * two_i * H, dtype=w_gate_up.dtype, device=w_gate_up.device)
    _launch("ember_moe_gate_up_silu_pack_weight", _lib.load().ember_moe_gate_up_silu_pack_weight, w_gate_up.device,
            w_gate_up.data_ptr(), w_gate_up.stride(0), w_gate_up.stride(1), _lib.dtype_tag(w_gate_up.dtype), E, H,
            two_i // 2, packed.data_ptr())
    return PackedExperts(packed, E, H, two_i // 2)


def moe_gate_up_silu(x: Tensor, w_gate_up: Tensor, sorted_ids: Tensor, block_expert: Tensor, num_valid: int,
                     top_k: int, *, num_splits: int | None = None, packed: PackedExperts | None = None,
                     half_slabs: bool | None = None) -> Tensor:
    """act [num_valid, I]: act[id] = silu_and_mul(x[id // top_k] @ w_gate_up[e].T) for every
    assignment id in a block of expert e (moe_triton.py:339-340, fused). With `packed`
    (`pack_moe_gate_up_weight(w_gate_up)`), the kernel reads the packed copy instead (the same
    bits); `half_slabs` (packed, one split; default `moe_half_slabs`) runs it over two-wave
    workgroups of 32 columns."""
    assert x.dim() == 2 and w_gate_up.dim() == 3 and w_gate_up.shape[2] == x.shape[1], (x.shape, w_gate_up.shape)
    assert w_gate_up.shape[1] % 2 == 0
    assert sorted_ids.dtype == torch.int32 and block_expert.dtype == torch.int32
    assert sorted_ids.numel() == block_expert.numel() * BLOCK_M, (sorted_ids.shape, block_expert.shape)
    if not fused_enabled(x):
        return moe_gate_up_silu_torch(x, w_gate_up, sorted_ids, block_expert, num_valid, top_k)
    _require_device("moe_gate_up_silu", x, w_gate_up, sorted_ids, block_expert)
    E, two_i, H = w_gate_up.shape
    inter = two_i // 2
    out = torch.empty((num_valid, inter), dtype=x.dtype, device=x.device)
    if num_valid == 0:
        return out
    fits = (x.dtype == w_gate_up.dtype and x.dtype in SUPPORTED_DTYPES and H % 64 == 0 and inter % 64 == 0
            and x.stride(1) == 1 and w_gate_up.stride(2) == 1 and x.stride(0) % 8 == 0
            and w_gate_up.stride(1) % 8 == 0 and w_gate_up.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0 and w_gate_up.data_ptr() % 16 == 0
            and sorted_ids.is_contiguous() and block_expert.is_contiguous())
    if not fits:
        return moe_gate_up_silu_torch(x, w_gate_up, sorted_ids, block_expert, num_valid, top_k)
    if packed is not None and (packed.num_experts, packed.hidden, packed.inter, packed.dtype,
                               packed.device) != (E, H, inter, x.dtype, x.device):
        raise ValueError("moe_gate_up_silu: the packed weight does not match x and w_gate_up")
    if num_splits is None:
        num_splits = moe_num_splits(num_valid, E, H, inter, x.device, packed=packed is not None)
    num_splits = int(num_splits)
    if num_splits not in (1, 2, 4) or (H // 64) % num_splits or H // 64 // num_splits < 2:
        raise ValueError(f"moe_gate_up_silu: num_splits {num_splits} must be 1, 2 or 4 and divide hidden / 64 "
                         f"= {H // 64} with >= 2 steps per split")
    nb = block_expert.numel()
    ws = None
    if num_splits > 1:
        ws = _SCRATCH.get((num_splits, num_valid, inter, nb), lambda: _workspace_bytes(num_splits, num_valid, inter, nb),
                          x.device)
    ws_ptr, ws_bytes = (ws.data_ptr(), ws.numel() * 4) if ws is not None else (None, 0)
    if packed is not None:
        if half_slabs is None:
            half_slabs = num_splits == 1 and moe_half_slabs(num_valid, E, inter, x.device)
        if half_slabs and num_splits != 1:
            raise ValueError("moe_gate_up_silu: half_slabs needs one k split")
        _launch("ember_moe_gate_up_silu_packed", _lib.load().ember_moe_gate_up_silu_packed, x.device,
                x.data_ptr(), x.stride(0), x.shape[0], packed.packed.data_ptr(), _lib.dtype_tag(x.dtype), E, H, inter,
                sorted_ids.data_ptr(), block_expert.data_ptr(), block_expert.numel(), num_valid, top_k, num_splits,
                int(bool(half_slabs)), ws_ptr, ws_bytes, out.data_ptr(), out.stride(0))
    else:
        _launch("ember_moe_gate_up_silu", _lib.load().ember_moe_gate_up_silu, x.device,
                x.data_ptr(), x.stride(0), x.shape[0], w_gate_up.data_ptr(), w_gate_up.stride(0), w_gate_up.stride(1),
                _lib.dtype_tag(x.dtype), E, H, inter, sorted_ids.data_ptr(), block_expert.data_ptr(),
                block_expert.numel(), num_valid, top_k, num_splits, ws_ptr, ws_bytes, out.data_ptr(), out.stride(0))
    if _check_indices():
        if ws is not None:
            need, cnt = _workspace_bytes(num_splits, num_valid, inter, nb), nb * (inter // 64)
            _SCRATCH.verify_counters(ws, need - round_up(cnt * 4, 256), need - round_up(cnt * 4, 256) + cnt * 4)
        if _lib.read_errors(clear=True) & _lib.ERR_ROW_INDEX:
            raise IndexError("emberserve_amd.moe_gate_up_silu: assignment id past the token rows")
    return out


GEMM_BLOCK_M = 256  # rows per block of the prefill GEMM's layout (its token tile)
# fused_moe_gate_up: the GEMM from GEMM_FROM assignments (128-row blocks below
# GEMM_WIDE_FROM, 256-row ones from there), the packed 16-block kernel up to
# PACKED_MAX_ASSIGNMENTS. Measured at Moonlight's geometry (bf16, µs, alignment included;
# row kernel at its default splits | GEMM 256 x 128 | GEMM 128 x 128): 1536 assignments
# 226 | 259 | 200, 3072: 291 | 292 | 204, 6144: 499 | 282 | 243, 12288: 840 | 341 | 294,
# 49152: 2722 | 688 | 736. The packed kernel: 384 assignments 115 against the row
# kernel's 136; 1536: 228 against 205.
GEMM_FROM = 1536
GEMM_WIDE_FROM = 24576
PACKED_MAX_ASSIGNMENTS = 768


def moe_gate_up_silu_gemm(x: Tensor, w_gate_up: Tensor | None, topk_ids: Tensor, *, column_tile: int = 128,
                          block_rows: int = GEMM_BLOCK_M, packed: PackedExperts | None = None) -> Tensor:
    """act [N * k, I] at prefill sizes (`ember_moe_gate_up_silu_gemm`): moe_align with
    block_rows-row blocks (256, or 128 with 128-column tiles), then the MFMA GEMM of
    `gate_up_silu_gemm` with one block per token tile over the block's gathered x
    rows and its expert's weight, silu_and_mul in the epilogue, rows scattered back to
    assignment order. The first grouped GEMM + silu_and_mul of moe_triton.py:339-340;
    bit-identical to `moe_gate_up_silu` for every assignment. With `packed`
    (`pack_moe_gate_up_weight`) the GEMM reads the packed experts
    (`ember_moe_gate_up_silu_gemm_packed`: contiguous 16 KiB units per stage, the same
    bits) and w_gate_up may be None."""
    assert x.dim() == 2 and topk_ids.dim() == 2, (x.shape, topk_ids.shape)
    if packed is not None:
        E, two_i, H = packed.num_experts, 2 * packed.inter, packed.hidden
        _require_device("moe_gate_up_silu_gemm", x, packed.packed, topk_ids)
        wdtype = packed.dtype
    else:
        assert w_gate_up is not None and w_gate_up.dim() == 3, "moe_gate_up_silu_gemm: w_gate_up or packed"
        _require_device("moe_gate_up_silu_gemm", x, w_gate_up, topk_ids)
        E, two_i, H = w_gate_up.shape
        wdtype = w_gate_up.dtype
    inter = two_i // 2
    n, k = topk_ids.shape
    if x.shape[1] != H or two_i % 2 or n > x.shape[0]:
        raise ValueError(f"moe_gate_up_silu_gemm: x {tuple(x.shape)}, weights [{E}, {two_i}, {H}] and "
                         f"topk_ids {tuple(topk_ids.shape)} do not match")
    if (block_rows, column_tile) not in ((256, 64), (256, 128), (128, 128)):
        raise ValueError(f"moe_gate_up_silu_gemm: no ({block_rows}, {column_tile}) tile")
    sorted_ids, block_expert, num_valid = moe_align(topk_ids, E, block_rows)
    out = torch.empty((num_valid, inter), dtype=x.dtype, device=x.device)
    if num_valid == 0:
        return out
    fits = (x.dtype == wdtype and x.dtype in SUPPORTED_DTYPES and H % 64 == 0
            and inter % column_tile == 0 and x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0)
    if packed is None:
        fits = fits and (w_gate_up.stride(2) == 1 and w_gate_up.stride(1) % 8 == 0 and w_gate_up.stride(0) % 8 == 0
                         and w_gate_up.data_ptr() % 16 == 0)
    if not fits:
        raise ValueError(f"moe_gate_up_silu_gemm: shape, dtype or alignment not supported (H {H}, I {inter}, "
                         f"column_tile {column_tile}, {x.dtype})")
    if packed is not None:
        _launch("ember_moe_gate_up_silu_gemm_packed", _lib.load().ember_moe_gate_up_silu_gemm_packed, x.device,
                x.data_ptr(), x.stride(0), x.shape[0], packed.packed.data_ptr(), _lib.dtype_tag(x.dtype), E, H, inter,
                sorted_ids.data_ptr(), block_expert.data_ptr(), block_expert.numel(), block_rows, num_valid, k,
                column_tile, out.data_ptr(), out.stride(0))
    else:
        _launch("ember_moe_gate_up_silu_gemm", _lib.load().ember_moe_gate_up_silu_gemm, x.device,
                x.data_ptr(), x.stride(0), x.shape[0], w_gate_up.data_ptr(), w_gate_up.stride(0), w_gate_up.stride(1),
                _lib.dtype_tag(x.dtype), E, H, inter, sorted_ids.data_ptr(), block_expert.data_ptr(),
                block_expert.numel(), block_rows, num_valid, k, column_tile, out.data_ptr(), out.stride(0))
    if _check_indices() and _lib.read_errors(clear=True) & _lib.ERR_ROW_INDEX:
        raise IndexError("emberserve_amd.moe_gate_up_silu_gemm: assignment id past the token rows")
    return out


def moe_gate_up_silu_direct(x: Tensor, topk_ids: Tensor, packed: PackedExperts, *,
                            half_slabs: bool = False) -> Tensor:
    """act [N * k, I] straight from the routing ids, without moe_align
    (`ember_moe_gate_up_silu_direct`): the assignments of each expert in groups of 16, each
    group computed by the workgroups of its first assignment (one per slab), the others
    exiting. Bit-identical to moe_align + moe_gate_up_silu; for decode batches (at most 256
    assignments)."""
    assert x.dim() == 2 and topk_ids.dim() == 2, (x.shape, topk_ids.shape)
    _require_device("moe_gate_up_silu_direct", x, topk_ids, packed.packed)
    n, k = topk_ids.shape
    if (packed.hidden, packed.dtype, packed.device) != (x.shape[1], x.dtype, x.device) or n > x.shape[0]:
        raise ValueError("moe_gate_up_silu_direct: the packed weight, x and topk_ids do not match")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"moe_gate_up_silu_direct: int32/int64 ids expected, got {topk_ids.dtype}")
    ids = topk_ids.contiguous()
    out = torch.empty((n * k, packed.inter), dtype=x.dtype, device=x.device)
    if n * k == 0:
        return out
    _launch("ember_moe_gate_up_silu_direct", _lib.load().ember_moe_gate_up_silu_direct, x.device,
            x.data_ptr(), x.stride(0), x.shape[0], packed.packed.data_ptr(), _lib.dtype_tag(x.dtype),
            packed.num_experts, packed.hidden, packed.inter, ids.data_ptr(), ids.element_size(), n * k, k,
            int(bool(half_slabs)), out.data_ptr(), out.stride(0))
    if _check_indices() and _lib.read_errors(clear=True) & _lib.ERR_EXPERT_ID:
        raise IndexError("emberserve_amd.moe_gate_up_silu_direct: expert id out of range")
    return out


def fused_moe_gate_up(x: Tensor, topk_ids: Tensor, w_gate_up: Tensor, *, num_splits: int | None = None,
                      packed: PackedExperts | None = None) -> Tensor:
    """The routed experts' activations [N * k, I] in assignment order (the `act` of
    moe_triton.py:340): up to DIRECT_MAX_TOKENS tokens over a packed weight straight from the
    routing ids; from
    GEMM_FROM assignments the prefill GEMM (`moe_gate_up_silu_gemm`); otherwise moe_align +
    the 16-block kernel (`moe_gate_up_silu`, packed up to PACKED_MAX_ASSIGNMENTS). Every
    path gives the same bits as the 16-block kernel at one k split."""
    aligned = x.is_cuda and fused_enabled(x) and x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0
    n, k = topk_ids.shape
    if (packed is not None and num_splits is None and n <= DIRECT_MAX_TOKENS and n * k <= DIRECT_MAX_ASSIGNMENTS
            and aligned):
        # decode batches: straight from the routing ids, no alignment launch (the same bits)
        half = moe_direct_half_slabs(n * k, packed.num_experts, packed.inter, x.device)
        return moe_gate_up_silu_direct(x, topk_ids, packed, half_slabs=half)
    E, two_i, H = w_gate_up.shape
    if (num_splits is None and n * k >= GEMM_FROM and aligned and x.dtype == w_gate_up.dtype
            and x.dtype in SUPPORTED_DTYPES and H % 64 == 0 and (two_i // 2) % 64 == 0
            and w_gate_up.stride(2) == 1 and w_gate_up.stride(1) % 8 == 0 and w_gate_up.stride(0) % 8 == 0
            and w_gate_up.data_ptr() % 16 == 0):
        # over the packed experts when there are (contiguous units; the same bits)
        if (two_i // 2) % 128 == 0:
            rows = 128 if n * k < GEMM_WIDE_FROM else 256
            return moe_gate_up_silu_gemm(x, w_gate_up, topk_ids, column_tile=128, block_rows=rows, packed=packed)
        return moe_gate_up_silu_gemm(x, w_gate_up, topk_ids, column_tile=64, block_rows=256, packed=packed)
    if packed is not None and n * k > PACKED_MAX_ASSIGNMENTS:
        packed = None  # the row kernel is faster there (see PACKED_MAX_ASSIGNMENTS)
    sorted_ids, block_expert, num_valid = moe_align(topk_ids, E)
    return moe_gate_up_silu(x, w_gate_up, sorted_ids, block_expert, num_valid, k,
                            num_splits=num_splits, packed=packed)
