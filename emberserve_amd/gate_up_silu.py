"""The dense MLP's gate_up projection with silu_and_mul as its epilogue, for decode-sized
batches: `silu_and_mul(gate_up_proj(x))` of Qwen2MLP.forward (emberserve/model/qwen2.py:
60-61) as one launch of `ember_gate_up_silu` (libember_ops.so).

    x [..., H] (T = prod of leading dims <= 64 tokens), weight [2I, H] (rows [0, I) gate,
    [I, 2I) up: nn.Linear(H, 2I).weight, qwen2.py:49-57) -> out [..., I]

Numerics: the unfused pair's. The projection's output is rounded to the activation dtype
before silu_and_mul reads it (ops.py:84-87), so g and u are rounded dot products; the dot
products are fp32 MFMA sums whose term order is the kernel's own, so results agree with
another GEMM to within that rounding.

Dispatch: by default the kernel runs for up to FUSED_TOKENS tokens, where it measured
faster than the unfused pair (torch's linear, i.e. hipBLASLt, then this library's
silu_and_mul) on MI355X: Qwen3-8B (H 4096, I 12288) 40 vs 45 us at 1-16 tokens, Qwen2.5-7B
(H 3584, I 18944) 54.5 vs 54.8 us. From 32 tokens on the library GEMM was as fast or faster,
so the unfused pair runs there; `fused=True` forces the kernel (up to 64 tokens; above, the
prefill-size MFMA GEMM with the activation as its epilogue, `gate_up_silu_gemm`, which also
never materialises the [T, 2I] projection) and `fused=False` the pair. Over a weight packed at load time (`packed=`) the kernel runs by
default up to PACKED_FUSED_TOKENS: 35.3 vs 46.1 us at 16 tokens and 37.1 vs 45.8 at 32
(Qwen3-8B), 52.0 vs 56.7 at 32 (Qwen2.5-7B); at 48-64 tokens it is ahead at Qwen3-8B
(44.5 vs 47.8) and behind at Qwen2.5-7B (65.0 vs 63.0). Where the kernel does not apply (more than 64 tokens, fp32, shapes
that are not multiples of 64, unaligned operands) the pair runs. CPU tensors, or
`EMBERSERVE_FUSED_OPS=0`, take the eager forms.

The kernel is persistent: `num_workgroups` workgroups (default one per CU) take equal runs
of (64-column slab, 64-k step) units; a slab shared by several runs is merged from
partials. The count comes from the device only and the partial scratch is cached per
shape, so a captured HIP graph replays exactly what was captured.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib, ops
from ._scratch import ScratchCache, round_up
from .ops import _check_indices, _launch, _require_device, fused_enabled
from .paged_decode import num_sms

MAX_TOKENS = 64           # the kernels' limit
PACKED_MAX_TOKENS = 64
FUSED_TOKENS = 16         # default dispatch, row kernel: the kernel up to here, the pair above
PACKED_FUSED_TOKENS = 32  # default dispatch over a packed weight
# Prefill sizes (gate_up_silu_gemm): 256-token tiles of 64, 96 or 128 gate (and as many up)
# columns. A workgroup's time follows the bytes it streams from L2 into LDS (all 256 x rows
# plus its 2·columns weight rows, at ~40-45 GB/s per CU), so the call takes about
# ceil(tiles / CUs) rounds of 256 + 2·columns rows each; gemm_column_tile minimises that.
# Measured (bf16, µs, 64 | 96 | 128 columns): Qwen3-8B 256 tokens 66.2 | 95.5 | 96.8,
# 512 tokens 128.0 | 99.0 | 112.6, 8192 tokens 1585 | 1423 | 1324; Qwen2.5-7B 256 tokens
# 113.7 | 91.2 | 94.0, 512 tokens 167.5 | 164.6 | 179.7, 8192 tokens 2142 | 1961 | 1834.
GEMM_TILES = (64, 96, 128)


def _tile_ok(inter: int, tile: int) -> bool:
    return inter >= tile and inter % (16 if tile == 96 else tile) == 0


def gemm_column_tile(tokens: int, inter: int, device: torch.device, tiles: tuple[int, ...] = GEMM_TILES) -> int:
    """The prefill GEMM's column tile from shapes: the one of `tiles` (64, 96 and 128; 96
    needs inter only a multiple of 16: its last tile may be ragged) with the fewest rows
    streamed per CU, ceil(tiles / CUs) x (256 + 2 x columns); the narrower on a tie."""
    ok = [t for t in tiles if _tile_ok(inter, t)]
    if not ok:
        raise ValueError(f"gate_up_silu_gemm: no column tile for I {inter}")
    rows, cus = -(-tokens // 256), max(1, num_sms(device))
    return min(ok, key=lambda t: (-(-(rows * -(-inter // t)) // cus) * (256 + 2 * t), t))


SLAB = 64          # output columns per workgroup
STEP = 64          # k per pipeline stage
SUPPORTED_DTYPES = (torch.float16, torch.bfloat16)


def gate_up_silu_workgroups(device: torch.device) -> int:
    """Persistent workgroups: one per CU (a workgroup's four waves keep three stages of
    16 KB weight loads in flight, enough for a CU's share of HBM bandwidth)."""
    return num_sms(device)


def _workspace_bytes(programs: int, tiles: int, hidden: int, inter: int) -> int:
    return _lib.load().ember_gate_up_silu_workspace_bytes(16 * tiles, hidden, inter, programs)


# Partials and arrival counters, zero-filled once and cached per (workgroups, token tile
# count, hidden, inter, device, stream) so graph replays see captured addresses and two
# streams never share counters.
_SCRATCH = ScratchCache("gate_up_silu")


def gate_up_silu_torch(x: Tensor, weight: Tensor) -> Tensor:
    """The unfused pair: silu_and_mul(F.linear(x, weight))."""
    return ops.silu_and_mul(F.linear(x, weight))


def _fits(x2: Tensor, weight: Tensor, out: Tensor, max_tokens: int = MAX_TOKENS) -> bool:
    T, H = x2.shape
    I = weight.shape[0] // 2
    return (1 <= T <= max_tokens and x2.dtype == weight.dtype == out.dtype and x2.dtype in SUPPORTED_DTYPES
            and H % STEP == 0 and I % SLAB == 0 and I >= SLAB
            and x2.stride(1) == 1 and weight.stride(1) == 1 and out.stride(1) == 1
            and x2.stride(0) % 8 == 0 and weight.stride(0) % 8 == 0 and out.stride(0) % 4 == 0
            and x2.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0 and out.data_ptr() % 16 == 0)


def _gemm_fits(x2: Tensor, weight: Tensor, out: Tensor) -> bool:
    """What the prefill GEMM needs beyond its column tile: fp16/bf16, H a multiple of 64,
    unit inner strides, 16-byte aligned bases (I only has to suit the tile: _tile_ok)."""
    T, H = x2.shape
    return (1 <= T <= 1 << 24 and x2.dtype == weight.dtype == out.dtype and x2.dtype in SUPPORTED_DTYPES
            and H % 64 == 0 and x2.stride(1) == 1 and weight.stride(1) == 1 and out.stride(1) == 1
            and x2.stride(0) % 8 == 0 and weight.stride(0) % 8 == 0 and out.stride(0) % 4 == 0
            and x2.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0 and out.data_ptr() % 16 == 0)


class PackedGateUp:
    """A gate_up weight [2I, H] rearranged for `ember_gate_up_silu_packed` run with
    `num_workgroups` workgroups: every MFMA operand fragment of the decode kernel is one
    contiguous KiB, and the units of work sit in the order the grid reads them, so the whole
    grid streams the weights front to back. Made once per weight by `pack_gate_up_weight`;
    holds 2 I H elements (the same bytes as the weight, which the caller keeps for the
    unfused path above FUSED_TOKENS)."""

    def __init__(self, packed: Tensor, hidden: int, inter: int, num_workgroups: int) -> None:
        self.packed, self.hidden, self.inter, self.num_workgroups = packed, hidden, inter, num_workgroups

    @property
    def dtype(self) -> torch.dtype:
        return self.packed.dtype

    @property
    def device(self) -> torch.device:
        return self.packed.device


def packed_workgroups(inter: int, device: torch.device) -> int:
    """The default grid of the packed kernels: the most workgroups, up to one per CU, whose
    runs are whole 64-column slabs (no partial sums to merge), else one per CU. Qwen3-8B (192
    slabs): 192 workgroups, 30.5 us at one token against 35.4 over 256; Qwen2.5-7B (296
    slabs): 148, 43.8 against 47.5 us."""
    slabs, cus = inter // SLAB, gate_up_silu_workgroups(device)
    per = -(-slabs // cus)
    return slabs // per if slabs % per == 0 else cus


def pack_gate_up_weight(weight: Tensor, num_workgroups: int | None = None) -> PackedGateUp:
    """The packed copy of weight [2I, H] (fp16/bf16 on the GPU, H and I multiples of 64) for
    a grid of `num_workgroups` (default: `packed_workgroups`)."""
    if weight.dim() != 2 or weight.shape[0] % 2 != 0 or weight.dtype not in SUPPORTED_DTYPES:
        raise ValueError(f"pack_gate_up_weight: a [2I, H] fp16/bf16 weight expected, got {tuple(weight.shape)} "
                         f"{weight.dtype}")
    _require_device("pack_gate_up_weight", weight)
    two_i, H = weight.shape
    I = two_i // 2
    if H % STEP or I % SLAB or weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        raise ValueError("pack_gate_up_weight: H and I must be multiples of 64, rows unit-stride and 16-byte aligned")
    programs = packed_workgroups(I, weight.device) if num_workgroups is None else int(num_workgroups)
    if programs < 1:
        raise ValueError(f"pack_gate_up_weight: num_workgroups must be >= 1, got {programs}")
    packed = torch.empty(two_i * H, dtype=weight.dtype, device=weight.device)
    _launch("ember_gate_up_silu_pack_weight", _lib.load().ember_gate_up_silu_pack_weight, weight.device,
            weight.data_ptr(), weight.stride(0), _lib.dtype_tag(weight.dtype), H, I, programs, packed.data_ptr())
    return PackedGateUp(packed, H, I, programs)


def gate_up_silu_gemm(x: Tensor, weight: Tensor, *, column_tile: int = 128, token_tile: int = 256) -> Tensor:
    """silu_and_mul(F.linear(x, weight)) as one MFMA GEMM whose epilogue applies the
    activation (`ember_gate_up_silu_gemm`): token_tile x (column_tile gate + column_tile up)
    tiles ((256, 64), (256, 96), (256, 128) or (128, 128)), any token count. Needs fp16/bf16,
    H a multiple of 64, I of column_tile (of 16 for 96: a ragged last tile)."""
    if weight.dim() != 2 or weight.shape[0] % 2 != 0 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"gate_up_silu_gemm: x {tuple(x.shape)} and weight {tuple(weight.shape)} do not match "
                         "a [2I, H] gate_up projection")
    _require_device("gate_up_silu_gemm", x, weight)
    H = x.shape[-1]
    I = weight.shape[0] // 2
    x2 = x.reshape(-1, H)
    T = x2.shape[0]
    out = torch.empty((T, I), dtype=x.dtype, device=x.device)
    if T == 0:
        return out.view(*x.shape[:-1], I)
    if not (_gemm_fits(x2, weight, out) and _tile_ok(I, column_tile)
            and (token_tile, column_tile) in ((256, 64), (256, 96), (256, 128), (128, 128))):
        raise ValueError(f"gate_up_silu_gemm: shape, dtype or alignment not supported (H {H}, I {I}, "
                         f"column_tile {column_tile}, {x.dtype})")
    _launch("ember_gate_up_silu_gemm", _lib.load().ember_gate_up_silu_gemm, x.device,
            x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0), _lib.dtype_tag(x.dtype),
            T, H, I, token_tile, column_tile, out.data_ptr(), out.stride(0))
    return out.view(*x.shape[:-1], I)


PACKED_GEMM_TILES = (64, 128)  # the packed GEMM's column tiles: whole 64-row slabs


def gate_up_silu_gemm_packed(x: Tensor, packed: PackedGateUp, *, column_tile: int | None = None,
                             token_tile: int = 256) -> Tensor:
    """gate_up_silu_gemm over the packed weight (`ember_gate_up_silu_gemm_packed`): the same
    tiles but the 96-column one, the same results bit for bit. With it the packed copy is
    the only gate_up weight a model needs (decode kernels and prefill read it)."""
    H, I = packed.hidden, packed.inter
    if x.shape[-1] != H or x.dtype != packed.dtype:
        raise ValueError(f"gate_up_silu_gemm_packed: x {tuple(x.shape)} {x.dtype} does not match the packed "
                         f"[{2 * I}, {H}] {packed.dtype} weight")
    _require_device("gate_up_silu_gemm_packed", x, packed.packed)
    x2 = x.reshape(-1, H)
    T = x2.shape[0]
    out = torch.empty((T, I), dtype=x.dtype, device=x.device)
    if T == 0:
        return out.view(*x.shape[:-1], I)
    if column_tile is None:
        column_tile = gemm_column_tile(T, I, x.device, PACKED_GEMM_TILES)
    if not (T <= 1 << 24 and x2.stride(1) == 1 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0
            and (token_tile, column_tile) in ((256, 64), (256, 128), (128, 128)) and I % column_tile == 0):
        raise ValueError(f"gate_up_silu_gemm_packed: shape, stride or tile not supported (I {I}, "
                         f"column_tile {column_tile}, token_tile {token_tile})")
    _launch("ember_gate_up_silu_gemm_packed", _lib.load().ember_gate_up_silu_gemm_packed, x.device,
            x2.data_ptr(), x2.stride(0), packed.packed.data_ptr(), _lib.dtype_tag(x.dtype), T, H, I,
            packed.num_workgroups, token_tile, column_tile, out.data_ptr(), out.stride(0))
    return out.view(*x.shape[:-1], I)


def gate_up_silu(x: Tensor, weight: Tensor | None, *, num_workgroups: int | None = None,
                 fused: bool | None = None, packed: PackedGateUp | None = None) -> Tensor:
    """silu_and_mul(F.linear(x, weight)) with weight [2I, H] (qwen2.py:60-61). With `packed`
    (`pack_gate_up_weight(weight)`), the fused kernel reads the packed copy instead. With
    `packed` and weight None (a model that dropped the unpacked weight) every size runs on
    the packed copy: the decode kernel up to PACKED_MAX_TOKENS tokens, the packed prefill
    GEMM above."""
    if weight is None:
        if packed is None:
            raise ValueError("gate_up_silu: weight None needs the packed weight")
        if fused is False:
            raise ValueError("gate_up_silu: the unfused pair needs the unpacked weight")
        if x.reshape(-1, packed.hidden).shape[0] > PACKED_MAX_TOKENS:
            return gate_up_silu_gemm_packed(x, packed)
        return _packed_decode(x, packed, num_workgroups)
    return _gate_up_silu_decode(x, weight, num_workgroups, fused, packed)


def _packed_decode(x: Tensor, packed: PackedGateUp, num_workgroups: int | None) -> Tensor:
    """The decode kernel over the packed weight alone, 1..PACKED_MAX_TOKENS tokens."""
    H, I = packed.hidden, packed.inter
    if x.shape[-1] != H or x.dtype != packed.dtype:
        raise ValueError(f"gate_up_silu: x {tuple(x.shape)} {x.dtype} does not match the packed "
                         f"[{2 * I}, {H}] {packed.dtype} weight")
    _require_device("gate_up_silu", x, packed.packed)
    if num_workgroups is not None and int(num_workgroups) != packed.num_workgroups:
        raise ValueError(f"gate_up_silu: the weight was packed for {packed.num_workgroups} workgroups, "
                         f"not {num_workgroups}")
    x2 = x.reshape(-1, H)
    T = x2.shape[0]
    out = torch.empty((T, I), dtype=x.dtype, device=x.device)
    if T == 0:
        return out.view(*x.shape[:-1], I)
    if not (x2.stride(1) == 1 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0):
        raise ValueError("gate_up_silu: x needs unit inner stride, rows a multiple of 8 elements apart "
                         "and 16-byte alignment for the packed weight")
    _launch_packed(x2, packed, packed.num_workgroups, out)
    return out.view(*x.shape[:-1], I)


def _launch_packed(x2: Tensor, packed: PackedGateUp, programs: int, out: Tensor) -> None:
    T, H = x2.shape
    I = packed.inter
    tiles = -(-T // 16)
    ws = _SCRATCH.get((programs, tiles, H, I), lambda: _workspace_bytes(programs, tiles, H, I), x2.device)
    _launch("ember_gate_up_silu_packed", _lib.load().ember_gate_up_silu_packed, x2.device,
            x2.data_ptr(), x2.stride(0), packed.packed.data_ptr(), _lib.dtype_tag(x2.dtype),
            T, H, I, programs, ws.data_ptr(), ws.numel() * 4, out.data_ptr(), out.stride(0))
    if _check_indices():
        need, slabs = _workspace_bytes(programs, tiles, H, I), I // SLAB
        _SCRATCH.verify_counters(ws, need - round_up(slabs * 4, 256), need - round_up(slabs * 4, 256) + slabs * 4)


def _gate_up_silu_decode(x: Tensor, weight: Tensor, num_workgroups: int | None, fused: bool | None,
                         packed: PackedGateUp | None) -> Tensor:
    if weight.dim() != 2 or weight.shape[0] % 2 != 0 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"gate_up_silu: x {tuple(x.shape)} and weight {tuple(weight.shape)} do not match "
                         "a [2I, H] gate_up projection")
    if not fused_enabled(x):
        return gate_up_silu_torch(x, weight)
    _require_device("gate_up_silu", x, weight)
    H = x.shape[-1]
    I = weight.shape[0] // 2
    x2 = x.reshape(-1, H)
    T = x2.shape[0]
    out = torch.empty((T, I), dtype=x.dtype, device=x.device)
    if T == 0:
        return out.view(*x.shape[:-1], I)
    limit, default = (PACKED_MAX_TOKENS, PACKED_FUSED_TOKENS) if packed is not None else (MAX_TOKENS, FUSED_TOKENS)
    if fused is True and T > limit and _gemm_fits(x2, weight, out) and any(_tile_ok(I, t) for t in GEMM_TILES):
        # the fused form asked for at prefill sizes: the MFMA GEMM with the activation epilogue
        return gate_up_silu_gemm(x, weight, column_tile=gemm_column_tile(T, I, x.device))
    if fused is False or (fused is None and T > default) or not _fits(x2, weight, out, limit):
        return gate_up_silu_torch(x, weight)
    programs = gate_up_silu_workgroups(x.device) if num_workgroups is None else int(num_workgroups)
    if packed is not None:
        if num_workgroups is not None and programs != packed.num_workgroups:
            raise ValueError(f"gate_up_silu: the weight was packed for {packed.num_workgroups} workgroups, "
                             f"not {programs}")
        programs = packed.num_workgroups
    if programs < 1:
        raise ValueError(f"gate_up_silu: num_workgroups must be >= 1, got {programs}")
    if packed is not None:
        if (packed.hidden, packed.inter, packed.dtype, packed.device) != (H, I, x.dtype, x.device):
            raise ValueError("gate_up_silu: the packed weight does not match x and weight")
        _launch_packed(x2, packed, programs, out)
        return out.view(*x.shape[:-1], I)
    tiles = -(-T // 16)
    ws = _SCRATCH.get((programs, tiles, H, I), lambda: _workspace_bytes(programs, tiles, H, I), x.device)
    _launch("ember_gate_up_silu", _lib.load().ember_gate_up_silu, x.device,
            x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0), _lib.dtype_tag(x.dtype),
            T, H, I, programs, ws.data_ptr(), ws.numel() * 4, out.data_ptr(), out.stride(0))
    if _check_indices():
        need, slabs = _workspace_bytes(programs, tiles, H, I), I // SLAB
        _SCRATCH.verify_counters(ws, need - round_up(slabs * 4, 256), need - round_up(slabs * 4, 256) + slabs * 4)
    return out.view(*x.shape[:-1], I)
