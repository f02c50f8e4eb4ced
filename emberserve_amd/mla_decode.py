"""Absorbed-form MLA decode on MI355X: the drop-in for `mla_decode` / `mla_num_splits` of
emberserve/attn/mla_triton.py (:119-182, :188-202), with the same signature, argument
meaning, layout assertions and split-K contract, running `ember_mla_decode`
(libember_ops.so).

    q_abs: [B, H, DL + DR] = [q_c | q_pe], or the pair (q_c [B, H, DL], q_pe [B, H, DR]);
    latent_cache [num_blocks, block_size, DL + DR]; block_tables [B, max_blocks] int32
    (padding entries must be valid ids); context_lens [B] int32. Returns out_c [B, H, DL] =
    softmax(scores) . c in q's dtype (W_UV is applied by the caller).

Numerics: the reference kernel's tl.dot ones. fp16/bf16 q and cache of one dtype at the
DeepSeek/Moonlight geometry (DL 512, DR 64) run on MFMA with fp32 scores and the
probabilities rounded to the cache dtype before P.V; fp32 and other geometries compute in
fp32. CPU tensors take the eager form of mla_attention_absorbed with identity W
(attn/mla_torch.py:33-53), the definition the reference tests compare the kernel with.

The split count comes from shapes only, so a captured HIP graph replays exactly what was
captured; the split-K scratch is cached per shape for the same reason.
"""

from __future__ import annotations

import math
import os

import torch
from torch import Tensor

from . import _lib
from ._scratch import ScratchCache, round_up
from .ops import _check_indices, _launch, _require_device
from .paged_decode import num_sms

SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
BLOCK_MULTIPLE = 16
MAX_SPLITS = 128
TILE = 32                 # keys per kernel tile
MAX_DIM = 1024            # DL + DR of the fp32 kernel


def mla_num_splits(batch: int, device: torch.device, *, num_heads: int = 16,
                   max_context: int | None = None) -> int:
    """Split-K factor from SHAPES only (mla_triton.py:188-202 contract).

    `EMBERSERVE_TRITON_SPLITS=<n>` forces a value. Otherwise the grid is sized to one
    (sequence, 16-head chunk, split) workgroup per compute unit, and with `max_context`
    (the table width in keys) to about sqrt(max_context / 4) splits, at least 16 keys
    each: a split's fixed cost (three dependent reads before its first tile, its share of
    the merge) wants more keys per split as contexts grow. From 4 splits the merge is its
    own wide launch, which makes splits cheap. Measured on MI355X (bf16, 16 heads, block
    16), best split counts: B = 1 at 320 / 1024 / 4096 / 8192 / 32768 keys: 6-8 / 16 / 32
    / 48-64 / 128 (10.2, 11.3, 15.1, 18.6, 32.7 us); B = 128 x 2048: 2 (4.6 TB/s); B = 256
    x 2048: 1 (5.4 TB/s). The reference's signature (batch, device) stays valid."""
    forced = os.environ.get("EMBERSERVE_TRITON_SPLITS")
    if forced:
        return max(1, int(forced))
    chunks = -(-max(1, num_heads) // 16)
    programs = max(1, batch * chunks)
    want = max(1, num_sms(device) // programs)
    if max_context is not None:
        keys = max(0, max_context)
        want = min(want, max(1, math.isqrt(keys // 4)), max(1, -(-keys // 16)))
    return max(1, min(MAX_SPLITS, want))


def _workspace_bytes(num_splits: int, batch: int, num_heads: int, dl: int) -> int:
    return _lib.load().ember_mla_decode_workspace_bytes(batch, num_heads, dl, num_splits)


# Split-K partials and arrival counters, cached per (num_splits, B, H, DL, device, stream) so
# a graph replay reads the addresses that were captured (the reference's _SCRATCH) and two
# streams never share counters.
_SCRATCH = ScratchCache("mla_decode", min_bytes=16)


def mla_decode_torch(q_c: Tensor, q_pe: Tensor, latent_cache: Tensor, block_tables: Tensor,
                     context_lens: Tensor, scale: float, kv_lora_rank: int) -> Tensor:
    """mla_attention_absorbed with identity W_UK / W_UV per sequence (mla_torch.py:33-53)
    over PagedLatentCache.gather (kv/cache.py): the CPU-tensor path, fp32 math."""
    bs = latent_cache.shape[1]
    outs = []
    for b in range(q_c.shape[0]):
        n = int(context_lens[b])
        nb = -(-n // bs)
        idx = block_tables[b, :nb].to(device=latent_cache.device, dtype=torch.long)
        rows = latent_cache[idx].reshape(-1, latent_cache.shape[2])[:n].float()
        c, k_pe = rows[:, :kv_lora_rank], rows[:, kv_lora_rank:]
        scores = (q_c[b].float() @ c.T + q_pe[b].float() @ k_pe.T) * scale  # [H, n]
        outs.append(torch.softmax(scores, dim=-1) @ c)
    return torch.stack(outs).to(q_c.dtype)


def mla_decode(q_abs: Tensor | tuple[Tensor, Tensor], latent_cache: Tensor, block_tables: Tensor,
               context_lens: Tensor, scale: float, kv_lora_rank: int, *,
               num_splits: int | None = None, out: Tensor | None = None,
               num_warps: int = 8) -> Tensor:
    """One-query-per-sequence latent attention (mla_triton.py:119-182). `num_warps` is
    accepted for signature compatibility; the kernel's workgroup shape is fixed."""
    del num_warps
    DL = kv_lora_rank
    if isinstance(q_abs, tuple):
        q_c, q_pe = q_abs
        assert q_c.shape[:2] == q_pe.shape[:2] and q_c.shape[2] == DL, (q_c.shape, q_pe.shape)
        D = DL + q_pe.shape[2]
    else:
        q_c, q_pe = q_abs[..., :DL], q_abs[..., DL:]
        D = q_abs.shape[2]
    B, H = q_c.shape[:2]
    num_blocks, block_size, Dl = latent_cache.shape
    DR = D - DL
    assert Dl == D, (latent_cache.shape, D)
    assert DL & (DL - 1) == 0 and DR & (DR - 1) == 0 and DR >= 16, (DL, DR)
    assert D <= MAX_DIM, f"kv_lora_rank + rope dim {D} > {MAX_DIM}"
    assert q_c.dtype == q_pe.dtype == latent_cache.dtype and q_c.dtype in SUPPORTED_DTYPES, \
        (q_c.dtype, q_pe.dtype, latent_cache.dtype)
    assert q_c.stride(2) == 1 and q_pe.stride(2) == 1 and latent_cache.stride(2) == 1
    assert block_tables.dtype == torch.int32 and context_lens.dtype == torch.int32
    assert block_tables.shape[0] == B and context_lens.shape == (B,)
    assert block_size % BLOCK_MULTIPLE == 0, f"block_size {block_size} % {BLOCK_MULTIPLE} != 0"
    assert block_tables.stride(1) == 1 and context_lens.stride(0) == 1
    if out is None:
        out = torch.empty((B, H, DL), dtype=q_c.dtype, device=q_c.device)
    assert out.shape == (B, H, DL) and out.stride(2) == 1 and out.dtype == q_c.dtype
    if not q_c.is_cuda:
        out.copy_(mla_decode_torch(q_c, q_pe, latent_cache, block_tables, context_lens, scale, DL))
        return out
    _require_device("mla_decode", q_c, q_pe, latent_cache, block_tables, context_lens, out)
    if B == 0:
        return out
    max_blocks = block_tables.shape[1]
    max_context = max_blocks * block_size
    num_tiles_max = max(1, -(-max_context // TILE))
    if num_splits is None:
        num_splits = mla_num_splits(B, q_c.device, num_heads=H, max_context=max_context)
    num_splits = max(1, min(int(num_splits), num_tiles_max))
    ws = None
    if num_splits > 1:
        ws = _SCRATCH.get((num_splits, B, H, DL), lambda: _workspace_bytes(num_splits, B, H, DL), q_c.device)
    _launch("ember_mla_decode", _lib.load().ember_mla_decode, q_c.device,
            q_c.data_ptr(), q_c.stride(0), q_c.stride(1), q_pe.data_ptr(), q_pe.stride(0), q_pe.stride(1),
            _lib.dtype_tag(q_c.dtype), latent_cache.data_ptr(), num_blocks, block_size, DL, DR,
            latent_cache.stride(0), latent_cache.stride(1), _lib.dtype_tag(latent_cache.dtype),
            block_tables.data_ptr(), block_tables.stride(0), max_blocks, context_lens.data_ptr(), B, H,
            float(scale), num_splits,
            ws.data_ptr() if ws is not None else None, ws.numel() * 4 if ws is not None else 0,
            out.data_ptr(), out.stride(0), out.stride(1))
    if _check_indices():
        if ws is not None:
            need = _workspace_bytes(num_splits, B, H, DL)
            start = need - round_up(B * H * 4, 16)
            _SCRATCH.verify_counters(ws, start, start + B * H * 4)
        raise_decode_errors(_lib.read_errors(clear=True))
    return out


def raise_decode_errors(flags: int) -> None:
    """Maps the device error word after an mla_decode launch to an exception. A handshake
    that ran out (ERR_SYNC) has already turned the affected output rows into NaN in the
    kernel; the bit says why."""
    if flags & _lib.ERR_DECODE_CTX:
        raise IndexError("emberserve_amd.mla_decode: context length outside the block table")
    if flags & _lib.ERR_BLOCK_ID:
        raise IndexError("emberserve_amd.mla_decode: block id outside the cache")
    if flags & _lib.ERR_SYNC:
        raise RuntimeError("emberserve_amd.mla_decode: an in-kernel wave handshake timed out; the rows of "
                           "the affected workgroups were written as NaN")
