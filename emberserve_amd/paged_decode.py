"""Paged decode attention on MI355X: the drop-in for `paged_attention_decode` of
emberserve/attn/paged_triton.py (:323-399), with the same signature, argument meaning,
layout assertions and split-K contract, running `ember_paged_decode` (libember_ops.so).

    q [B, H, D]; k_cache / v_cache [num_blocks, block_size, Hkv, D]; block_tables
    [B, max_blocks] int32 (padding entries must be valid ids); context_lens [B] int32
    counting the token written this step. Returns [B, H, D] in q.dtype.

Numerics: the reference's default "dot" variant (EMBERSERVE_TRITON_VARIANT, :263-277):
fp16/bf16 q and cache of one dtype run on MFMA with fp32 scores and the probabilities
rounded to the cache dtype before P.V; variant="sum", fp32 caches and dtype mixes compute
in fp32 throughout. CPU tensors take the eager form of PagedTorchAttentionBackend._decode
(attn/paged_torch.py:87-98).

The split count comes from shapes only (batch, table width), never from tensor values, so
a captured HIP graph replays exactly what was captured; the split-K scratch is cached per
shape for the same reason (paged_triton.py:293-310).
"""

from __future__ import annotations

import os

import torch
from torch import Tensor

from . import _lib
from ._scratch import ScratchCache, round_up
from .ops import _check_indices, _launch, _require_device

BLOCK_MULTIPLE = 16
SUPPORTED_HEAD_DIMS = (64, 128)
SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
VARIANTS = ("sum", "dot")
MAX_SPLITS = 32
TILE = 32                 # keys per kernel tile
MIN_KEYS_PER_SPLIT = 256
LONG_SPLIT_KEYS = 512     # keys per split at which MAX_SPLITS splits are allowed


def interpreter_enabled() -> bool:
    """The reference's Triton-interpreter switch (paged_triton.py:69-70); kept for the API.
    This module never interprets: CPU tensors take the eager form."""
    return False


def is_available() -> bool:
    """True when a GPU is present and the library loads (the reference's availability probe,
    paged_triton.py:73-80)."""
    if not torch.cuda.is_available():
        return False
    try:
        _lib.load()
    except RuntimeError:
        return False
    return True


_CU_COUNT: dict[int, int] = {}


def num_sms(device: torch.device) -> int:
    """Compute units of `device` (the reference's SM count, paged_triton.py:240-247)."""
    if device.type != "cuda":
        return 1
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CU_COUNT[idx]


def default_num_splits(batch: int, num_kv_heads: int, max_context: int, device: torch.device,
                       num_heads: int | None = None, head_dim: int = 128) -> int:
    """Split-K factor from SHAPES only (paged_triton.py:250-276 contract).

    `EMBERSERVE_TRITON_SPLITS=<n>` forces a value (1 disables split-K). Otherwise the grid
    is sized to one workgroup per compute unit: a (sequence, KV head, 16-head chunk)
    workgroup (8 waves at head_dim 64, 4 at 128) keeps one CU's share of HBM bandwidth in
    flight, and more workgroups only add merge work (measured on MI355X, rotated inputs:
    128 x 2048 keys at D=64 4.8 TB/s unsplit vs 4.4 at 2 splits; 8 x 8192 keys at D=128
    5.0 TB/s at 4 splits = 256 workgroups). Contexts are cut into round(CUs / programs)
    pieces, never below MIN_KEYS_PER_SPLIT keys each, and at most MAX_SPLITS / 2 unless the
    context gives every one of MAX_SPLITS splits LONG_SPLIT_KEYS keys. `head_dim` is
    accepted for callers that size by it; the rule does not need it.
    """
    forced = os.environ.get("EMBERSERVE_TRITON_SPLITS")
    if forced:
        return max(1, int(forced))
    del head_dim
    chunks = 1
    if num_heads is not None and num_kv_heads > 0:
        chunks = -(-(num_heads // num_kv_heads) // 16)
    programs = max(1, batch * num_kv_heads * chunks)
    target = num_sms(device)
    want = (target + programs // 2) // programs
    by_context = max(1, max_context // MIN_KEYS_PER_SPLIT)
    # The in-kernel merge grows with the split count: 32 splits pay only once every split
    # holds >= 512 keys (measured, B = 1, 32q/8kv x 128, splits 16 / 32: ctx 8192 16.7 /
    # 17.4 us; ctx 16384 25.0 / 22.9; ctx 32768 41.7 / 33.5; 40-64 splits were slower than
    # 32 up to 65536 keys).
    cap = MAX_SPLITS if max_context >= MAX_SPLITS * LONG_SPLIT_KEYS else MAX_SPLITS // 2
    return max(1, min(cap, want, by_context))


def default_variant() -> str:
    """`EMBERSERVE_TRITON_VARIANT=sum|dot`, default `dot` (paged_triton.py:263-277)."""
    v = os.environ.get("EMBERSERVE_TRITON_VARIANT", "dot").lower()
    if v not in VARIANTS:
        raise ValueError(f"EMBERSERVE_TRITON_VARIANT must be one of {VARIANTS}, got {v!r}")
    return v


def _workspace_bytes(num_splits: int, batch: int, num_heads: int, head_dim: int) -> int:
    return _lib.load().ember_paged_decode_workspace_bytes(batch, num_heads, head_dim, num_splits)


# Split-K partials and arrival counters, cached per (num_splits, B, H, D, device, stream) so a
# graph replay reads the addresses that were captured (paged_triton.py:293-310) and two
# streams never share counters.
_SCRATCH = ScratchCache("paged_attention_decode", min_bytes=16)


def paged_decode_torch(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_tables: Tensor,
                       context_lens: Tensor, scale: float) -> Tensor:
    """PagedTorchAttentionBackend._decode (attn/paged_torch.py:87-98) over the gather of
    PagedKVCache.gather_batch (kv/cache.py:81-107): the CPU-tensor path."""
    bs = k_cache.shape[1]
    ctx = context_lens.to(device=k_cache.device, dtype=torch.long)
    max_ctx = int(ctx.max())
    nb = -(-max_ctx // bs)
    idx = block_tables[:, :nb].to(device=k_cache.device, dtype=torch.long).clamp_min(0)
    b = idx.shape[0]
    k = k_cache[idx].reshape(b, nb * bs, k_cache.shape[2], k_cache.shape[3])[:, :max_ctx]
    v = v_cache[idx].reshape(b, nb * bs, v_cache.shape[2], v_cache.shape[3])[:, :max_ctx]
    valid = torch.arange(max_ctx, device=k_cache.device)[None, :] < ctx[:, None]
    groups = q.shape[1] // k_cache.shape[2]
    kf = k.float().repeat_interleave(groups, dim=2)
    vf = v.float().repeat_interleave(groups, dim=2)
    scores = torch.einsum("bhd,bkhd->bhk", q.float(), kf) * scale
    scores = scores.masked_fill(~valid[:, None, :], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    return torch.einsum("bhk,bkhd->bhd", probs, vf).to(q.dtype)


def paged_attention_decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_tables: Tensor,
                           context_lens: Tensor, scale: float, *, num_splits: int | None = None,
                           out: Tensor | None = None, num_warps: int = 4,
                           variant: str | None = None) -> Tensor:
    """One-token-per-sequence paged attention (paged_triton.py:323-399). `num_warps` is
    accepted for signature compatibility; the kernel's workgroup shape is fixed."""
    del num_warps
    B, H, D = q.shape
    num_blocks, block_size, Hkv, Dk = k_cache.shape
    assert Dk == D and v_cache.shape == k_cache.shape, (q.shape, k_cache.shape, v_cache.shape)
    assert D in SUPPORTED_HEAD_DIMS, f"head_dim {D} not in {SUPPORTED_HEAD_DIMS}"
    assert block_size % BLOCK_MULTIPLE == 0, f"block_size {block_size} % {BLOCK_MULTIPLE} != 0"
    assert H % Hkv == 0, (H, Hkv)
    assert k_cache.dtype in SUPPORTED_DTYPES, k_cache.dtype
    assert v_cache.dtype == k_cache.dtype, (k_cache.dtype, v_cache.dtype)
    assert q.dtype in SUPPORTED_DTYPES, q.dtype
    assert block_tables.dtype == torch.int32 and block_tables.shape[0] == B, block_tables.shape
    assert context_lens.dtype == torch.int32 and context_lens.shape == (B,), context_lens.shape
    assert q.stride(2) == 1 and k_cache.stride(3) == 1 and v_cache.stride(3) == 1
    assert block_tables.stride(1) == 1 and context_lens.stride(0) == 1
    variant = variant or default_variant()
    assert variant in VARIANTS, variant
    if out is None:
        out = torch.empty_like(q)
    assert out.shape == q.shape and out.stride(2) == 1 and out.dtype == q.dtype
    if not q.is_cuda:
        out.copy_(paged_decode_torch(q, k_cache, v_cache, block_tables, context_lens, scale))
        return out
    _require_device("paged_attention_decode", q, k_cache, v_cache, block_tables, context_lens, out)
    if B == 0:
        return out
    max_blocks = block_tables.shape[1]
    max_context = max_blocks * block_size
    num_tiles_max = max(1, -(-max_context // TILE))
    if num_splits is None:
        num_splits = default_num_splits(B, Hkv, max_context, q.device, H, D)
    num_splits = max(1, min(int(num_splits), num_tiles_max))
    ws = None
    if num_splits > 1:
        ws = _SCRATCH.get((num_splits, B, H, D), lambda: _workspace_bytes(num_splits, B, H, D), q.device)
    flags = _lib.DECODE_FP32 if variant == "sum" else 0
    _launch("ember_paged_decode", _lib.load().ember_paged_decode, q.device,
            q.data_ptr(), q.stride(0), q.stride(1), _lib.dtype_tag(q.dtype),
            k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, block_size, Hkv, D,
            k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
            v_cache.stride(0), v_cache.stride(1), v_cache.stride(2), _lib.dtype_tag(k_cache.dtype),
            block_tables.data_ptr(), block_tables.stride(0), max_blocks, context_lens.data_ptr(), B, H,
            float(scale), num_splits, flags,
            ws.data_ptr() if ws is not None else None, ws.numel() * 4 if ws is not None else 0,
            out.data_ptr(), out.stride(0), out.stride(1))
    if _check_indices():
        if ws is not None:
            need = _workspace_bytes(num_splits, B, H, D)
            _SCRATCH.verify_counters(ws, need - round_up(B * H * 4, 16), need - round_up(B * H * 4, 16) + B * H * 4)
        flags = _lib.read_errors(clear=True)
        if flags & _lib.ERR_DECODE_CTX:
            raise IndexError("emberserve_amd.paged_attention_decode: context length outside the block table")
        if flags & _lib.ERR_BLOCK_ID:
            raise IndexError("emberserve_amd.paged_attention_decode: block id outside the cache")
    return out
