"""The ops registered with the PyTorch dispatcher as `torch.ops.emberserve.*`.

`emberserve_amd.ops` launches the kernels straight through the C ABI, which serves eager
code and HIP-graph capture. Registering the same functions as `torch.library` custom ops
adds what the dispatcher offers on top: a declared schema (which arguments each op
mutates), fake-tensor kernels, so `torch.compile` and FakeTensor tracing see the right
output shapes without launching anything, and one name per op that survives export.

Every implementation calls the corresponding `emberserve_amd.ops` function, so the
dispatch is the same as for direct calls: the HIP library for GPU tensors (failing loudly
if it is missing), the eager torch forms for CPU tensors or with `EMBERSERVE_FUSED_OPS=0`.
The ops that work in place (rope, qk-norm + rope, the MLA q_pe rotation, the cache writes)
return nothing at the dispatcher level and always write their results into the
arguments their schema names as mutated; the eager forms return new tensors, so their
results are copied back. The wrappers at the bottom return those tensors, as the
reference's functions do (`model/ops.py:92-115`).
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.library import custom_op

from . import ops as _ops

__all__ = ["rmsnorm", "fused_add_rmsnorm", "rope", "silu_and_mul", "embedding", "qk_norm_rope",
           "mla_latent_rope", "kv_cache_write", "latent_cache_write", "paged_attention_decode", "mla_decode",
           "gate_up_silu", "moe_gate_up_silu"]


def _empty(shape, like: Tensor) -> Tensor:
    return torch.empty(tuple(shape), dtype=like.dtype, device=like.device)


def _into(dst: Tensor, src: Tensor) -> None:
    if src is not dst:
        dst.copy_(src)


# ---- rmsnorm / fused add + rmsnorm (model/ops.py:92-102) ---------------------------------

@custom_op("emberserve::rmsnorm", mutates_args=())
def _rmsnorm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    return _ops.rmsnorm(x, weight, eps)


@_rmsnorm.register_fake
def _(x, weight, eps):
    return _empty(x.shape, x)


@custom_op("emberserve::fused_add_rmsnorm", mutates_args=())
def _fused_add_rmsnorm(x: Tensor, residual: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    return _ops.fused_add_rmsnorm(x, residual, weight, eps)


@_fused_add_rmsnorm.register_fake
def _(x, residual, weight, eps):
    return _empty(x.shape, x), _empty(residual.shape, x)


# ---- rope (model/ops.py:104-109), in place ----------------------------------------------

@custom_op("emberserve::rope", mutates_args=("q", "k"))
def _rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor, positions: Tensor) -> None:
    q2, k2 = _ops.rope(q, k, cos, sin, positions)
    _into(q, q2)
    _into(k, k2)


@_rope.register_fake
def _(q, k, cos, sin, positions):
    return None


# ---- silu_and_mul (model/ops.py:111-115) -------------------------------------------------

@custom_op("emberserve::silu_and_mul", mutates_args=())
def _silu_and_mul(x: Tensor) -> Tensor:
    return _ops.silu_and_mul(x)


@_silu_and_mul.register_fake
def _(x):
    return _empty(tuple(x.shape[:-1]) + (x.shape[-1] // 2,), x)


# ---- gate_up projection + silu_and_mul (model/qwen2.py:60-61) -----------------------------

@custom_op("emberserve::gate_up_silu", mutates_args=())
def _gate_up_silu(x: Tensor, weight: Tensor) -> Tensor:
    from .gate_up_silu import gate_up_silu as impl
    return impl(x, weight)


@_gate_up_silu.register_fake
def _(x, weight):
    return _empty(tuple(x.shape[:-1]) + (weight.shape[0] // 2,), x)


@custom_op("emberserve::moe_gate_up_silu", mutates_args=())
def _moe_gate_up_silu(x: Tensor, w_gate_up: Tensor, sorted_ids: Tensor, block_expert: Tensor, num_valid: int,
                      top_k: int) -> Tensor:
    from .moe import moe_gate_up_silu as impl
    return impl(x, w_gate_up, sorted_ids, block_expert, num_valid, top_k)


@_moe_gate_up_silu.register_fake
def _(x, w_gate_up, sorted_ids, block_expert, num_valid, top_k):
    return _empty((num_valid, w_gate_up.shape[1] // 2), x)


@custom_op("emberserve::moe_align", mutates_args=())
def _moe_align(topk_ids: Tensor, num_experts: int, block_m: int) -> tuple[Tensor, Tensor]:
    from .moe import moe_align as impl
    sorted_ids, block_expert, _ = impl(topk_ids, num_experts, block_m)
    return sorted_ids, block_expert


@_moe_align.register_fake
def _(topk_ids, num_experts, block_m):
    nv = topk_ids.numel()
    padded = (nv + num_experts * (block_m - 1) + block_m - 1) // block_m * block_m
    return (topk_ids.new_empty((padded,), dtype=torch.int32),
            topk_ids.new_empty((padded // block_m,), dtype=torch.int32))


@custom_op("emberserve::fused_moe_gate_up", mutates_args=())
def _fused_moe_gate_up(x: Tensor, topk_ids: Tensor, w_gate_up: Tensor) -> Tensor:
    from .moe import fused_moe_gate_up as impl
    return impl(x, topk_ids, w_gate_up)


@_fused_moe_gate_up.register_fake
def _(x, topk_ids, w_gate_up):
    return _empty((topk_ids.numel(), w_gate_up.shape[1] // 2), x)


# ---- embedding (nn.Embedding in model/qwen2.py:172) ---------------------------------------

@custom_op("emberserve::embedding", mutates_args=())
def _embedding(ids: Tensor, weight: Tensor) -> Tensor:
    return _ops.embedding(ids, weight)


@_embedding.register_fake
def _(ids, weight):
    return _empty(tuple(ids.shape) + (weight.shape[1],), weight)


# ---- Qwen3 qk-norm + rope (model/qwen2.py:95-101), in place ------------------------------

@custom_op("emberserve::qk_norm_rope", mutates_args=("q", "k"))
def _qk_norm_rope(q: Tensor, k: Tensor, q_weight: Tensor, k_weight: Tensor, eps: float, cos: Tensor,
                  sin: Tensor, positions: Tensor) -> None:
    q2, k2 = _ops.qk_norm_rope(q, k, q_weight, k_weight, eps, cos, sin, positions)
    _into(q, q2)
    _into(k, k2)


@_qk_norm_rope.register_fake
def _(q, k, q_weight, k_weight, eps, cos, sin, positions):
    return None


# ---- MLA latent norm + decoupled rope (model/deepseek.py:126-133) -------------------------

@custom_op("emberserve::mla_latent_rope", mutates_args=("q_pe",))
def _mla_latent_rope(c: Tensor, k_pe: Tensor, q_pe: Tensor, weight: Tensor, eps: float, cos: Tensor,
                     sin: Tensor, positions: Tensor) -> Tensor:
    q2, latent = _ops.mla_latent_rope(c, k_pe, q_pe, weight, eps, cos, sin, positions)
    _into(q_pe, q2)
    return latent


@_mla_latent_rope.register_fake
def _(c, k_pe, q_pe, weight, eps, cos, sin, positions):
    return _empty(tuple(c.shape[:-1]) + (c.shape[-1] + k_pe.shape[-1],), c)


# ---- paged cache writes (kv/cache.py:54-61, 152-157) --------------------------------------

@custom_op("emberserve::kv_cache_write", mutates_args=("k_cache", "v_cache"))
def _kv_cache_write(k: Tensor, v: Tensor, slot_mapping: Tensor, k_cache: Tensor, v_cache: Tensor) -> None:
    _ops.kv_cache_write(k, v, slot_mapping, k_cache, v_cache)


@_kv_cache_write.register_fake
def _(k, v, slot_mapping, k_cache, v_cache):
    return None


@custom_op("emberserve::latent_cache_write", mutates_args=("cache",))
def _latent_cache_write(latent: Tensor, slot_mapping: Tensor, cache: Tensor) -> None:
    _ops.latent_cache_write(latent, slot_mapping, cache)


@_latent_cache_write.register_fake
def _(latent, slot_mapping, cache):
    return None


# ---- decode attention (attn/paged_triton.py:323-399, attn/mla_triton.py:119-182) ----------

@custom_op("emberserve::paged_attention_decode", mutates_args=())
def _paged_attention_decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_tables: Tensor,
                            context_lens: Tensor, scale: float, num_splits: int | None = None) -> Tensor:
    from .paged_decode import paged_attention_decode as impl
    return impl(q, k_cache, v_cache, block_tables, context_lens, scale, num_splits=num_splits)


@_paged_attention_decode.register_fake
def _(q, k_cache, v_cache, block_tables, context_lens, scale, num_splits=None):
    return _empty(q.shape, q)


@custom_op("emberserve::mla_decode", mutates_args=())
def _mla_decode(q_c: Tensor, q_pe: Tensor, latent_cache: Tensor, block_tables: Tensor, context_lens: Tensor,
                scale: float, kv_lora_rank: int, num_splits: int | None = None) -> Tensor:
    from .mla_decode import mla_decode as impl
    return impl((q_c, q_pe), latent_cache, block_tables, context_lens, scale, kv_lora_rank, num_splits=num_splits)


@_mla_decode.register_fake
def _(q_c, q_pe, latent_cache, block_tables, context_lens, scale, kv_lora_rank, num_splits=None):
    return _empty((q_c.shape[0], q_c.shape[1], kv_lora_rank), q_c)


# ---- the reference's calling conventions over the registered ops -------------------------

def rmsnorm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    return torch.ops.emberserve.rmsnorm(x, weight, eps)


def fused_add_rmsnorm(x: Tensor, residual: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    return torch.ops.emberserve.fused_add_rmsnorm(x, residual, weight, eps)


def rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor, positions: Tensor) -> tuple[Tensor, Tensor]:
    torch.ops.emberserve.rope(q, k, cos, sin, positions)
    return q, k


def silu_and_mul(x: Tensor) -> Tensor:
    return torch.ops.emberserve.silu_and_mul(x)


def embedding(ids: Tensor, weight: Tensor) -> Tensor:
    return torch.ops.emberserve.embedding(ids, weight)


def gate_up_silu(x: Tensor, weight: Tensor) -> Tensor:
    return torch.ops.emberserve.gate_up_silu(x, weight)


def moe_gate_up_silu(x: Tensor, w_gate_up: Tensor, sorted_ids: Tensor, block_expert: Tensor, num_valid: int,
                     top_k: int) -> Tensor:
    return torch.ops.emberserve.moe_gate_up_silu(x, w_gate_up, sorted_ids, block_expert, num_valid, top_k)


def moe_align(topk_ids: Tensor, num_experts: int, block_m: int = 16) -> tuple[Tensor, Tensor, int]:
    sorted_ids, block_expert = torch.ops.emberserve.moe_align(topk_ids, num_experts, block_m)
    return sorted_ids, block_expert, topk_ids.numel()


def fused_moe_gate_up(x: Tensor, topk_ids: Tensor, w_gate_up: Tensor) -> Tensor:
    return torch.ops.emberserve.fused_moe_gate_up(x, topk_ids, w_gate_up)


def qk_norm_rope(q: Tensor, k: Tensor, q_weight: Tensor, k_weight: Tensor, eps: float, cos: Tensor,
                 sin: Tensor, positions: Tensor) -> tuple[Tensor, Tensor]:
    torch.ops.emberserve.qk_norm_rope(q, k, q_weight, k_weight, eps, cos, sin, positions)
    return q, k


def mla_latent_rope(c: Tensor, k_pe: Tensor, q_pe: Tensor, weight: Tensor, eps: float, cos: Tensor,
                    sin: Tensor, positions: Tensor) -> tuple[Tensor, Tensor]:
    latent = torch.ops.emberserve.mla_latent_rope(c, k_pe, q_pe, weight, eps, cos, sin, positions)
    return q_pe, latent


def kv_cache_write(k: Tensor, v: Tensor, slot_mapping: Tensor, k_cache: Tensor, v_cache: Tensor) -> None:
    torch.ops.emberserve.kv_cache_write(k, v, slot_mapping, k_cache, v_cache)


def latent_cache_write(latent: Tensor, slot_mapping: Tensor, cache: Tensor) -> None:
    torch.ops.emberserve.latent_cache_write(latent, slot_mapping, cache)


def paged_attention_decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_tables: Tensor,
                           context_lens: Tensor, scale: float, num_splits: int | None = None) -> Tensor:
    return torch.ops.emberserve.paged_attention_decode(q, k_cache, v_cache, block_tables, context_lens, scale,
                                                       num_splits)


def mla_decode(q_c: Tensor, q_pe: Tensor, latent_cache: Tensor, block_tables: Tensor, context_lens: Tensor,
               scale: float, kv_lora_rank: int, num_splits: int | None = None) -> Tensor:
    return torch.ops.emberserve.mla_decode(q_c, q_pe, latent_cache, block_tables, context_lens, scale,
                                           kv_lora_rank, num_splits)
