"""PyTorch-eager forms of the fused ops: what CPU tensors run, and what GPU tensors run
when `EMBERSERVE_FUSED_OPS=0` asks for the unfused A/B path (emberserve/model/ops.py:15,
43-46). They carry the reference's `*_torch` names because the reference's own tests import
those names from the ops module (tests/test_fused_ops.py:30-31).

This is not the parity checker (that is `oracle/`, outside the package) and GPU tensors
never reach it unless the caller opts out explicitly.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def rmsnorm_torch(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """emberserve/model/ops.py:51-55."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * (xf * inv).to(x.dtype)


def fused_add_rmsnorm_torch(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                            eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/ops.py:58-63: the activation-dtype sum is the new residual."""
    new_residual = residual + x
    return rmsnorm_torch(new_residual, weight, eps), new_residual


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    """emberserve/model/ops.py:66-68: (x1, x2) -> (-x2, x1) over the last dim."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope_torch(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/ops.py:71-81; returns new tensors."""
    c = cos[positions].unsqueeze(1)
    s = sin[positions].unsqueeze(1)

    def _rot(t: torch.Tensor) -> torch.Tensor:
        tf = t.float()
        return (tf * c + _rotate_half(tf) * s).to(t.dtype)

    return _rot(q), _rot(k)


def silu_and_mul_torch(x: torch.Tensor) -> torch.Tensor:
    """emberserve/model/ops.py:84-87."""
    i = x.shape[-1] // 2
    return F.silu(x[..., :i]) * x[..., i:]


def embedding_torch(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """torch.nn.Embedding.forward (qwen2.py:182)."""
    return F.embedding(ids, weight)


def qk_norm_rope_torch(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                       k_weight: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor,
                       positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/qwen2.py:95-101: per-head rmsnorm of q and k, then rope."""
    n, hq, d = q.shape
    hk = k.shape[1]
    qn = rmsnorm_torch(q.reshape(n * hq, d), q_weight, eps).view(n, hq, d)
    kn = rmsnorm_torch(k.reshape(n * hk, d), k_weight, eps).view(n, hk, d)
    return rope_torch(qn, kn, cos, sin, positions)


def mla_latent_rope_torch(c: torch.Tensor, k_pe: torch.Tensor, q_pe: torch.Tensor,
                          weight: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor,
                          positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """emberserve/model/deepseek.py:126-133 (folded-rope branch): returns (q_pe, latent)."""
    cn = rmsnorm_torch(c, weight, eps)
    kp = k_pe.reshape(k_pe.shape[0], 1, -1)
    q_rot, k_rot = rope_torch(q_pe, kp, cos, sin, positions)
    return q_rot, torch.cat([cn, k_rot.squeeze(1)], dim=-1)


# The slot of a padding row (a step padded up to a captured token bucket): the cache writes
# skip it. Any other out-of-range slot is an error, as in index_copy_.
PAD_SLOT = -1


def kv_cache_write_torch(k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
                         k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    """emberserve/kv/cache.py:54-61 for one layer: index_copy_ of k and v into the flat
    [num_slots, Hkv, D] views of the caches."""
    slots = slot_mapping.to(device=k_cache.device, dtype=torch.long)
    flat = (-1, k.shape[1], k.shape[2])
    keep = slots != PAD_SLOT  # padding rows of a bucketed step are not stored
    if not bool(keep.all()):
        slots, k, v = slots[keep], k[keep], v[keep]
    k_cache.view(flat).index_copy_(0, slots, k.to(k_cache.dtype))
    v_cache.view(flat).index_copy_(0, slots, v.to(v_cache.dtype))


def latent_cache_write_torch(latent: torch.Tensor, slot_mapping: torch.Tensor, cache: torch.Tensor) -> None:
    """emberserve/kv/cache.py:152-157 for one layer."""
    slots = slot_mapping.to(device=cache.device, dtype=torch.long)
    keep = slots != PAD_SLOT
    if not bool(keep.all()):
        slots, latent = slots[keep], latent[keep]
    cache.view(-1, latent.shape[-1]).index_copy_(0, slots, latent.to(cache.dtype))
