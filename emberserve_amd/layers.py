"""nn.Module drop-ins for the callers of the fused ops.

* `RMSNorm` mirrors emberserve/model/qwen2.py:30-45 (`forward`, `forward_with_residual`).
* `Embedding` is an nn.Embedding whose forward is the gfx950 gather; it keeps `.weight`
  [vocab, hidden] so weight tying (qwen2.py:204-205) and loading (weights.py:244) work.
* `qwen3_pre_attention_rope` and `mla_pre_attention_rope` are the fused forms of the
  elementwise tails of Qwen2Attention.pre_attention (qwen2.py:92-101) and
  MLAAttention.pre_attention (deepseek.py:119-133), taking the projection output.
"""

from __future__ import annotations

import torch
from torch import nn

from . import ops
from .rope import RotaryEmbedding


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.rmsnorm(x, self.weight, self.variance_epsilon)

    def forward_with_residual(self, x: torch.Tensor,
                              residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return ops.fused_add_rmsnorm(x, residual, self.weight, self.variance_epsilon)


class Embedding(nn.Embedding):
    """nn.Embedding with the bit-exact gfx950 row gather as its forward on GPU weights."""

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        if self.padding_idx is None and self.max_norm is None:
            return ops.embedding(ids, self.weight)
        return super().forward(ids)


class SwiGLUMLP(nn.Module):
    """Qwen2MLP (emberserve/model/qwen2.py:48-61) with the same parameters (`gate_up_proj`
    [2I, H] with gate rows first, `down_proj` [H, I], no biases), so checkpoints load
    unchanged; the forward runs gate_up_silu (the fused kernel at decode batches, the
    unfused pair otherwise). The tensor-parallel all-reduce after down_proj stays the
    caller's, as in the reference's `tpdist.all_reduce(...)`.

    `pack_weights()`, called once after the weights are loaded, adds a packed copy of
    gate_up_proj's weight (the same number of bytes again, outside the state dict) that the
    decode kernel streams faster; the copy is dropped when the weight tensor is replaced or
    modified in place, and the forward then reads the weight itself.
    `pack_weights(keep_weight=False)` instead replaces the weight by its packed copy: the
    module then holds one copy of the gate_up weight (gate_up_proj.weight becomes an empty
    tensor) and every batch runs on the packed copy, the decode kernel up to 64 tokens and
    the packed prefill GEMM above. Load checkpoints before dropping the weight."""

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.intermediate_size = intermediate_size
        self.gate_up_proj = nn.Linear(hidden_size, 2 * intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)
        self._packed = None
        self._packed_of = None  # (data_ptr, version) of the weight the copy was made from

    def _weight_key(self):
        w = self.gate_up_proj.weight
        return (w.data_ptr(), w._version)

    @torch.no_grad()
    def pack_weights(self, num_workgroups: int | None = None, keep_weight: bool = True) -> None:
        from .gate_up_silu import pack_gate_up_weight
        if self._packed_of == "only":
            raise RuntimeError("SwiGLUMLP.pack_weights: the unpacked weight was already dropped")
        w = self.gate_up_proj.weight
        self._packed = pack_gate_up_weight(w.detach(), num_workgroups)
        if keep_weight:
            self._packed_of = self._weight_key()
        else:
            self.gate_up_proj.weight = nn.Parameter(w.new_empty(0), requires_grad=False)
            self._packed_of = "only"  # w is freed with its last reference: stream-ordered after the packing

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from .gate_up_silu import gate_up_silu
        packed = self._packed
        if self._packed_of == "only":
            return self.down_proj(gate_up_silu(x, None, packed=packed))
        if packed is not None and self._packed_of != self._weight_key():
            self._packed = self._packed_of = packed = None
        return self.down_proj(gate_up_silu(x, self.gate_up_proj.weight, packed=packed))


def qwen3_pre_attention_rope(qkv: torch.Tensor, num_heads: int, num_kv_heads: int, head_dim: int,
                             q_norm: RMSNorm, k_norm: RMSNorm, rotary_emb: RotaryEmbedding,
                             positions: torch.Tensor):
    """`(q, k, v)` views of qkv [n, (H + 2 Hkv) * D] after Qwen3 qk-norm and rope, the
    norm and rope done in place in one kernel (qwen2.py:92-101)."""
    n = qkv.shape[0]
    q_size, kv_size = num_heads * head_dim, num_kv_heads * head_dim
    q, k, v = qkv.split([q_size, kv_size, kv_size], dim=-1)
    q = q.view(n, num_heads, head_dim)
    k = k.view(n, num_kv_heads, head_dim)
    v = v.view(n, num_kv_heads, head_dim)
    cos, sin = rotary_emb.full_tables(positions.device)
    q, k = ops.qk_norm_rope(q, k, q_norm.weight, k_norm.weight, q_norm.variance_epsilon, cos, sin,
                            positions)
    return q, k, v


def mla_pre_attention_rope(qkv_a: torch.Tensor, num_heads: int, qk_nope: int, qk_rope: int,
                           kv_lora_rank: int, kv_a_layernorm: RMSNorm, rotary_emb: RotaryEmbedding,
                           positions: torch.Tensor):
    """`(q_nope, q_pe, latent)` from the fused qkv_a projection [n, H*(Dn+Dr) + R + Dr]
    (deepseek.py:119-133 without q_lora, rope folded into the weights)."""
    n = qkv_a.shape[0]
    q_size = num_heads * (qk_nope + qk_rope)
    q, ckv = qkv_a.split([q_size, kv_lora_rank + qk_rope], dim=-1)
    q = q.view(n, num_heads, qk_nope + qk_rope)
    q_nope, q_pe = q.split([qk_nope, qk_rope], dim=-1)
    c, k_pe = ckv.split([kv_lora_rank, qk_rope], dim=-1)
    cos, sin = rotary_emb.full_tables(positions.device)
    q_pe, latent = ops.mla_latent_rope(c, k_pe, q_pe, kv_a_layernorm.weight,
                                       kv_a_layernorm.variance_epsilon, cos, sin, positions)
    return q_nope, q_pe, latent
