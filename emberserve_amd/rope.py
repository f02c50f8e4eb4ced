"""Rotary position embedding tables and module (neox / rotate-half convention).

Drop-in for emberserve/model/rope.py:54-97: `RotaryEmbedding` builds fp32 cos/sin tables
`[max_position_embeddings, head_dim]` lazily on the device of the first positions it sees,
with both halves of a row equal (`cat(freqs, freqs)`), and `forward` hands them to
`ops.rope`. The gfx950 rope kernel reads only the first half of each row, which is exact
for these tables.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import ops


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """(x1, x2) -> (-x2, x1) over the halves of the last dim (rope.py:18-22)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotates x [N, H, D] by per-token cos/sin [N, D] in fp32, result in x.dtype
    (rope.py:25-33)."""
    xf = x.float()
    c = cos.float().unsqueeze(1)
    s = sin.float().unsqueeze(1)
    return (xf * c + rotate_half(xf) * s).to(x.dtype)


def llama3_scale_inv_freq(inv_freq: torch.Tensor, scaling: dict) -> torch.Tensor:
    """Llama 3.1 frequency scaling (rope.py:36-51): wavelengths longer than
    original_max_position_embeddings / low_freq_factor are slowed by `factor`, shorter than
    .../high_freq_factor are kept, and the band between is interpolated."""
    factor = float(scaling["factor"])
    lo = float(scaling["low_freq_factor"])
    hi = float(scaling["high_freq_factor"])
    ctx = float(scaling["original_max_position_embeddings"])
    wavelen = 2 * math.pi / inv_freq
    scaled = torch.where(wavelen > ctx / lo, inv_freq / factor, inv_freq)
    t = (ctx / wavelen - lo) / (hi - lo)
    blended = (1 - t) * scaled / factor + t * scaled
    in_band = ~(wavelen < ctx / hi) & ~(wavelen > ctx / lo)
    return torch.where(in_band, blended, scaled)


class RotaryEmbedding(nn.Module):
    """cos/sin tables `[max_position_embeddings, head_dim]` (fp32), built on first use on
    the positions' device; `forward(q, k, positions)` rotates q/k through `ops.rope`."""

    def __init__(self, head_dim: int, max_position_embeddings: int, base: float,
                 rope_scaling: dict | None = None) -> None:
        super().__init__()
        if head_dim % 2 != 0:
            raise AssertionError("head_dim must be even for RoPE")
        self.head_dim = head_dim
        self.max_position_embeddings = max_position_embeddings
        self.base = float(base)
        self.rope_scaling = rope_scaling
        self._cos: torch.Tensor | None = None
        self._sin: torch.Tensor | None = None

    def inv_freq(self, device: torch.device | None = None) -> torch.Tensor:
        """1 / base^(2i/D), i < D/2, fp32 (rope.py:68-75)."""
        exponent = torch.arange(0, self.head_dim, 2, dtype=torch.float32, device=device) / self.head_dim
        inv = 1.0 / (self.base ** exponent)
        sc = self.rope_scaling
        if sc and sc.get("rope_type", sc.get("type")) == "llama3":
            inv = llama3_scale_inv_freq(inv, sc)
        return inv

    def _build_tables(self, device: torch.device) -> None:
        pos = torch.arange(self.max_position_embeddings, dtype=torch.float32, device=device)
        freqs = torch.outer(pos, self.inv_freq(device))
        emb = torch.cat((freqs, freqs), dim=-1)
        self._cos = emb.cos()
        self._sin = emb.sin()

    def _ensure(self, device: torch.device) -> None:
        if self._cos is None or self._cos.device != device:
            self._build_tables(device)

    def tables(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin rows [N, D] (fp32) at int64 positions."""
        self._ensure(positions.device)
        return self._cos[positions], self._sin[positions]

    def full_tables(self, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        """The whole [max_pos, D] tables on `device` (what the fused ops take)."""
        self._ensure(device)
        return self._cos, self._sin

    def forward(self, q: torch.Tensor, k: torch.Tensor,
                positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        self._ensure(positions.device)
        return ops.rope(q, k, self._cos, self._sin, positions)
