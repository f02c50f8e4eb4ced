"""A whole decoder layer built from the drop-in modules, run with the fused HIP path on and
off (EMBERSERVE_FUSED_OPS), as the reference's tests/test_fused_ops_gpu.py:71-94 does for its
tiny model. The layer follows emberserve/model/qwen2.py:140-187 (Qwen3 flavour: qk-norm)
and deepseek.py:115-134 (MLA pre-attention): projections and attention are plain torch, the
elementwise ops are ours."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch import nn

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import layers, ops  # noqa: E402
from emberserve_amd.rope import RotaryEmbedding  # noqa: E402

DEV = "cuda"


class TinyQwen3(nn.Module):
    """embed -> [input norm -> qkv -> qk-norm + rope -> causal attention -> o_proj ->
    post norm (fused add) -> gate_up -> silu_and_mul -> down] x L -> final norm."""

    def __init__(self, vocab=512, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512, layers_n=2):
        super().__init__()
        self.h, self.kv, self.d = heads, kv_heads, head_dim
        self.embed = layers.Embedding(vocab, hidden)
        self.rot = RotaryEmbedding(head_dim, 4096, 1e6)
        self.blocks = nn.ModuleList()
        for _ in range(layers_n):
            b = nn.Module()
            b.inp = layers.RMSNorm(hidden, 1e-6)
            b.post = layers.RMSNorm(hidden, 1e-6)
            b.qkv = nn.Linear(hidden, (heads + 2 * kv_heads) * head_dim, bias=False)
            b.q_norm = layers.RMSNorm(head_dim, 1e-6)
            b.k_norm = layers.RMSNorm(head_dim, 1e-6)
            b.o = nn.Linear(heads * head_dim, hidden, bias=False)
            b.gate_up = nn.Linear(hidden, 2 * inter, bias=False)
            b.down = nn.Linear(inter, hidden, bias=False)
            self.blocks.append(b)
        self.norm = layers.RMSNorm(hidden, 1e-6)

    def forward(self, ids, positions):
        x = self.embed(ids)
        residual = None
        n = ids.shape[0]
        for b in self.blocks:
            if residual is None:
                residual, h = x, b.inp(x)
            else:
                h, residual = b.inp.forward_with_residual(x, residual)
            q, k, v = layers.qwen3_pre_attention_rope(b.qkv(h), self.h, self.kv, self.d, b.q_norm, b.k_norm,
                                                      self.rot, positions)
            rep = self.h // self.kv
            att = F.scaled_dot_product_attention(
                q.transpose(0, 1), k.repeat_interleave(rep, 1).transpose(0, 1),
                v.repeat_interleave(rep, 1).transpose(0, 1), is_causal=True)
            x = b.o(att.transpose(0, 1).reshape(n, -1))
            h, residual = b.post.forward_with_residual(x, residual)
            x = b.down(ops.silu_and_mul(b.gate_up(h)))
        out, _ = self.norm.forward_with_residual(x, residual)
        return out


def _init(model, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("weight") and p.dim() == 1:  # norm weights ~ N(1, 0.1)
                p.copy_(torch.randn(p.shape, generator=g) * 0.1 + 1)
            else:
                p.copy_(torch.randn(p.shape, generator=g) * (0.5 / p.shape[-1] ** 0.5))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qwen3_layers_fused_vs_eager(dtype, monkeypatch):
    model = TinyQwen3()
    _init(model, 0)
    model = model.to(DEV, dtype).eval()
    ids = torch.randint(0, 512, (40,), generator=torch.Generator().manual_seed(1)).to(DEV)
    positions = torch.arange(40, device=DEV)

    def run():
        with torch.inference_mode():
            return model(ids, positions).float().cpu()

    monkeypatch.setenv("EMBERSERVE_FUSED_OPS", "0")
    ref = run()
    monkeypatch.setenv("EMBERSERVE_FUSED_OPS", "1")
    fused = run()
    # the reference's own bar for this comparison: fp32 1e-4, half 5e-2 (test_fused_ops_gpu.py:93)
    tol = dict(atol=1e-4, rtol=1e-4) if dtype == torch.float32 else dict(atol=5e-2, rtol=1e-2)
    torch.testing.assert_close(fused, ref, **tol)


def test_mla_pre_attention_fused_vs_eager(monkeypatch):
    """deepseek.py:115-134 with the fused latent op, against the eager composition."""
    n, heads, nope, rope_d, rank, hidden = 24, 16, 128, 64, 512, 256
    g = torch.Generator().manual_seed(3)
    proj = nn.Linear(hidden, heads * (nope + rope_d) + rank + rope_d, bias=False)
    with torch.no_grad():
        proj.weight.copy_(torch.randn(proj.weight.shape, generator=g) * 0.05)
    proj = proj.to(DEV, torch.bfloat16)
    norm = layers.RMSNorm(rank, 1e-6).to(DEV, torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(rank, generator=g) * 0.1 + 1)
    rot = RotaryEmbedding(rope_d, 4096, 5e4)
    hidden_in = torch.randn(n, hidden, generator=g).to(DEV, torch.bfloat16)
    positions = torch.randint(0, 4096, (n,), generator=g).to(DEV)

    def run():
        with torch.inference_mode():
            q_nope, q_pe, latent = layers.mla_pre_attention_rope(proj(hidden_in), heads, nope, rope_d, rank, norm,
                                                                 rot, positions)
            return q_nope.float().cpu(), q_pe.float().cpu(), latent.float().cpu()

    monkeypatch.setenv("EMBERSERVE_FUSED_OPS", "0")
    ref = run()
    monkeypatch.setenv("EMBERSERVE_FUSED_OPS", "1")
    fused = run()
    torch.testing.assert_close(fused[0], ref[0], atol=0, rtol=0)  # q_nope untouched
    torch.testing.assert_close(fused[1], ref[1], atol=0, rtol=0)  # rope is bit-exact
    torch.testing.assert_close(fused[2], ref[2], atol=2e-2, rtol=1e-2)  # normed latent
