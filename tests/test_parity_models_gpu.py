"""Parity at the shapes of other models the reference's families cover, beyond the
configurations the main parity file mirrors: the hidden sizes, MLP widths and head layouts
of the Qwen2.5 / Qwen3 range (0.5B to 72B) and DeepSeek-V2/V3. Each shape takes the kernel
configuration its size selects (row-team widths, packs per lane, query-head passes), so
this sweeps those paths against the oracle with the tolerances of tests/test_parity_gpu.py
(bit-exact residual, rope and embedding; <= 2 ulp for the normalised and silu outputs).
The fused gate_up + silu_and_mul rows (Qwen3-4B, Qwen2.5-14B MLPs; DeepSeek-V3's expert
shape) use tests.helpers.check_gate_up's accumulation-error bound."""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib, ops  # noqa: E402
from oracle import inputs as gen  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402
from tests.helpers import assert_bitexact, assert_ulp  # noqa: E402

DEV = "cuda"
BF = torch.bfloat16
HIDDEN = [1536, 2048, 2560, 5120, 8192, 16384]           # 1.5B, 3B, Qwen3-4B, 32B, 72B, wide
INTER = [8960, 9728, 13824, 25600, 29568]                 # 1.5B, Qwen3-4B, 14B, Qwen3-32B, 72B
HEADS = [(12, 2, 128), (16, 8, 128), (40, 8, 128), (64, 8, 128), (128, 8, 128), (16, 2, 64)]


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield
    assert _lib.read_errors() == 0


@pytest.mark.parametrize("hidden", HIDDEN)
@pytest.mark.parametrize("rows", [3, 257])
def test_add_rmsnorm_model_hidden_sizes(hidden, rows):
    _say(f"add+rmsnorm hidden={hidden} rows={rows}")
    x, r, w = gen.add_rmsnorm_inputs(rows, hidden, BF, seed=hidden + rows)
    got, got_res = ops.fused_add_rmsnorm_hip(x.to(DEV), r.to(DEV), w.to(DEV), 1e-6)
    want, want_res = ref.fused_add_rmsnorm(x, r, w, 1e-6)
    assert_bitexact(got_res, want_res, "residual")
    assert_ulp(got, want, 2, "normed")
    assert_ulp(ops.rmsnorm_hip(x.to(DEV), w.to(DEV), 1e-6), ref.rmsnorm(x, w, 1e-6), 2, "rmsnorm")


@pytest.mark.parametrize("inter", INTER)
def test_silu_and_mul_model_widths(inter):
    _say(f"silu_and_mul inter={inter}")
    x = gen.silu_inputs(65, inter, BF, seed=inter)
    assert_ulp(ops.silu_and_mul_hip(x.to(DEV)), ref.silu_and_mul(x), 2, "silu_and_mul")


@pytest.mark.parametrize("heads", HEADS)
def test_rope_and_qk_norm_rope_model_heads(heads):
    """q/k as views of the fused qkv projection output at each head layout; rope bit-exact,
    qk-norm + rope within the norm's 2 ulp carried through the rotation (+1 ulp)."""
    hq, hk, d = heads
    n = 33
    _say(f"rope / qk-norm heads={heads}")
    qkv, qw, kw, pos = gen.qkv_inputs(n, hq, hk, d, 32768, BF, seed=hq * 7 + hk)
    cos, sin = ref.rope_tables(d, 32768, 1e6)
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    want_q, want_k = ref.rope(q, k, cos, sin, pos)
    qkv_d = qkv.to(DEV)
    qd = qkv_d[:, :hq * d].view(n, hq, d)
    kd = qkv_d[:, hq * d:(hq + hk) * d].view(n, hk, d)
    ops.rope_hip(qd, kd, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_bitexact(qd, want_q, "rope q")
    assert_bitexact(kd, want_k, "rope k")
    assert_bitexact(qkv_d[:, (hq + hk) * d:], qkv[:, (hq + hk) * d:], "v untouched")
    want_q, want_k = ref.qk_norm_rope(q, k, qw, kw, 1e-6, cos, sin, pos)
    qkv_d = qkv.to(DEV)
    qd = qkv_d[:, :hq * d].view(n, hq, d)
    kd = qkv_d[:, hq * d:(hq + hk) * d].view(n, hk, d)
    ops.qk_norm_rope_hip(qd, kd, qw.to(DEV), kw.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_ulp(qd, want_q, 3, "qk-norm q")
    assert_ulp(kd, want_k, 3, "qk-norm k")


@pytest.mark.parametrize("hidden", [1536, 5120, 8192])
def test_embedding_model_tables(hidden):
    _say(f"embedding hidden={hidden}")
    ids, w = gen.embedding_inputs(129, 32000, hidden, BF, seed=hidden)
    assert_bitexact(ops.embedding_hip(ids.to(DEV), w.to(DEV)), ref.embedding(ids, w), "embedding")


@pytest.mark.parametrize("heads", [16, 128])
def test_mla_latent_rope_deepseek_heads(heads):
    """DeepSeek-V2-Lite / Moonlight (16 heads) and V3 (128 heads): kv_lora_rank 512, rope 64,
    nope 128."""
    n = 17
    _say(f"mla latent heads={heads}")
    kv_a, q, w, pos = gen.mla_inputs(n, heads, 128, 64, 512, 4096, BF, seed=heads)
    cos, sin = ref.rope_tables(64, 4096, 5e4)
    c, k_pe = kv_a[:, :512], kv_a[:, 512:]
    q_pe = q[..., 128:]
    want_q, want_latent = ref.mla_latent_rope(c, k_pe, q_pe, w, 1e-6, cos, sin, pos)
    qd = q.to(DEV)
    kv_d = kv_a.to(DEV)
    got_q, got_latent = ops.mla_latent_rope_hip(kv_d[:, :512], kv_d[:, 512:], qd[..., 128:],
                                                w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_bitexact(got_q, want_q, "q_pe")
    assert_bitexact(qd[..., :128], q[..., :128], "q_nope untouched")
    assert_bitexact(got_latent[:, 512:], want_latent[:, 512:], "k_pe")
    assert_ulp(got_latent[:, :512], want_latent[:, :512], 2, "latent c")


@pytest.mark.parametrize("hidden,inter", [(2560, 9728), (5120, 13824)])   # Qwen3-4B, Qwen2.5-14B
@pytest.mark.parametrize("tokens", [1, 16])
def test_gate_up_silu_model_mlps(hidden, inter, tokens):
    """The fused gate_up + silu_and_mul at other models' MLP shapes, decode batches."""
    from emberserve_amd.gate_up_silu import gate_up_silu
    from tests.helpers import check_gate_up
    _say(f"gate_up_silu H={hidden} I={inter} T={tokens}")
    x, w = gen.gate_up_inputs(tokens, hidden, inter, BF, seed=hidden + tokens)
    got = gate_up_silu(x.to(DEV), w.to(DEV), fused=True)
    gu = (x.double() @ w.double().T).to(BF)
    absdot = x.double().abs() @ w.double().abs().T
    check_gate_up(got, ref.gate_up_silu(x, w), gu, absdot, hidden, f"H={hidden} T={tokens}")


def test_moe_gate_up_deepseek_v3_expert_shape():
    """DeepSeek-V3's routed-expert geometry (H 7168, I 2048, top-8), over 8 experts so the
    weights stay at 470 MB: every token uses every expert; 1 and 2 k splits."""
    from emberserve_amd.moe import fused_moe_gate_up
    from tests.helpers import check_gate_up
    h, inter, ne, k, n = 7168, 2048, 8, 8, 3
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(n, h, generator=g) * 0.5).to(BF)
    w = (torch.randn(ne, 2 * inter, h, generator=g) * 1.5 / h ** 0.5).to(BF)
    ids = torch.stack([torch.randperm(ne, generator=g) for _ in range(n)])
    rows = [(t, int(ids[t, c])) for t in range(n) for c in range(k)]
    want = ref.moe_gate_up_silu(x, ids, w)
    gu = torch.cat([(x[t:t + 1].double() @ w[e].double().T).to(BF) for t, e in rows])
    absdot = torch.cat([x[t:t + 1].double().abs() @ w[e].double().abs().T for t, e in rows])
    dx, dw, dids = x.to(DEV), w.to(DEV), ids.to(DEV)
    for splits in (1, 2):
        _say(f"moe gate_up DeepSeek-V3 shape splits={splits}")
        got = fused_moe_gate_up(dx, dids, dw, num_splits=splits)
        check_gate_up(got, want, gu, absdot, h, f"V3 splits={splits}", parts=0)
