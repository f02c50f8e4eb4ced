"""Parity of the gfx950 kernels (through ops.*_hip -> the C ABI) with the CPU oracle, on
identical seeded inputs.

Tolerances (stated per op; ulp of the storage dtype, fp32 accumulation on both sides):
  embedding                       bit-exact
  fused_add_rmsnorm residual      bit-exact
  rope (q, k)                     bit-exact (same fp32 expression, separately rounded)
  untouched columns (v, q_nope)   bit-exact
  rmsnorm / fused-add normed      bit-exact fp16/bf16 rows of <= 512 elements (a multiple
                                  of 32: the kernels sum in torch's CPU order); otherwise
                                  <= 2 ulp fp16/bf16, <= 16 ulp fp32
  silu_and_mul                    <= 2 ulp fp16/bf16, <= 16 ulp fp32
  MLA latent (normed c)           <= 2 ulp fp16/bf16, <= 16 ulp fp32
  qk_norm_rope                    bit-exact fp16/bf16 at head_dim 64/128/256 (the norm is
                                  bit-exact and the rotation is the same fp32 expression);
                                  fp32 and hosts whose torch sums in another order: the
                                  norm's budget (2 ulp fp16/bf16, 16 fp32) propagated through
                                  the exact rotation, + 1 ulp of the output
The cases mirror the reference's tests (tests/test_fused_ops.py, test_fused_ops_gpu.py:
same shapes and seeds) plus the BASELINE configurations.
"""

from __future__ import annotations

import os
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib, ops  # noqa: E402
from oracle import inputs as gen  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402
from tests.helpers import (ulp_diff, assert_bitexact, assert_rope_of_norm_close, assert_ulp,  # noqa: E402
                           norm_bitexact_expected)

DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
# fp32 outputs: the fp32 sum-of-squares order (torch's cascade vs the kernel's DPP tree)
# moves the variance by a few ulp at H ~ 7k; 16 ulp (~1e-6 relative) is still 80x tighter
# than the reference's own fp32 tolerance (rtol 1e-5, test_fused_ops_gpu.py:30).
ULP = {torch.float32: 16, torch.float16: 2, torch.bfloat16: 2}


def _rand(*shape, dtype, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield


# ---------------------------------------------------------------- rmsnorm / fused add

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hidden", [64, 128, 512, 896, 3584, 4096, 7168])
@pytest.mark.parametrize("rows", [1, 37, 300])
def test_rmsnorm(dtype, hidden, rows):
    _say(f"rmsnorm {dtype} rows={rows} hidden={hidden}")
    x = _rand(rows, hidden, dtype=dtype, seed=1, scale=3.0)
    w = _rand(hidden, dtype=dtype, seed=3, scale=0.3) + 1.0
    got = ops.rmsnorm_hip(x.to(DEV), w.to(DEV), 1e-6)
    assert got.dtype == dtype and got.shape == x.shape
    if norm_bitexact_expected(dtype, hidden):
        assert_bitexact(got, ref.rmsnorm(x, w, 1e-6), "rmsnorm (torch summation order)")
    else:
        assert_ulp(got, ref.rmsnorm(x, w, 1e-6), ULP[dtype], "rmsnorm")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hidden", [64, 896, 4096])
@pytest.mark.parametrize("rows", [1, 7, 37, 300])
def test_fused_add_rmsnorm(dtype, hidden, rows):
    _say(f"fused_add_rmsnorm {dtype} rows={rows} hidden={hidden}")
    x = _rand(rows, hidden, dtype=dtype, seed=3)
    r = _rand(rows, hidden, dtype=dtype, seed=4, scale=4.0)
    w = _rand(hidden, dtype=dtype, seed=5, scale=0.3) + 1.0
    xd, rd = x.to(DEV), r.to(DEV)
    got, got_res = ops.fused_add_rmsnorm_hip(xd, rd, w.to(DEV), 1e-6)
    want, want_res = ref.fused_add_rmsnorm(x, r, w, 1e-6)
    assert_bitexact(got_res, want_res, "residual")
    if norm_bitexact_expected(dtype, hidden):
        assert_bitexact(got, want, "normed (torch summation order)")
    else:
        assert_ulp(got, want, ULP[dtype], "normed")
    assert_bitexact(xd, x, "x unmodified")
    assert_bitexact(rd, r, "residual input unmodified")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rmsnorm_fp32_weight(dtype):
    """fp32 weights with half activations: out = round(fp32(y * w)), in x's dtype (the
    reference kernel's behaviour, ops_triton.py:31-33)."""
    x = _rand(33, 896, dtype=dtype, seed=11)
    w = _rand(896, dtype=torch.float32, seed=12, scale=0.1) + 1.0
    got = ops.rmsnorm_hip(x.to(DEV), w.to(DEV), 1e-6)
    want = ref.rmsnorm(x, w, 1e-6).to(dtype)
    assert got.dtype == dtype
    assert_ulp(got, want, 2, "rmsnorm fp32 weight")


def test_add_rmsnorm_config1():
    """[256, 896] fp16, w ~ N(1, 0.1), eps 1e-6."""
    x, r, w = gen.add_rmsnorm_inputs(256, 896, torch.float16)
    got, got_res = ops.fused_add_rmsnorm_hip(x.to(DEV), r.to(DEV), w.to(DEV), 1e-6)
    want, want_res = ref.fused_add_rmsnorm(x, r, w, 1e-6)
    assert_bitexact(got_res, want_res, "residual")
    assert_ulp(got, want, 2, "normed")


@pytest.mark.parametrize("tokens", [256, 8192])
def test_add_rmsnorm_config4c(tokens):
    """BASELINE config 4c: [T, 4096] bf16."""
    x, r, w = gen.add_rmsnorm_inputs(tokens, 4096, torch.bfloat16, seed=40)
    got, got_res = ops.fused_add_rmsnorm_hip(x.to(DEV), r.to(DEV), w.to(DEV), 1e-6)
    want, want_res = ref.fused_add_rmsnorm(x, r, w, 1e-6)
    assert_bitexact(got_res, want_res, "residual")
    assert_ulp(got, want, 2, "normed")


# ---------------------------------------------------------------- rope

def _tables(d, max_pos, theta):
    cos, sin = ref.rope_tables(d, max_pos, theta)
    return cos, sin


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("heads", [(14, 2), (4, 4), (3, 1), (28, 4), (32, 8)])
@pytest.mark.parametrize("d", [64, 128])
def test_rope_in_place_strided(dtype, heads, d):
    """q/k as strided views of one fused qkv buffer (test_fused_ops.py:65-86)."""
    h, hk = heads
    n = 50
    _say(f"rope {dtype} heads={heads} d={d}")
    cos, sin = _tables(d, 4096, 1e6)
    positions = torch.randint(0, 4096, (n,), generator=torch.Generator().manual_seed(9))
    positions[:6] = torch.tensor([0, 1, 5, 100, 4095, 17])
    qkv = _rand(n, (h + 2 * hk) * d, dtype=dtype, seed=6)
    q = qkv[:, :h * d].view(n, h, d)
    k = qkv[:, h * d:(h + hk) * d].view(n, hk, d)
    want_q, want_k = ref.rope(q, k, cos, sin, positions)
    qkv_d = qkv.to(DEV)
    qd = qkv_d[:, :h * d].view(n, h, d)
    kd = qkv_d[:, h * d:(h + hk) * d].view(n, hk, d)
    got_q, got_k = ops.rope_hip(qd, kd, cos.to(DEV), sin.to(DEV), positions.to(DEV))
    assert got_q.data_ptr() == qd.data_ptr() and got_k.data_ptr() == kd.data_ptr(), "in place"
    assert_bitexact(got_q, want_q, "q")
    assert_bitexact(got_k, want_k, "k")
    assert_bitexact(qkv_d[:, (h + hk) * d:], qkv[:, (h + hk) * d:], "v untouched")


@pytest.mark.parametrize("tokens", [256, 4096])
def test_rope_config2(tokens):
    """Qwen2.5-7B, q [T,28,128], k [T,4,128] bf16, theta 1e6,
    positions in [0, 32768)."""
    q, k, pos = gen.rope_inputs(tokens, 28, 4, 128, 32768, torch.bfloat16, seed=20)
    cos, sin = _tables(128, 32768, 1e6)
    want_q, want_k = ref.rope(q, k, cos, sin, pos)
    qd, kd = q.to(DEV), k.to(DEV)
    ops.rope_hip(qd, kd, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_bitexact(qd, want_q, "q")
    assert_bitexact(kd, want_k, "k")


def test_rope_position_out_of_range(monkeypatch):
    """A position past the table leaves its token untouched and, with index checks on,
    raises IndexError (torch's eager indexing raises too)."""
    d, n = 64, 8
    cos, sin = _tables(d, 128, 1e4)
    q = _rand(n, 2, d, dtype=torch.bfloat16, seed=1)
    k = _rand(n, 1, d, dtype=torch.bfloat16, seed=2)
    pos = torch.arange(n) * 7
    pos[3] = 128  # one past the end
    qd, kd = q.to(DEV), k.to(DEV)
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    with pytest.raises(IndexError):
        ops.rope_hip(qd, kd, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_bitexact(qd[3], q[3], "bad token untouched")
    good = torch.tensor([i for i in range(n) if i != 3])
    want_q, _ = ref.rope(q[good], k[good], cos, sin, pos[good])
    assert_bitexact(qd[good.to(DEV)], want_q, "good tokens rotated")


def test_rope_zero_tokens():
    q = torch.empty(0, 4, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(0, 1, 64, dtype=torch.bfloat16, device=DEV)
    cos, sin = _tables(64, 16, 1e4)
    got_q, got_k = ops.rope_hip(q, k, cos.to(DEV), sin.to(DEV), torch.empty(0, dtype=torch.int64, device=DEV))
    assert got_q.shape == (0, 4, 64) and got_k.shape == (0, 1, 64)


# ---------------------------------------------------------------- silu_and_mul

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("inter", [128, 4864, 18944])
@pytest.mark.parametrize("rows", [1, 3, 33])
def test_silu_and_mul(dtype, inter, rows):
    _say(f"silu {dtype} rows={rows} inter={inter}")
    x = _rand(rows, 2 * inter, dtype=dtype, seed=7, scale=2.0)
    got = ops.silu_and_mul_hip(x.to(DEV))
    assert got.shape == (rows, inter) and got.dtype == dtype
    assert_ulp(got, ref.silu_and_mul(x), ULP[dtype], "silu_and_mul")


@pytest.mark.parametrize("tokens", [1, 256])
def test_silu_config3(tokens):
    """Qwen2.5-7B, [T, 2*18944] fp16 ~ N(0, 2)."""
    x = gen.silu_inputs(tokens, 18944, torch.float16, seed=30)
    got = ops.silu_and_mul_hip(x.to(DEV))
    assert_ulp(got, ref.silu_and_mul(x), 2, "silu")


def test_silu_config3_full_sampled_rows():
    """T = 8192 at full size on the GPU; the op is row-wise, so 64 sampled rows checked
    against the oracle pin every row's code path."""
    x = gen.silu_inputs(8192, 18944, torch.float16, seed=31)
    got = ops.silu_and_mul_hip(x.to(DEV)).cpu()
    rows = torch.randint(0, 8192, (64,), generator=torch.Generator().manual_seed(5))
    rows[0], rows[1] = 0, 8191
    assert_ulp(got[rows], ref.silu_and_mul(x[rows]), 2, "silu sampled rows")


# ---------------------------------------------------------------- embedding

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hidden", [4096, 896, 7, 3])
def test_embedding_bitexact(dtype, hidden):
    ids, w = gen.embedding_inputs(300, 1000, hidden, dtype, seed=2)
    got = ops.embedding_hip(ids.to(DEV), w.to(DEV))
    assert_bitexact(got, ref.embedding(ids, w), "embedding")


@pytest.mark.parametrize("tokens", [256, 8192])
def test_embedding_config4a(tokens):
    """BASELINE config 4a: [151936, 4096] bf16 table, ids uniform over the vocabulary."""
    ids, w = gen.embedding_inputs(tokens, 151936, 4096, torch.bfloat16, seed=41)
    got = ops.embedding_hip(ids.to(DEV), w.to(DEV))
    assert_bitexact(got, ref.embedding(ids, w), "embedding")


def test_embedding_shapes_and_bad_ids(monkeypatch):
    w = _rand(50, 64, dtype=torch.float16, seed=3).to(DEV)
    ids = torch.tensor([[1, 2, 3], [4, 5, 49]], device=DEV)
    got = ops.embedding_hip(ids, w)
    assert got.shape == (2, 3, 64)
    assert_bitexact(got, w.cpu()[ids.cpu()], "2-D ids")
    bad = torch.tensor([0, 50, -1, 7], device=DEV)
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    with pytest.raises(IndexError):
        out = ops.embedding_hip(bad, w)
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "0")
    out = ops.embedding_hip(bad, w).cpu()
    assert (out[1] == 0).all() and (out[2] == 0).all(), "out-of-range ids give zero rows"
    assert_bitexact(out[0], w.cpu()[0], "row 0")
    assert_bitexact(out[3], w.cpu()[7], "row 3")
    assert _lib.read_errors(clear=True) & _lib.ERR_EMBED_ID


# ---------------------------------------------------------------- Qwen3 qk-norm + rope

def _check_qk(got_q, got_k, want_q, want_k, q, k, qw, kw, cos, sin, pos, norm_ulp):
    """qk-norm+rope: bit-exact where the kernel's norm sums in the oracle's order (half
    precision, head_dim 64/128/256); elsewhere the norm's ulp budget propagated through the
    (exact) rotation, which is the plain ulp bound where the rotation does not cancel."""
    n, hq, d = q.shape
    if norm_bitexact_expected(q.dtype, d):
        assert_bitexact(got_q, want_q, "q")
        assert_bitexact(got_k, want_k, "k")
        return
    hk = k.shape[1]
    half = d // 2
    yq = ref.rmsnorm(q.reshape(n * hq, d), qw, 1e-6).view(n, hq, d)
    yk = ref.rmsnorm(k.reshape(n * hk, d), kw, 1e-6).view(n, hk, d)
    c, s = cos[pos][:, :half], sin[pos][:, :half]
    assert_rope_of_norm_close(got_q, want_q, yq, c, s, norm_ulp, "q")
    assert_rope_of_norm_close(got_k, want_k, yk, c, s, norm_ulp, "k")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("heads,d", [((32, 8), 128), ((16, 8), 128), ((4, 2), 64), ((14, 2), 64)])
def test_qk_norm_rope_strided(dtype, heads, d):
    hq, hk = heads
    n = 40
    _say(f"qk_norm_rope {dtype} heads={heads} d={d}")
    qkv, qw, kw, pos = gen.qkv_inputs(n, hq, hk, d, 40960, dtype, seed=50)
    cos, sin = _tables(d, 40960, 1e6)
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    want_q, want_k = ref.qk_norm_rope(q, k, qw, kw, 1e-6, cos, sin, pos)
    qkv_d = qkv.to(DEV)
    qd = qkv_d[:, :hq * d].view(n, hq, d)
    kd = qkv_d[:, hq * d:(hq + hk) * d].view(n, hk, d)
    got_q, got_k = ops.qk_norm_rope_hip(qd, kd, qw.to(DEV), kw.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV),
                                        pos.to(DEV))
    assert got_q.data_ptr() == qd.data_ptr()
    _check_qk(got_q, got_k, want_q, want_k, q, k, qw, kw, cos, sin, pos, ULP[dtype])
    assert_bitexact(qkv_d[:, (hq + hk) * d:], qkv[:, (hq + hk) * d:], "v untouched")


@pytest.mark.parametrize("tokens", [256, 8192])
def test_qk_norm_rope_config4b(tokens):
    """BASELINE config 4b: Qwen3-8B, 32 q + 8 kv heads x 128 bf16, theta 1e6."""
    qkv, qw, kw, pos = gen.qkv_inputs(tokens, 32, 8, 128, 40960, torch.bfloat16, seed=42)
    cos, sin = _tables(128, 40960, 1e6)
    q = qkv[:, :4096].view(tokens, 32, 128)
    k = qkv[:, 4096:5120].view(tokens, 8, 128)
    want_q, want_k = ref.qk_norm_rope(q, k, qw, kw, 1e-6, cos, sin, pos)
    qkv_d = qkv.to(DEV)
    qd = qkv_d[:, :4096].view(tokens, 32, 128)
    kd = qkv_d[:, 4096:5120].view(tokens, 8, 128)
    ops.qk_norm_rope_hip(qd, kd, qw.to(DEV), kw.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    for name, got, want in (("q", qd, want_q), ("k", kd, want_k)):
        d = ulp_diff(got.cpu(), want)
        print(f"qk_norm_rope config 4b T={tokens} {name}: worst {int(d.max())} ulp, {int((d > 2).sum())} of "
              f"{d.numel()} elements above 2 ulp, {float((d == 0).float().mean()):.6f} bit-exact", flush=True)
    _check_qk(qd, kd, want_q, want_k, q, k, qw, kw, cos, sin, pos, 2)
    assert_bitexact(qkv_d[:, 5120:], qkv[:, 5120:], "v untouched")
    # Decomposition, which holds on any host: the output is the oracle's rope applied to the
    # kernel's own normed heads bit for bit (the unfused HIP rmsnorm gives those heads; the
    # fused kernel equals it, test_qk_norm_rope_equals_unfused_hip_chain), and every output
    # element off by more than 2 ulp has a normed input that differs from the oracle's.
    yq = ops.rmsnorm_hip(qkv.to(DEV)[:, :4096].reshape(tokens * 32, 128), qw.to(DEV), 1e-6).cpu()
    yk = ops.rmsnorm_hip(qkv.to(DEV)[:, 4096:5120].reshape(tokens * 8, 128), kw.to(DEV), 1e-6).cpu()
    rq, rk = ref.rope(yq.view(tokens, 32, 128), yk.view(tokens, 8, 128), cos, sin, pos)
    assert_bitexact(qd, rq, "q = rope(kernel-normed q)")
    assert_bitexact(kd, rk, "k = rope(kernel-normed k)")
    for name, y, w, got, want in (("q", yq, qw, qd, want_q), ("k", yk, kw, kd, want_k)):
        y_ref = ref.rmsnorm(qkv[:, :4096].reshape(tokens * 32, 128) if name == "q"
                            else qkv[:, 4096:5120].reshape(tokens * 8, 128), w, 1e-6)
        flips = ulp_diff(y, y_ref).view(got.shape)
        assert int(flips.max()) <= 1, f"{name}: a normed value off by {int(flips.max())} ulp"
        # an output element depends on its own and its rotation partner's normed value
        half = flips.shape[-1] // 2
        partner = torch.cat((flips[..., half:], flips[..., :half]), dim=-1)
        touched = (flips > 0) | (partner > 0)
        far = ulp_diff(got.cpu(), want).view(got.shape) > 2
        assert not bool((far & ~touched).any()), f"{name}: an output off by > 2 ulp with exact normed inputs"
        print(f"qk_norm_rope config 4b T={tokens} {name}: {int((flips > 0).sum())} normed values differ by 1 ulp",
              flush=True)


def test_qk_norm_rope_equals_unfused_hip_chain():
    """The fused kernel against the two HIP rmsnorm launches + the HIP rope launch that the
    reference's Qwen3 path runs (qwen2.py:95-101)."""
    n, hq, hk, d = 64, 32, 8, 128
    qkv, qw, kw, pos = gen.qkv_inputs(n, hq, hk, d, 40960, torch.bfloat16, seed=43)
    cos, sin = (t.to(DEV) for t in _tables(d, 40960, 1e6))
    a = qkv.to(DEV)
    b = a.clone()
    qa, ka = a[:, :4096].view(n, hq, d), a[:, 4096:5120].view(n, hk, d)
    ops.qk_norm_rope_hip(qa, ka, qw.to(DEV), kw.to(DEV), 1e-6, cos, sin, pos.to(DEV))
    qb = ops.rmsnorm_hip(b[:, :4096].reshape(n * hq, d), qw.to(DEV), 1e-6).view(n, hq, d)
    kb = ops.rmsnorm_hip(b[:, 4096:5120].reshape(n * hk, d), kw.to(DEV), 1e-6).view(n, hk, d)
    yq, yk = qb.cpu(), kb.cpu()
    ops.rope_hip(qb, kb, cos, sin, pos.to(DEV))
    # both paths sum the squares in the same order: the fused kernel's normed heads are the
    # unfused rmsnorm's, and the rotation is the same fp32 expression
    assert_bitexact(qa, qb, "q")
    assert_bitexact(ka, kb, "k")
    del yq, yk


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_qk_norm_rope_fp32_weights(dtype):
    """fp32 norm weights with half activations: y = round(fp32(round(x*inv) * w))."""
    n, hq, hk, d = 24, 8, 2, 128
    qkv, _, _, pos = gen.qkv_inputs(n, hq, hk, d, 4096, dtype, seed=70)
    qw = _rand(d, dtype=torch.float32, seed=71, scale=0.1) + 1
    kw = _rand(d, dtype=torch.float32, seed=72, scale=0.1) + 1
    cos, sin = _tables(d, 4096, 1e6)
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    yq = ref.rmsnorm(q.reshape(n * hq, d), qw, 1e-6).to(dtype).view(n, hq, d)  # rounded as the kernel does
    yk = ref.rmsnorm(k.reshape(n * hk, d), kw, 1e-6).to(dtype).view(n, hk, d)
    want_q, want_k = ref.rope(yq, yk, cos, sin, pos)
    qkv_d = qkv.to(DEV)
    gq, gk = ops.qk_norm_rope_hip(qkv_d[:, :hq * d].view(n, hq, d), qkv_d[:, hq * d:(hq + hk) * d].view(n, hk, d),
                                  qw.to(DEV), kw.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    c, s = cos[pos][:, :d // 2], sin[pos][:, :d // 2]
    assert_rope_of_norm_close(gq, want_q, yq, c, s, 2, "q")
    assert_rope_of_norm_close(gk, want_k, yk, c, s, 2, "k")


def test_rope_and_qk_norm_without_k_heads():
    """num_k_heads == 0 (a q-only rotation): the k pointer is never dereferenced."""
    n, h, d = 16, 4, 128
    q = _rand(n, h, d, dtype=torch.bfloat16, seed=73)
    cos, sin = _tables(d, 256, 1e6)
    pos = torch.randint(0, 256, (n,), generator=torch.Generator().manual_seed(74))
    empty_k = torch.empty(n, 0, d, dtype=torch.bfloat16)
    want_q, _ = ref.rope(q, empty_k, cos, sin, pos)
    qd = q.to(DEV)
    ops.rope_hip(qd, empty_k.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_bitexact(qd, want_q, "q only")
    w = _rand(d, dtype=torch.bfloat16, seed=75, scale=0.1) + 1
    want_q, _ = ref.qk_norm_rope(q, empty_k, w, w, 1e-6, cos, sin, pos)
    qd = q.to(DEV)
    ops.qk_norm_rope_hip(qd, empty_k.to(DEV), w.to(DEV), w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    yq = ref.rmsnorm(q.reshape(n * h, d), w, 1e-6).view(n, h, d)
    assert_rope_of_norm_close(qd, want_q, yq, cos[pos][:, :d // 2], sin[pos][:, :d // 2], 2, "q only, normed")


def test_rmsnorm_on_strided_latent_view():
    """kv_a_layernorm on the c view of the fused MLA projection (row stride 3648,
    deepseek.py:126): no copy, same result as on a contiguous copy."""
    buf = _rand(40, 3648, dtype=torch.bfloat16, seed=76)
    w = _rand(512, dtype=torch.bfloat16, seed=77, scale=0.1) + 1
    c = buf[:, 3072:3584]
    got = ops.rmsnorm_hip(buf.to(DEV)[:, 3072:3584], w.to(DEV), 1e-6)
    assert_ulp(got, ref.rmsnorm(c, w, 1e-6), 2, "strided c")


# ---------------------------------------------------------------- MLA latent path

def _mla_case(tokens, in_model, dtype=torch.bfloat16, seed=60, heads=16, nope=128, dr=64, rank=512):
    kv_a, q, w, pos = gen.mla_inputs(tokens, heads, nope, dr, rank, 8192, dtype, seed=seed)
    if in_model:  # the real layout: every piece a view of one [T, H*(Dn+Dr) + R + Dr] row
        qsize = heads * (nope + dr)
        buf = torch.cat([q.reshape(tokens, qsize), kv_a], dim=-1)
        return buf, w, pos, qsize
    return (q, kv_a), w, pos, None


@pytest.mark.parametrize("in_model", [False, True])
@pytest.mark.parametrize("tokens", [1, 64, 8192])
def test_mla_latent_rope_config5(in_model, tokens):
    """Moonlight / DeepSeek-V3 shape, kv_a [T, 576], q [T, 16, 192] bf16,
    theta 5e4, positions in [0, 8192). Both the separate-tensor and the in-model (strided
    views of one buffer) layouts."""
    heads, nope, dr, rank = 16, 128, 64, 512
    data, w, pos, qsize = _mla_case(tokens, in_model)
    cos, sin = _tables(dr, 8192, 5e4)

    def views(q_buf, kv):
        q = q_buf.view(tokens, heads, nope + dr)
        return q[..., :nope], q[..., nope:], kv[:, :rank], kv[:, rank:]

    if in_model:
        buf = data
        q_nope, q_pe, c, k_pe = views(buf[:, :qsize], buf[:, qsize:])
        buf_d = buf.to(DEV)
        q_nope_d, q_pe_d, c_d, k_pe_d = views(buf_d[:, :qsize], buf_d[:, qsize:])
    else:
        q, kv_a = data
        q_nope, q_pe, c, k_pe = views(q, kv_a)
        q_dev, kv_dev = q.to(DEV), kv_a.to(DEV)
        q_nope_d, q_pe_d, c_d, k_pe_d = views(q_dev, kv_dev)
    want_q_pe, want_lat = ref.mla_latent_rope(c, k_pe, q_pe, w, 1e-6, cos, sin, pos)
    c_before, kpe_before = c.clone(), k_pe.clone()
    got_q_pe, lat = ops.mla_latent_rope_hip(c_d, k_pe_d, q_pe_d, w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV),
                                            pos.to(DEV))
    assert lat.shape == (tokens, rank + dr)
    assert got_q_pe.data_ptr() == q_pe_d.data_ptr()
    assert_ulp(lat[:, :rank], want_lat[:, :rank], 2, "latent c")
    assert_bitexact(lat[:, rank:], want_lat[:, rank:], "latent k_pe (rope)")
    assert_bitexact(got_q_pe, want_q_pe, "q_pe (rope)")
    assert_bitexact(q_nope_d, q_nope, "q_nope untouched")
    assert_bitexact(c_d, c_before, "c unmodified")
    assert_bitexact(k_pe_d, kpe_before, "k_pe unmodified")


def test_mla_fp32_weight():
    kv_a, q, _, pos = gen.mla_inputs(30, 16, 128, 64, 512, 8192, torch.bfloat16, seed=78)
    w = _rand(512, dtype=torch.float32, seed=79, scale=0.1) + 1
    cos, sin = _tables(64, 8192, 5e4)
    qv = q.view(30, 16, 192)
    want_q_pe, want_lat = ref.mla_latent_rope(kv_a[:, :512], kv_a[:, 512:], qv[..., 128:], w, 1e-6, cos, sin, pos)
    kd, qd = kv_a.to(DEV), q.to(DEV)
    got_q_pe, lat = ops.mla_latent_rope_hip(kd[:, :512], kd[:, 512:], qd[..., 128:], w.to(DEV), 1e-6, cos.to(DEV),
                                            sin.to(DEV), pos.to(DEV))
    # fp32 weight: the oracle's product is fp32 (torch promotion); the kernel rounds it once
    assert_ulp(lat[:, :512], want_lat[:, :512].to(torch.bfloat16), 2, "latent c, fp32 weight")
    assert_bitexact(lat[:, 512:], want_lat[:, 512:].to(torch.bfloat16), "latent k_pe")
    assert_bitexact(got_q_pe, want_q_pe, "q_pe")


def test_mla_position_out_of_range(monkeypatch):
    kv_a, q, w, pos = gen.mla_inputs(8, 4, 32, 64, 128, 64, torch.bfloat16, seed=80)
    pos[5] = 64
    cos, sin = _tables(64, 64, 1e4)
    kd, qd = kv_a.to(DEV), q.to(DEV)
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    with pytest.raises(IndexError):
        ops.mla_latent_rope_hip(kd[:, :128], kd[:, 128:], qd[..., 32:], w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV),
                                pos.to(DEV))
    assert_bitexact(qd[5], q[5], "bad token's q untouched")


@pytest.mark.parametrize("dtype", DTYPES)
def test_mla_small_shapes(dtype):
    """A DeepSeek-V2-Lite-like shape (kv_lora_rank 512, Dr 64, 16 heads) and a tiny one
    (rank 64, Dr 16, 3 heads) in every dtype."""
    for heads, nope, dr, rank in [(16, 128, 64, 512), (3, 32, 16, 64)]:
        kv_a, q, w, pos = gen.mla_inputs(20, heads, nope, dr, rank, 512, dtype, seed=61)
        cos, sin = _tables(dr, 512, 1e4)
        qv = q.view(20, heads, nope + dr)
        want_q_pe, want_lat = ref.mla_latent_rope(kv_a[:, :rank], kv_a[:, rank:], qv[..., nope:], w, 1e-6,
                                                  cos, sin, pos)
        qd, kd = q.to(DEV), kv_a.to(DEV)
        got_q_pe, lat = ops.mla_latent_rope_hip(kd[:, :rank], kd[:, rank:], qd[..., nope:], w.to(DEV), 1e-6,
                                                cos.to(DEV), sin.to(DEV), pos.to(DEV))
        assert_ulp(lat, want_lat, ULP[dtype], f"latent {heads},{rank}")
        assert_bitexact(got_q_pe, want_q_pe, "q_pe")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads,dr,rank", [
    (3, 32, 64),      # one-token kernel: 4-lane head groups, one partly filled query pass
    (5, 64, 256),     # 40 of 64 lanes in the query pass
    (32, 64, 512),    # four query passes
    (8, 128, 1024),   # 16-lane head groups, two latent packs per lane
    (64, 64, 512),    # eight query passes: the task-split kernel
    (16, 64, 1536),   # three latent packs per lane: the task-split kernel
])
def test_mla_kernel_shapes(dtype, heads, dr, rank):
    """Every shape class of the one-token MLA kernel (head-group widths 4/8/16 lanes, 1-4
    query passes, 1-2 latent packs) and the shapes routed to the task-split kernel, with a
    bad position in the batch."""
    n = 37
    kv_a, q, w, pos = gen.mla_inputs(n, heads, 16, dr, rank, 300, dtype, seed=81)
    cos, sin = _tables(dr, 300, 1e4)
    qv = q.view(n, heads, 16 + dr)
    want_q_pe, want_lat = ref.mla_latent_rope(kv_a[:, :rank], kv_a[:, rank:], qv[..., 16:], w, 1e-6, cos, sin, pos)
    pos[11] = 300  # out of range: latent key zeroed, q_pe untouched (the oracle's row 11 is not used)
    qd, kd = q.to(DEV), kv_a.to(DEV)
    got_q_pe, lat = ops.mla_latent_rope_hip(kd[:, :rank], kd[:, rank:], qd.view(n, heads, 16 + dr)[..., 16:],
                                            w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    good = torch.ones(n, dtype=torch.bool)
    good[11] = False
    assert_ulp(lat[good, :rank], want_lat[good, :rank], ULP[dtype], "latent c")
    assert_bitexact(lat[good, rank:], want_lat[good, rank:], "latent k_pe")
    assert_bitexact(got_q_pe[good], want_q_pe[good], "q_pe")
    assert_bitexact(got_q_pe[11], qv[11, :, 16:], "bad position: q_pe untouched")
    assert_bitexact(lat[11, rank:], torch.zeros(dr, dtype=dtype), "bad position: latent key zeroed")
    assert_bitexact(qd.view(n, heads, 16 + dr)[..., :16], qv[..., :16], "q_nope untouched")


# ---------------------------------------------------------------- scalar (unaligned) paths

def test_unaligned_views_take_the_scalar_kernels():
    """Views offset by one element are not 16-byte aligned: the library must still give
    the same results (its scalar kernels)."""
    dt = torch.bfloat16
    # rmsnorm / fused add on [rows, 895] slices of a wider buffer
    base = _rand(9, 900, dtype=dt, seed=1)
    res = _rand(9, 900, dtype=dt, seed=2)
    w = _rand(895, dtype=dt, seed=3, scale=0.1) + 1
    x, r = base[:, 1:896], res[:, 3:898]
    got, got_res = ops.fused_add_rmsnorm_hip(base.to(DEV)[:, 1:896], res.to(DEV)[:, 3:898], w.to(DEV), 1e-6)
    want, want_res = ref.fused_add_rmsnorm(x, r, w, 1e-6)
    assert_bitexact(got_res, want_res, "residual")
    assert_ulp(got, want, 2, "normed")
    # silu on an odd intermediate size
    xs = _rand(5, 2 * 37, dtype=dt, seed=4, scale=2.0)
    assert_ulp(ops.silu_and_mul_hip(xs.to(DEV)), ref.silu_and_mul(xs), 2, "silu odd")
    # rope with head_dim 96 (J not a power of two) and an odd head offset
    n, h, hk, d = 10, 3, 1, 96
    cos, sin = _tables(d, 256, 1e4)
    pos = torch.randint(0, 256, (n,), generator=torch.Generator().manual_seed(3))
    qkv = _rand(n, 1 + (h + hk) * d, dtype=dt, seed=5)
    q, k = qkv[:, 1:1 + h * d].view(n, h, d), qkv[:, 1 + h * d:].view(n, hk, d)
    want_q, want_k = ref.rope(q, k, cos, sin, pos)
    dq = qkv.to(DEV)
    gq, gk = ops.rope_hip(dq[:, 1:1 + h * d].view(n, h, d), dq[:, 1 + h * d:].view(n, hk, d), cos.to(DEV),
                          sin.to(DEV), pos.to(DEV))
    assert_bitexact(gq, want_q, "rope q scalar")
    assert_bitexact(gk, want_k, "rope k scalar")
    # qk-norm rope scalar path
    qw = _rand(d, dtype=dt, seed=6, scale=0.1) + 1
    kw = _rand(d, dtype=dt, seed=7, scale=0.1) + 1
    want_q, want_k = ref.qk_norm_rope(q, k, qw, kw, 1e-6, cos, sin, pos)
    dq = qkv.to(DEV)
    gq, gk = ops.qk_norm_rope_hip(dq[:, 1:1 + h * d].view(n, h, d), dq[:, 1 + h * d:].view(n, hk, d),
                                  qw.to(DEV), kw.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV), pos.to(DEV))
    assert_ulp(gq, want_q, 2, "qk-norm q scalar")
    assert_ulp(gk, want_k, 2, "qk-norm k scalar")
    # MLA scalar path (rank 100 is not a multiple of 8)
    kv_a, qm, wm, pm = gen.mla_inputs(6, 2, 8, 16, 100, 64, dt, seed=8)
    cos, sin = _tables(16, 64, 1e4)
    qv = qm.view(6, 2, 24)
    want_q_pe, want_lat = ref.mla_latent_rope(kv_a[:, :100], kv_a[:, 100:], qv[..., 8:], wm, 1e-6, cos, sin, pm)
    kd, qd = kv_a.to(DEV), qm.to(DEV)
    got_q_pe, lat = ops.mla_latent_rope_hip(kd[:, :100], kd[:, 100:], qd[..., 8:], wm.to(DEV), 1e-6, cos.to(DEV),
                                            sin.to(DEV), pm.to(DEV))
    assert_ulp(lat, want_lat, 2, "mla latent scalar")
    assert_bitexact(got_q_pe, want_q_pe, "mla q_pe scalar")


# ---------------------------------------------------------------- dispatch, loading, graphs

def test_dispatch_runs_the_hip_library(monkeypatch):
    """With the fused path on, GPU tensors never reach the eager functions, and the
    process has libember_ops.so mapped."""
    def boom(*a, **k):
        raise AssertionError("eager path used on a GPU tensor")

    for name in ["rmsnorm_torch", "fused_add_rmsnorm_torch", "rope_torch", "silu_and_mul_torch",
                 "embedding_torch", "qk_norm_rope_torch", "mla_latent_rope_torch"]:
        monkeypatch.setattr(ops, name, boom)
    monkeypatch.setenv("EMBERSERVE_FUSED_OPS", "1")
    x = torch.randn(4, 64, device=DEV, dtype=torch.float16)
    w = torch.ones(64, device=DEV, dtype=torch.float16)
    ops.rmsnorm(x, w, 1e-6)
    ops.fused_add_rmsnorm(x, x, w, 1e-6)
    ops.silu_and_mul(x)
    cos, sin = (t.to(DEV) for t in _tables(16, 32, 1e4))
    ops.rope(x.clone().view(4, 4, 16), x.clone().view(4, 4, 16)[:, :1], cos, sin, torch.arange(4, device=DEV))
    ops.embedding(torch.arange(3, device=DEV), w.view(4, 16))
    torch.cuda.synchronize()
    maps = open("/proc/self/maps").read()
    assert "libember_ops.so" in maps


def test_fused_ops_off_uses_eager(monkeypatch):
    monkeypatch.setenv("EMBERSERVE_FUSED_OPS", "0")
    x = torch.randn(4, 64, device=DEV)
    assert not ops.fused_enabled(x)
    torch.testing.assert_close(ops.rmsnorm(x, torch.ones(64, device=DEV), 1e-6),
                               ops.rmsnorm_torch(x, torch.ones(64, device=DEV), 1e-6))


def test_graph_capture_replays_match_eager():
    """A per-layer chain recorded in a torch.cuda.graph: every replay (inputs changed in
    between, eager work and syncs interleaved) equals the eager launches."""
    n, hq, hk, d, hidden, inter = 96, 8, 2, 128, 1024, 1536
    dt = torch.bfloat16
    cos, sin = (t.to(DEV) for t in _tables(d, 4096, 1e6))
    s_x = torch.empty(n, hidden, dtype=dt, device=DEV)
    s_r = torch.empty(n, hidden, dtype=dt, device=DEV)
    s_qkv = torch.empty(n, (hq + 2 * hk) * d, dtype=dt, device=DEV)
    s_gu = torch.empty(n, 2 * inter, dtype=dt, device=DEV)
    s_pos = torch.empty(n, dtype=torch.int64, device=DEV)
    w = torch.randn(hidden, dtype=dt, device=DEV) * 0.1 + 1
    qw = torch.randn(d, dtype=dt, device=DEV) * 0.1 + 1
    kw = torch.randn(d, dtype=dt, device=DEV) * 0.1 + 1

    def chain():
        normed, res = ops.fused_add_rmsnorm_hip(s_x, s_r, w, 1e-6)
        q = s_qkv[:, :hq * d].view(n, hq, d)
        k = s_qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
        ops.qk_norm_rope_hip(q, k, qw, kw, 1e-6, cos, sin, s_pos)
        act = ops.silu_and_mul_hip(s_gu)
        return normed, res, act

    def fill(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        s_x.copy_(torch.randn(n, hidden, generator=g, device=DEV).to(dt))
        s_r.copy_(torch.randn(n, hidden, generator=g, device=DEV).to(dt))
        s_qkv.copy_(torch.randn(s_qkv.shape, generator=g, device=DEV).to(dt))
        s_gu.copy_(torch.randn(s_gu.shape, generator=g, device=DEV).to(dt))
        s_pos.copy_(torch.randint(0, 4096, (n,), generator=g, device=DEV))

    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain()  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = chain()
    for seed in range(1, 5):
        fill(seed)
        qkv_before = s_qkv.clone()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs] + [s_qkv.clone()]
        s_qkv.copy_(qkv_before)
        want = list(chain()) + [s_qkv.clone()]
        torch.cuda.synchronize()
        for g, wv, name in zip(got, want, ["normed", "residual", "act", "qkv"]):
            assert_bitexact(g, wv, f"replay {seed} {name}")


def test_graph_capture_multi_layer_with_kv_write():
    """Three decoder layers of the Qwen3-shaped elementwise kernels (input add+RMSNorm,
    qk-norm + rope + paged KV write, post-attention add+RMSNorm, silu_and_mul) recorded in
    one torch.cuda.graph, as a full-step graph runner records them. Each replay (new inputs,
    new slots, eager work and syncs in between) equals the eager launches bit for bit,
    KV caches included."""
    n, hq, hk, d, hidden, inter, layers = 24, 8, 2, 128, 512, 768, 3
    blocks, bs = 16, 16
    dt = torch.bfloat16
    cos, sin = (t.to(DEV) for t in _tables(d, 4096, 1e6))
    bufs = {name: torch.empty(shape, dtype=dt, device=DEV) for name, shape in
            [("x", (n, hidden)), ("r", (n, hidden)), ("qkv", (layers, n, (hq + 2 * hk) * d)),
             ("gu", (n, 2 * inter))]}
    pos = torch.empty(n, dtype=torch.int64, device=DEV)
    slots = torch.empty(n, dtype=torch.int64, device=DEV)
    kc = torch.zeros(layers, blocks, bs, hk, d, dtype=dt, device=DEV)
    vc = torch.zeros_like(kc)
    w = torch.randn(hidden, dtype=dt, device=DEV) * 0.1 + 1
    qw = torch.randn(d, dtype=dt, device=DEV) * 0.1 + 1
    kw = torch.randn(d, dtype=dt, device=DEV) * 0.1 + 1

    def step(b, kcache, vcache):
        outs = []
        for layer in range(layers):
            normed, res = ops.fused_add_rmsnorm_hip(b["x"], b["r"], w, 1e-6)
            qkv = b["qkv"][layer]
            ops.rope_kv_cache_hip(qkv[:, :hq * d].view(n, hq, d), qkv[:, hq * d:(hq + hk) * d].view(n, hk, d),
                                  qkv[:, (hq + hk) * d:].view(n, hk, d), cos, sin, pos, slots, kcache[layer],
                                  vcache[layer], qw, kw, 1e-6)
            normed2, res2 = ops.fused_add_rmsnorm_hip(normed, res, w, 1e-6)
            outs += [normed2, res2, ops.silu_and_mul_hip(b["gu"])]
        return outs

    def fill(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        for t in bufs.values():
            t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(dt))
        pos.copy_(torch.randint(0, 4096, (n,), generator=g, device=DEV))
        slots.copy_(torch.randperm(blocks * bs, generator=g, device=DEV)[:n])

    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(bufs, kc, vc)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step(bufs, kc, vc)
    for seed in range(1, 4):
        fill(seed)
        before = {k: v.clone() for k, v in bufs.items()}
        kc_e, vc_e = kc.clone(), vc.clone()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs] + [bufs["qkv"].clone(), kc.clone(), vc.clone()]
        want = step(before, kc_e, vc_e) + [before["qkv"], kc_e, vc_e]
        torch.cuda.synchronize()
        names = [f"layer {i // 3} {('normed', 'residual', 'act')[i % 3]}" for i in range(3 * layers)]
        for g, wv, name in zip(got, want, names + ["qkv (q/k rotated in place)", "k cache", "v cache"]):
            assert_bitexact(g, wv, f"replay {seed} {name}")


# ---------------------------------------------------------------- paged KV-cache writes

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hk,d", [(8, 128), (4, 128), (2, 64), (1, 6)])
def test_kv_cache_write_bitexact(dtype, hk, d):
    """k, v as views of a fused qkv buffer scattered into [blocks, block_size, Hkv, D]
    caches (kv/cache.py:54-61); unwritten slots keep their contents. (1, 6) takes the
    scalar path (12-byte rows)."""
    n, hq, blocks, bs = 100, 4, 16, 16
    _say(f"kv_cache_write {dtype} hk={hk} d={d}")
    g = torch.Generator().manual_seed(90)
    qkv = _rand(n, (hq + 2 * hk) * d, dtype=dtype, seed=91)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    v = qkv[:, (hq + hk) * d:].view(n, hk, d)
    slots = torch.randperm(blocks * bs, generator=g)[:n]
    kc0 = _rand(blocks, bs, hk, d, dtype=dtype, seed=92)  # stale contents must survive where unwritten
    vc0 = _rand(blocks, bs, hk, d, dtype=dtype, seed=93)
    want_k, want_v = kc0.clone(), vc0.clone()
    ref.kv_cache_write(k, v, slots, want_k, want_v)
    qkv_d = qkv.to(DEV)
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    ops.kv_cache_write_hip(qkv_d[:, hq * d:(hq + hk) * d].view(n, hk, d), qkv_d[:, (hq + hk) * d:].view(n, hk, d),
                           slots.to(DEV), kc, vc)
    assert_bitexact(kc, want_k, "k cache")
    assert_bitexact(vc, want_v, "v cache")


def test_kv_cache_write_qwen3_prefill_and_bad_slot(monkeypatch):
    """Qwen3-8B prefill shape (8 kv heads x 128, T = 8192) into a 1024-block cache, then a
    slot past the end: skipped, and IndexError under EMBERSERVE_CHECK_INDICES=1."""
    n, hk, d, blocks, bs = 8192, 8, 128, 1024, 16
    g = torch.Generator().manual_seed(94)
    k = _rand(n, hk, d, dtype=torch.bfloat16, seed=95)
    v = _rand(n, hk, d, dtype=torch.bfloat16, seed=96)
    slots = torch.randperm(blocks * bs, generator=g)[:n]
    want_k = torch.zeros(blocks, bs, hk, d, dtype=torch.bfloat16)
    want_v = torch.zeros_like(want_k)
    ref.kv_cache_write(k, v, slots, want_k, want_v)
    kc = torch.zeros(blocks, bs, hk, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    ops.kv_cache_write_hip(k.to(DEV), v.to(DEV), slots.to(DEV), kc, vc)
    assert_bitexact(kc, want_k, "k cache")
    assert_bitexact(vc, want_v, "v cache")
    bad = slots[:4].clone()
    bad[2] = blocks * bs
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    kc2 = torch.zeros_like(kc)
    with pytest.raises(IndexError):
        ops.kv_cache_write_hip(k[:4].to(DEV), v[:4].to(DEV), bad.to(DEV), kc2, torch.zeros_like(kc2))
    assert int(torch.count_nonzero(kc2.view(-1, hk, d)[bad[[0, 1, 3]].to(DEV)].float() == 0)) < 3 * hk * d


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_latent_cache_write_bitexact(dtype):
    """MLA latent rows [T, 576] (and a view with row stride 3648) into [blocks, bs, 576]."""
    n, dim, blocks, bs = 500, 576, 64, 16
    g = torch.Generator().manual_seed(97)
    buf = _rand(n, 3648, dtype=dtype, seed=98)
    slots = torch.randperm(blocks * bs, generator=g)[:n]
    for lat, lat_d in [(buf[:, 3072:], buf.to(DEV)[:, 3072:]), (buf[:, :dim].contiguous(), buf[:, :dim].contiguous().to(DEV))]:
        want = torch.zeros(blocks, bs, dim, dtype=dtype)
        ref.latent_cache_write(lat, slots, want)
        cache = torch.zeros(blocks, bs, dim, dtype=dtype, device=DEV)
        ops.latent_cache_write_hip(lat_d, slots.to(DEV), cache)
        assert_bitexact(cache, want, "latent cache")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("heads,d", [((32, 8), 128), ((28, 4), 128), ((14, 2), 64)])
def test_rope_kv_cache_fused(dtype, norm, heads, d):
    """rope (+ Qwen3 qk-norm) then PagedKVCache.write, in one kernel: q/k in place as the
    unfused ops leave them, the cache holds exactly the in-place k rows and the v rows."""
    hq, hk = heads
    n, blocks, bs = 64, 16, 16
    _say(f"rope_kv_cache {dtype} norm={norm} heads={heads} d={d}")
    qkv, qw, kw, pos = gen.qkv_inputs(n, hq, hk, d, 4096, dtype, seed=100)
    cos, sin = _tables(d, 4096, 1e6)
    slots = torch.randperm(blocks * bs, generator=torch.Generator().manual_seed(101))[:n]
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    v = qkv[:, (hq + hk) * d:].view(n, hk, d)
    if norm:
        want_q, want_k = ref.qk_norm_rope(q, k, qw, kw, 1e-6, cos, sin, pos)
    else:
        want_q, want_k = ref.rope(q, k, cos, sin, pos)
    want_kc = torch.zeros(blocks, bs, hk, d, dtype=dtype)
    want_vc = torch.zeros_like(want_kc)
    ref.kv_cache_write(want_k, v, slots, want_kc, want_vc)

    qkv_d = qkv.to(DEV)
    qd = qkv_d[:, :hq * d].view(n, hq, d)
    kd = qkv_d[:, hq * d:(hq + hk) * d].view(n, hk, d)
    vd = qkv_d[:, (hq + hk) * d:].view(n, hk, d)
    kc = torch.zeros(blocks, bs, hk, d, dtype=dtype, device=DEV)
    vc = torch.zeros_like(kc)
    ops.rope_kv_cache_hip(qd, kd, vd, cos.to(DEV), sin.to(DEV), pos.to(DEV), slots.to(DEV), kc, vc,
                          qw.to(DEV) if norm else None, kw.to(DEV) if norm else None, 1e-6)
    if norm:
        _check_qk(qd, kd, want_q, want_k, q, k, qw, kw, cos, sin, pos, ULP[dtype])
    else:
        assert_bitexact(qd, want_q, "q")
        assert_bitexact(kd, want_k, "k")
    # the cache holds exactly the in-place k rows (same bits), and exactly v
    assert_bitexact(kc.view(-1, hk, d)[slots.to(DEV)], kd, "k cache rows == rotated k")
    assert_bitexact(vc, want_vc, "v cache")
    assert_bitexact(vd, v, "v untouched")
    untouched = torch.ones(blocks * bs, dtype=torch.bool)
    untouched[slots] = False
    assert not bool(kc.view(-1, hk, d)[untouched.to(DEV)].any()), "unwritten slots stay zero"


def test_rope_kv_cache_unaligned_falls_back():
    """Views offset by one element: the fused kernel refuses (EMBER_EALIGN) and the wrapper
    runs rope + kv write; same result as the oracle composition."""
    n, hq, hk, d = 12, 4, 2, 64
    dt = torch.bfloat16
    qkv = _rand(n, 1 + (hq + 2 * hk) * d, dtype=dt, seed=102)
    cos, sin = _tables(d, 256, 1e4)
    pos = torch.randint(0, 256, (n,), generator=torch.Generator().manual_seed(103))
    slots = torch.randperm(64, generator=torch.Generator().manual_seed(104))[:n]

    def views(buf):
        return (buf[:, 1:1 + hq * d].view(n, hq, d), buf[:, 1 + hq * d:1 + (hq + hk) * d].view(n, hk, d),
                buf[:, 1 + (hq + hk) * d:].view(n, hk, d))

    q, k, v = views(qkv)
    want_q, want_k = ref.rope(q, k, cos, sin, pos)
    want_kc = torch.zeros(4, 16, hk, d, dtype=dt)
    want_vc = torch.zeros_like(want_kc)
    ref.kv_cache_write(want_k, v, slots, want_kc, want_vc)
    buf = qkv.to(DEV)
    qd, kd, vd = views(buf)
    kc = torch.zeros(4, 16, hk, d, dtype=dt, device=DEV)
    vc = torch.zeros_like(kc)
    ops.rope_kv_cache_hip(qd, kd, vd, cos.to(DEV), sin.to(DEV), pos.to(DEV), slots.to(DEV), kc, vc)
    assert_bitexact(qd, want_q, "q")
    assert_bitexact(kc, want_kc, "k cache")
    assert_bitexact(vc, want_vc, "v cache")


@pytest.mark.parametrize("return_latent", [True, False])
@pytest.mark.parametrize("in_model", [False, True])
def test_mla_latent_rope_cache_fused(return_latent, in_model):
    """MLA latent path with the latent rows written straight into the paged latent cache:
    the cache rows equal mla_latent_rope's latent rows bit for bit, and match the oracle's
    latent + PagedLatentCache.write."""
    tokens, heads, nope, dr, rank, blocks, bs = 96, 16, 128, 64, 512, 16, 16
    data, w, pos, qsize = _mla_case(tokens, in_model, seed=110)
    cos, sin = _tables(dr, 8192, 5e4)
    slots = torch.randperm(blocks * bs, generator=torch.Generator().manual_seed(111))[:tokens]

    def views(q_buf, kv):
        q = q_buf.view(tokens, heads, nope + dr)
        return q[..., :nope], q[..., nope:], kv[:, :rank], kv[:, rank:]

    if in_model:
        _, q_pe, c, k_pe = views(data[:, :qsize], data[:, qsize:])
        dev_buf = data.to(DEV)
        _, q_pe_d, c_d, k_pe_d = views(dev_buf[:, :qsize], dev_buf[:, qsize:])
    else:
        q, kv_a = data
        _, q_pe, c, k_pe = views(q, kv_a)
        _, q_pe_d, c_d, k_pe_d = views(q.to(DEV), kv_a.to(DEV))
    want_q_pe, want_lat = ref.mla_latent_rope(c, k_pe, q_pe, w, 1e-6, cos, sin, pos)
    want_cache = torch.zeros(blocks, bs, rank + dr, dtype=torch.bfloat16)
    ref.latent_cache_write(want_lat, slots, want_cache)
    cache = torch.zeros(blocks, bs, rank + dr, dtype=torch.bfloat16, device=DEV)
    got_q_pe, lat = ops.mla_latent_rope_cache_hip(c_d, k_pe_d, q_pe_d, w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV),
                                                  pos.to(DEV), slots.to(DEV), cache, return_latent)
    assert_bitexact(got_q_pe, want_q_pe, "q_pe")
    rows = cache.view(-1, rank + dr)[slots.to(DEV)]
    assert_ulp(rows[:, :rank], want_lat[:, :rank], 2, "cached latent c")
    assert_bitexact(rows[:, rank:], want_lat[:, rank:], "cached latent k_pe")
    untouched = torch.ones(blocks * bs, dtype=torch.bool)
    untouched[slots] = False
    assert not bool(cache.view(-1, rank + dr)[untouched.to(DEV)].any())
    if return_latent:
        assert_bitexact(lat, rows, "latent tensor == cached rows")
    else:
        assert lat is None


def test_mla_latent_rope_cache_unaligned_falls_back():
    kv_a, q, w, pos = gen.mla_inputs(6, 2, 8, 16, 100, 64, torch.bfloat16, seed=112)  # rank 100: not 16-B rows
    cos, sin = _tables(16, 64, 1e4)
    slots = torch.tensor([3, 9, 0, 15, 4, 7])
    qv = q.view(6, 2, 24)
    want_q_pe, want_lat = ref.mla_latent_rope(kv_a[:, :100], kv_a[:, 100:], qv[..., 8:], w, 1e-6, cos, sin, pos)
    want_cache = torch.zeros(2, 8, 116, dtype=torch.bfloat16)
    ref.latent_cache_write(want_lat, slots, want_cache)
    kd, qd = kv_a.to(DEV), q.to(DEV)
    cache = torch.zeros(2, 8, 116, dtype=torch.bfloat16, device=DEV)
    got_q_pe, lat = ops.mla_latent_rope_cache_hip(kd[:, :100], kd[:, 100:], qd[..., 8:], w.to(DEV), 1e-6, cos.to(DEV),
                                                  sin.to(DEV), pos.to(DEV), slots.to(DEV), cache)
    assert_bitexact(got_q_pe, want_q_pe, "q_pe")
    assert_ulp(cache, want_cache, 2, "cache")
