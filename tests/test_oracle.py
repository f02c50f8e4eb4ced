"""Pins the CPU oracle (oracle/ref_ops.py) against what the mathematics fixes, so that the
GPU parity tests compare against something checked: float64 closed forms, exact
invariances, IEEE sums done by numpy, and the reference's own closed-form rope tests
(tests/test_rope.py of the reference). Each check is chosen so that a plausible slip in the
restatement (a dropped eps, a wrong half in rotate_half, a swapped sign, rounding at the
wrong point) fails it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import inputs as gen
from oracle import ref_ops as ref
from tests.helpers import assert_bitexact, assert_ulp, ulp_diff

torch.set_num_threads(4)


def _rand(*shape, dtype, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _round_bf16_np(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even of float32 values to bfloat16, returned as float32 (numpy has
    no bfloat16: done on the bit pattern)."""
    b = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16
    return rounded.astype(np.uint32).view(np.float32)


# ---------------------------------------------------------------- rmsnorm

def _rmsnorm_f64(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xd = x.double()
    inv = 1.0 / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps)
    y = (xd * inv).to(x.dtype).double()  # the reference rounds before the weight multiply
    return (y * w.double()).to(x.dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hidden", [64, 896, 4096])
def test_rmsnorm_matches_float64(dtype, hidden):
    x = _rand(9, hidden, dtype=dtype, seed=1, scale=3.0)
    w = _rand(hidden, dtype=dtype, seed=2, scale=0.5) + 1.0
    got = ref.rmsnorm(x, w, 1e-6)
    want = _rmsnorm_f64(x, w, 1e-6)
    # the inner rounding happens at the same point on both sides; only fp32 vs fp64
    # arithmetic separates them
    assert_ulp(got, want, 1 if dtype != torch.float32 else 4, "rmsnorm vs float64")


def test_rmsnorm_eps_enters():
    """A dropped or misplaced eps shows on a row of tiny values: eps dominates there."""
    x = torch.full((1, 16), 1e-4, dtype=torch.float32)
    w = torch.ones(16)
    got = ref.rmsnorm(x, w, 1e-6)
    want = 1e-4 / math.sqrt(1e-8 + 1e-6)
    torch.testing.assert_close(got, torch.full((1, 16), want), atol=0, rtol=1e-6)


def test_rmsnorm_constant_row_closed_form():
    for v in [0.5, -3.0, 7.25]:
        x = torch.full((2, 128), v, dtype=torch.float32)
        w = torch.linspace(0.5, 1.5, 128)
        got = ref.rmsnorm(x, w, 1e-6)
        want = w * (v / math.sqrt(v * v + 1e-6))
        torch.testing.assert_close(got, want.expand(2, 128), atol=0, rtol=2e-7)


def test_rmsnorm_power_of_two_scale_invariance():
    """With eps = 0, scaling a row by 2^k leaves the output bit-identical (every step is
    exact under power-of-two scaling)."""
    x = _rand(6, 896, dtype=torch.float16, seed=3)
    w = _rand(896, dtype=torch.float16, seed=4, scale=0.2) + 1.0
    assert_bitexact(ref.rmsnorm(x * 4, w, 0.0), ref.rmsnorm(x, w, 0.0), "x4")
    assert_bitexact(ref.rmsnorm(x / 8, w, 0.0), ref.rmsnorm(x, w, 0.0), "/8")


def test_rmsnorm_unit_rms():
    x = _rand(16, 4096, dtype=torch.float32, seed=5, scale=5.0)
    out = ref.rmsnorm(x, torch.ones(4096), 1e-6)
    rms = out.pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones(16), atol=1e-5, rtol=0)


# ---------------------------------------------------------------- fused add

def test_fused_add_residual_is_the_ieee_fp16_sum():
    x = _rand(7, 896, dtype=torch.float16, seed=3)
    r = _rand(7, 896, dtype=torch.float16, seed=4, scale=4.0)
    w = _rand(896, dtype=torch.float16, seed=5, scale=0.3) + 1.0
    normed, res = ref.fused_add_rmsnorm(x, r, w, 1e-6)
    want = (r.numpy() + x.numpy()).astype(np.float16)
    assert np.array_equal(res.numpy().view(np.uint16), want.view(np.uint16))
    assert_bitexact(normed, ref.rmsnorm(res, w, 1e-6), "normed = rmsnorm(new residual)")


def test_fused_add_residual_is_the_rne_bf16_sum():
    x = _rand(5, 4096, dtype=torch.bfloat16, seed=6)
    r = _rand(5, 4096, dtype=torch.bfloat16, seed=7, scale=4.0)
    _, res = ref.fused_add_rmsnorm(x, r, torch.ones(4096, dtype=torch.bfloat16), 1e-6)
    want = _round_bf16_np(r.float().numpy() + x.float().numpy())
    assert np.array_equal(res.float().numpy().view(np.uint32), want.view(np.uint32))


def test_fused_add_does_not_modify_inputs():
    x = _rand(3, 64, dtype=torch.float16, seed=1)
    r = _rand(3, 64, dtype=torch.float16, seed=2)
    xc, rc = x.clone(), r.clone()
    ref.fused_add_rmsnorm(x, r, torch.ones(64, dtype=torch.float16), 1e-6)
    assert_bitexact(x, xc)
    assert_bitexact(r, rc)


# ---------------------------------------------------------------- rope

def _complex_rotate(x: torch.Tensor, positions: torch.Tensor, base: float) -> torch.Tensor:
    """Dims (i, i + D/2) as (re, im), multiplied by exp(i * pos * base^(-2i/D)), in float64
    (the reference's independent check, tests/test_rope.py:17-27)."""
    d = x.shape[-1]
    half = d // 2
    inv = 1.0 / (base ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = positions.double()[:, None] * inv[None, :]
    rot = torch.polar(torch.ones_like(ang), ang)
    z = torch.complex(x[..., :half].double(), x[..., half:].double()) * rot[:, None, :]
    return torch.cat((z.real, z.imag), dim=-1)


def test_rotate_half_on_arange():
    x = torch.arange(6.0).view(1, 1, 6)
    assert torch.equal(ref.rotate_half(x), torch.tensor([[[-3.0, -4.0, -5.0, 0.0, 1.0, 2.0]]]))


def test_rope_matches_complex_reference():
    cos, sin = ref.rope_tables(16, 128, 1e4)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(40, 4, 16, generator=g)
    k = torch.randn(40, 2, 16, generator=g)
    pos = torch.randint(0, 128, (40,), generator=g)
    qo, ko = ref.rope(q, k, cos, sin, pos)
    torch.testing.assert_close(qo.double(), _complex_rotate(q, pos, 1e4), atol=1e-5, rtol=0)
    torch.testing.assert_close(ko.double(), _complex_rotate(k, pos, 1e4), atol=1e-5, rtol=0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rope_half_precision_within_one_ulp_of_float64(dtype):
    """In 16-bit storage the final cast dominates: the result is within 1 ulp (relative)
    of the float64 rotation of the same inputs, plus an absolute slack for the fp32 angle
    and product errors, which only matter where the result cancels to near zero."""
    cos, sin = ref.rope_tables(128, 64, 1e6)
    q = _rand(30, 8, 128, dtype=dtype, seed=3)
    pos = torch.randint(0, 64, (30,), generator=torch.Generator().manual_seed(4))
    qo, _ = ref.rope(q, q[:, :1], cos, sin, pos)
    one_ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    torch.testing.assert_close(qo.double(), _complex_rotate(q, pos, 1e6), atol=4e-5, rtol=one_ulp)


def test_rope_position_zero_is_identity():
    cos, sin = ref.rope_tables(64, 8, 1e6)
    q = _rand(5, 4, 64, dtype=torch.bfloat16, seed=5)
    qo, ko = ref.rope(q, q[:, :2], cos, sin, torch.zeros(5, dtype=torch.int64))
    assert_bitexact(qo, q)
    assert_bitexact(ko, q[:, :2])


def test_rope_preserves_norm_and_is_relative():
    cos, sin = ref.rope_tables(16, 128, 1e4)
    g = torch.Generator().manual_seed(4)
    q = torch.randn(32, 4, 16, generator=g)
    pos = torch.randint(0, 128, (32,), generator=g)
    qo, _ = ref.rope(q, q, cos, sin, pos)
    torch.testing.assert_close(qo.norm(dim=-1), q.norm(dim=-1), atol=1e-5, rtol=0)
    a = torch.randn(1, 1, 16, generator=g)
    b = torch.randn(1, 1, 16, generator=g)

    def score(m, n):
        am, _ = ref.rope(a, a, cos, sin, torch.tensor([m]))
        bn, _ = ref.rope(b, b, cos, sin, torch.tensor([n]))
        return (am * bn).sum()

    torch.testing.assert_close(score(10, 3), score(27, 20), atol=1e-5, rtol=0)


def test_rope_tables_against_float64():
    cos, sin = ref.rope_tables(128, 4096, 1e6)
    assert cos.shape == (4096, 128) and cos.dtype == torch.float32
    assert torch.equal(cos[:, :64], cos[:, 64:]) and torch.equal(sin[:, :64], sin[:, 64:])
    inv32 = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).double()
    ang = torch.arange(4096, dtype=torch.float64)[:, None] * inv32[None, :]
    # fp32 angle products carry ~pos * 2^-24 absolute error; cos/sin within that plus 1 ulp
    tol = 4096 * 2.0 ** -23
    torch.testing.assert_close(cos[:, :64].double(), torch.cos(ang), atol=tol, rtol=0)
    torch.testing.assert_close(sin[:, :64].double(), torch.sin(ang), atol=tol, rtol=0)


def test_llama3_scaling_bands():
    """High frequencies kept, low frequencies divided by `factor`, monotone in between
    (the reference checks the same bands, tests/test_model_families.py:70-90)."""
    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    out = ref.llama3_scale_inv_freq(inv, sc)
    wavelen = 2 * math.pi / inv
    hi = wavelen < 8192 / 4
    lo = wavelen > 8192 / 1
    assert torch.equal(out[hi], inv[hi])
    torch.testing.assert_close(out[lo], inv[lo] / 8)
    mid = ~hi & ~lo
    assert bool(((out[mid] <= inv[mid]) & (out[mid] >= inv[mid] / 8)).all())


# ---------------------------------------------------------------- silu

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_silu_and_mul_matches_float64(dtype):
    x = _rand(3, 2 * 4864, dtype=dtype, seed=7, scale=2.0)
    got = ref.silu_and_mul(x)
    g, u = x[:, :4864].double(), x[:, 4864:].double()
    act = (g / (1 + torch.exp(-g))).to(dtype).double()  # rounded before the multiply
    assert_ulp(got, (act * u).to(dtype), 1, "silu vs float64")


def test_silu_special_values():
    x = torch.tensor([[0.0, 20.0, -20.0, 1.0, 3.0, 3.0, 2.0, -1.0]], dtype=torch.float32)
    out = ref.silu_and_mul(x)
    assert out[0, 0] == 0.0
    torch.testing.assert_close(out[0, 1], torch.tensor(20.0 * 3.0), rtol=1e-7, atol=0)  # ~g*u
    assert abs(float(out[0, 2])) < 1e-6  # silu(-20) ~ -4e-8, times 2
    torch.testing.assert_close(out[0, 3], torch.tensor(1.0 / (1 + math.exp(-1.0)) * -1.0))


# ---------------------------------------------------------------- gate_up + silu_and_mul

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gate_up_silu_brute_force(dtype):
    """Per element: Python float sums of x[t, k] * w[j, k] rounded to the dtype (the linear
    layer's output), then the activation in float64 rounded as silu_and_mul rounds."""
    x, w = gen.gate_up_inputs(3, 24, 5, dtype, seed=11)
    got = ref.gate_up_silu(x, w)
    assert got.shape == (3, 5) and got.dtype == dtype
    xs, ws = x.double().tolist(), w.double().tolist()
    for t in range(3):
        for j in range(5):
            g = torch.tensor(math.fsum(a * b for a, b in zip(xs[t], ws[j])), dtype=torch.float64).to(dtype)
            u = torch.tensor(math.fsum(a * b for a, b in zip(xs[t], ws[5 + j])), dtype=torch.float64).to(dtype)
            gd, ud = float(g), float(u)
            act = torch.tensor(gd / (1 + math.exp(-gd)), dtype=torch.float64).to(dtype)
            want = torch.tensor(float(act) * ud, dtype=torch.float64).to(dtype)
            assert_ulp(got[t:t + 1, j:j + 1], want.view(1, 1), 1, f"t={t} j={j}")


def test_gate_up_silu_unit_rows_and_halves():
    """Gate row j = e_(2j), up row j = e_(2j+1) * 2: g and u are single x entries exactly, so
    out = silu_and_mul of those entries; the halves are rows [0, I) and [I, 2I)."""
    H, I = 16, 4
    x = _rand(2, H, dtype=torch.bfloat16, seed=3)
    w = torch.zeros(2 * I, H, dtype=torch.bfloat16)
    for j in range(I):
        w[j, 2 * j] = 1.0
        w[I + j, 2 * j + 1] = 2.0
    got = ref.gate_up_silu(x, w)
    pairs = torch.cat([x[:, 0::2][:, :I], x[:, 1::2][:, :I] * 2], dim=1)
    assert torch.equal(got, ref.silu_and_mul(pairs))
    w[I:] = 0
    assert torch.equal(ref.gate_up_silu(x, w), torch.zeros(2, I, dtype=torch.bfloat16))


# ---------------------------------------------------------------- embedding

def test_embedding_matches_numpy_take():
    ids, w = gen.embedding_inputs(300, 1000, 96, torch.bfloat16, seed=2)
    got = ref.embedding(ids, w)
    want = np.take(w.view(torch.int16).numpy(), ids.numpy(), axis=0)
    assert np.array_equal(got.view(torch.int16).numpy(), want)


def test_embedding_rejects_out_of_range():
    w = torch.zeros(10, 4)
    with pytest.raises(IndexError):
        ref.embedding(torch.tensor([10]), w)


# ---------------------------------------------------------------- composed ops

def test_qk_norm_rope_matches_float64():
    n, hq, hk, d = 12, 4, 2, 128
    qkv, qw, kw, pos = gen.qkv_inputs(n, hq, hk, d, 64, torch.bfloat16, seed=50)
    cos, sin = ref.rope_tables(d, 64, 1e6)
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hk) * d].view(n, hk, d)
    qo, ko = ref.qk_norm_rope(q, k, qw, kw, 1e-6, cos, sin, pos)
    for x, w, o in [(q, qw, qo), (k, kw, ko)]:
        y = _rmsnorm_f64(x.reshape(-1, d), w, 1e-6).view(x.shape)  # bf16, as the model stores it
        want = _complex_rotate(y, pos, 1e6).to(torch.bfloat16)
        assert ulp_diff(o, want).max() <= 2


def test_mla_latent_rope_matches_float64():
    n, h, dn, dr, r = 10, 4, 32, 64, 512
    kv_a, q, w, pos = gen.mla_inputs(n, h, dn, dr, r, 256, torch.bfloat16, seed=61)
    cos, sin = ref.rope_tables(dr, 256, 5e4)
    qv = q.view(n, h, dn + dr)
    q_pe, latent = ref.mla_latent_rope(kv_a[:, :r], kv_a[:, r:], qv[..., dn:], w, 1e-6, cos, sin, pos)
    assert latent.shape == (n, r + dr)
    assert_ulp(latent[:, :r], _rmsnorm_f64(kv_a[:, :r], w, 1e-6), 1, "latent c")
    want_k = _complex_rotate(kv_a[:, r:].unsqueeze(1), pos, 5e4).squeeze(1).to(torch.bfloat16)
    assert ulp_diff(latent[:, r:], want_k).max() <= 1
    want_q = _complex_rotate(qv[..., dn:], pos, 5e4).to(torch.bfloat16)
    assert ulp_diff(q_pe, want_q).max() <= 1


def test_ulp_helper_counts_ulps():
    a = torch.tensor([1.0, -1.0, 0.0], dtype=torch.float16)
    b = torch.tensor([1.0 + 2 ** -10, -1.0 - 2 * 2 ** -10, -0.0], dtype=torch.float16)
    assert ulp_diff(a, b).tolist() == [1, 2, 0]


# ---------------------------------------------------------------- KV-cache writes

def test_kv_cache_write_matches_slot_loop():
    g = torch.Generator().manual_seed(9)
    n, hk, d, blocks, bs = 10, 2, 16, 4, 8
    k = torch.randn(n, hk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(n, hk, d, generator=g).to(torch.bfloat16)
    slots = torch.randperm(blocks * bs, generator=g)[:n]
    kc = torch.zeros(blocks, bs, hk, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    ref.kv_cache_write(k, v, slots, kc, vc)
    want_k = torch.zeros_like(kc).view(-1, hk, d)
    want_v = torch.zeros_like(vc).view(-1, hk, d)
    for t in range(n):
        want_k[int(slots[t])] = k[t]
        want_v[int(slots[t])] = v[t]
    assert_bitexact(kc.view(-1, hk, d), want_k)
    assert_bitexact(vc.view(-1, hk, d), want_v)


def test_latent_cache_write_matches_slot_loop():
    g = torch.Generator().manual_seed(10)
    n, dim = 7, 576
    lat = torch.randn(n, dim, generator=g).to(torch.bfloat16)
    slots = torch.tensor([5, 0, 31, 8, 9, 17, 2])
    cache = torch.zeros(4, 8, dim, dtype=torch.bfloat16)
    ref.latent_cache_write(lat, slots, cache)
    want = torch.zeros(32, dim, dtype=torch.bfloat16)
    for t in range(n):
        want[int(slots[t])] = lat[t]
    assert_bitexact(cache.view(-1, dim), want)


# ---- paged decode attention --------------------------------------------------------------
def _decode_brute_force(q, kc, vc, bt, ctx, scale):
    """Key-by-key float64 softmax over the block table with Python sums and math.exp."""
    B, H, D = q.shape
    hkv = kc.shape[2]
    bs = kc.shape[1]
    G = H // hkv
    out = np.zeros((B, H, D))
    qd, kd, vd = q.double().numpy(), kc.double().numpy(), vc.double().numpy()
    for b in range(B):
        for h in range(H):
            kvh = h // G
            rows = [(int(bt[b, j // bs]), j % bs) for j in range(int(ctx[b]))]
            s = [scale * sum(qd[b, h, e] * kd[blk, sl, kvh, e] for e in range(D)) for blk, sl in rows]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            tot = sum(w)
            for e in range(D):
                out[b, h, e] = sum(wj * vd[blk, sl, kvh, e] for wj, (blk, sl) in zip(w, rows)) / tot
    return out


def test_paged_decode_matches_brute_force():
    q, kc, vc, bt, ctx = gen.decode_inputs([5, 19, 40], 4, 2, 8, 16, torch.float32, seed=3)
    out = ref.paged_decode(q, kc, vc, bt, ctx, 8 ** -0.5)
    bf = _decode_brute_force(q, kc, vc, bt, ctx, 8 ** -0.5)
    np.testing.assert_allclose(out.double().numpy(), bf, rtol=0, atol=2e-6)


def test_paged_decode_single_key_returns_its_value_row():
    q, kc, vc, bt, ctx = gen.decode_inputs([1, 1], 6, 3, 16, 16, torch.float32, seed=4)
    out = ref.paged_decode(q, kc, vc, bt, ctx, 0.25)
    for b in range(2):
        blk = int(bt[b, 0])
        expect = vc[blk, 0].repeat_interleave(2, dim=0)  # head h -> KV head h // 2
        assert torch.equal(out[b], expect)


def test_paged_decode_equal_keys_average_the_values():
    q, kc, vc, bt, ctx = gen.decode_inputs([37], 2, 1, 16, 16, torch.float32, seed=5)
    kc[:] = kc[0, 0]  # every key identical -> uniform attention
    out = ref.paged_decode(q, kc, vc, bt, ctx, 0.3)
    k, v, _ = ref.gather_batch(kc, vc, bt, ctx)
    expect = v[0, :37, 0].double().mean(0)
    for h in range(2):
        np.testing.assert_allclose(out[0, h].double().numpy(), expect.numpy(), rtol=0, atol=1e-6)


def test_paged_decode_is_invariant_to_block_relocation():
    q, kc, vc, bt, ctx = gen.decode_inputs([23, 48], 4, 2, 8, 16, torch.float32, seed=6, spare_blocks=3)
    base = ref.paged_decode(q, kc, vc, bt, ctx, 0.35)
    perm = torch.randperm(kc.shape[0], generator=gen.gen(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    kc2, vc2 = kc[perm], vc[perm]  # block p of the new pool is old block perm[p]
    bt2 = inv[bt.long()].to(torch.int32)
    assert torch.equal(ref.paged_decode(q, kc2, vc2, bt2, ctx, 0.35), base)


def test_paged_decode_gqa_maps_head_to_kv_head_group():
    q, kc, vc, bt, ctx = gen.decode_inputs([30], 6, 2, 8, 16, torch.float32, seed=7)
    out = ref.paged_decode(q, kc, vc, bt, ctx, 0.35)
    for h in range(6):  # the same head against a one-KV-head cache holding KV head h // 3
        one = ref.paged_decode(q[:, h:h + 1], kc[:, :, h // 3:h // 3 + 1], vc[:, :, h // 3:h // 3 + 1],
                               bt, ctx, 0.35)
        torch.testing.assert_close(out[:, h:h + 1], one, rtol=0, atol=1e-6)


def test_paged_decode_equals_per_sequence_causal_attention():
    """attn/base.py:105-128 with Tq = 1 (the last key is the query's own position) over
    each sequence's gathered context: the formulation the reference tests decode against."""
    q, kc, vc, bt, ctx = gen.decode_inputs([17, 49, 1], 14, 2, 64, 16, torch.float32, seed=8)
    out = ref.paged_decode(q, kc, vc, bt, ctx, 64 ** -0.5)
    k, v, _ = ref.gather_batch(kc, vc, bt, ctx)
    for b, n in enumerate(ctx.tolist()):
        kk = k[b, :n].float().repeat_interleave(7, dim=1).transpose(0, 1)  # [H, n, D]
        vv = v[b, :n].float().repeat_interleave(7, dim=1).transpose(0, 1)
        sc = torch.matmul(q[b].float()[:, None, :], kk.transpose(-1, -2)) / 8.0
        o = torch.matmul(torch.softmax(sc, dim=-1), vv)[:, 0]
        torch.testing.assert_close(out[b], o, rtol=0, atol=2e-6)


def test_paged_decode_prob_mass_bounds_the_output():
    q, kc, vc, bt, ctx = gen.decode_inputs([40, 3], 4, 2, 16, 16, torch.float32, seed=10)
    out = ref.paged_decode(q, kc, vc, bt, ctx, 0.25)
    mass = ref.paged_decode_prob_mass(q, kc, vc, bt, ctx, 0.25)
    assert bool((out.abs() <= mass + 1e-6).all())
    assert bool((mass <= vc.abs().amax() + 1e-6).all())


# ---------------------------------------------------------------- MLA decode

def _mla_brute_force(q_abs, lat, bt, ctx, scale, dl):
    """Key by key in float64 Python arithmetic (math.exp, explicit sums)."""
    qd, ld = q_abs.double().tolist(), lat.double().tolist()
    B, H, D = q_abs.shape
    bs = lat.shape[1]
    out = np.zeros((B, H, dl))
    for b in range(B):
        rows = [ld[int(bt[b, j // bs])][j % bs] for j in range(int(ctx[b]))]
        for h in range(H):
            s = [scale * sum(qd[b][h][e] * r[e] for e in range(D)) for r in rows]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            tot = sum(w)
            for e in range(dl):
                out[b, h, e] = sum(wj * r[e] for wj, r in zip(w, rows)) / tot
    return out


def _mla_ref(q_abs, lat, bt, ctx, scale, dl):
    return ref.mla_decode(q_abs[..., :dl], q_abs[..., dl:], lat, bt, ctx, scale, dl)


def test_mla_decode_matches_brute_force():
    q, lat, bt, ctx = gen.mla_decode_inputs([5, 19, 33], 3, 8, 4, 16, torch.float32, seed=11)
    out = _mla_ref(q, lat, bt, ctx, 0.4, 8)
    np.testing.assert_allclose(out.double().numpy(), _mla_brute_force(q, lat, bt, ctx, 0.4, 8), rtol=0, atol=2e-6)


def test_mla_decode_single_key_returns_its_latent_row():
    q, lat, bt, ctx = gen.mla_decode_inputs([1, 1], 4, 16, 8, 16, torch.float32, seed=12)
    out = _mla_ref(q, lat, bt, ctx, 0.3, 16)
    for b in range(2):
        c = lat[int(bt[b, 0]), 0, :16]
        assert torch.equal(out[b], c.expand(4, 16))


def test_mla_decode_zero_query_averages_the_latents():
    q, lat, bt, ctx = gen.mla_decode_inputs([45], 2, 16, 8, 16, torch.float32, seed=13)
    q.zero_()  # every score 0 -> uniform attention over the context
    out = _mla_ref(q, lat, bt, ctx, 0.3, 16)
    rows = ref.gather_latent(lat, bt[0], 45)
    expect = rows[:, :16].double().mean(0)
    for h in range(2):
        np.testing.assert_allclose(out[0, h].double().numpy(), expect.numpy(), rtol=0, atol=1e-6)


def test_mla_decode_is_invariant_to_block_relocation():
    q, lat, bt, ctx = gen.mla_decode_inputs([23, 48], 4, 16, 8, 16, torch.float32, seed=14)
    base = _mla_ref(q, lat, bt, ctx, 0.35, 16)
    perm = torch.randperm(lat.shape[0], generator=gen.gen(15))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    torch.testing.assert_close(_mla_ref(q, lat[perm], inv[bt.long()].to(torch.int32), ctx, 0.35, 16), base,
                               rtol=0, atol=0)


def test_mla_decode_without_rope_part_is_mqa_paged_decode():
    """q_pe = 0 and k_pe = 0: MQA over the c part with K = V = c, which is paged_decode with
    one KV head."""
    q, lat, bt, ctx = gen.mla_decode_inputs([17, 40], 6, 16, 8, 16, torch.float32, seed=16)
    q[..., 16:] = 0
    lat[..., 16:] = 0
    out = _mla_ref(q, lat, bt, ctx, 0.25, 16)
    c = lat[..., :16].unsqueeze(2).contiguous()  # [blocks, bs, 1, DL]
    want = ref.paged_decode(q[..., :16].contiguous(), c, c, bt, ctx, 0.25)
    torch.testing.assert_close(out, want, rtol=0, atol=2e-6)


@pytest.mark.parametrize("q_len", [1, 5])
def test_mla_absorbed_equals_the_per_head_form(q_len):
    """The absorbed form against the per-head one it is derived from (mla_torch.py:1-17):
    k_nope[t, h] = W_UK[h] c[t], v[t, h] = W_UV[h] c[t], scores q_nope . k_nope + q_pe . k_pe,
    causal over the last q_len positions, out = softmax . v."""
    g = gen.gen(17)
    T, H, Dn, Dr, Dl, Dv = 20, 3, 6, 4, 16, 5
    lat = torch.randn(T, Dl + Dr, generator=g, dtype=torch.float64)
    q_nope = torch.randn(q_len, H, Dn, generator=g, dtype=torch.float64)
    q_pe = torch.randn(q_len, H, Dr, generator=g, dtype=torch.float64)
    w_uk = torch.randn(H, Dn, Dl, generator=g, dtype=torch.float64)
    w_uv = torch.randn(H, Dv, Dl, generator=g, dtype=torch.float64)
    got = ref.mla_attention_absorbed(q_nope, q_pe, lat, w_uk, w_uv, 0.3, Dl).double()
    c, k_pe = lat[:, :Dl], lat[:, Dl:]
    want = torch.empty(q_len, H, Dv, dtype=torch.float64)
    for i in range(q_len):
        n = T - q_len + i + 1  # keys visible to query i
        for h in range(H):
            k_nope = c[:n] @ w_uk[h].T  # [n, Dn]
            v = c[:n] @ w_uv[h].T  # [n, Dv]
            s = (k_nope @ q_nope[i, h] + k_pe[:n] @ q_pe[i, h]) * 0.3
            want[i, h] = torch.softmax(s, 0) @ v
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_mla_decode_prob_mass_bounds_the_output():
    q, lat, bt, ctx = gen.mla_decode_inputs([40, 3], 4, 16, 8, 16, torch.float32, seed=18)
    out = _mla_ref(q, lat, bt, ctx, 0.25, 16)
    mass = ref.mla_decode_prob_mass(q[..., :16], q[..., 16:], lat, bt, ctx, 0.25, 16)
    assert bool((out.abs() <= mass + 1e-6).all())


# ---------------------------------------------------------------- mixed-step pack / unpack

_MIXES = [[1, 1, 1], [5], [1, 7, 1, 3, 1], [2, 2], [1, 300, 1, 1], [4, 1, 9]]


@pytest.mark.parametrize("lens", _MIXES)
def test_mixed_pack_matches_the_slot_definition(lens):
    """Slot by slot on a small input: decode rows in batch order are the packed rows whose
    sequence has query length 1; prefill sequence p's slot r holds its query
    r - (max_q - n) (left padding), zeros before that."""
    T = sum(lens)
    q = torch.arange(T * 3 * 2, dtype=torch.float32).view(T, 3, 2)
    q_dec, qpad = ref.mixed_pack(q, lens)
    starts = [sum(lens[:i]) for i in range(len(lens))]
    dec = [s for s, n in zip(starts, lens) if n == 1]
    pre = [(s, n) for s, n in zip(starts, lens) if n != 1]
    if dec:
        for i, s in enumerate(dec):
            assert torch.equal(q_dec[i], q[s])
    else:
        assert q_dec is None
    if pre:
        max_q = max(n for _, n in pre)
        assert qpad.shape == (len(pre), max_q, 3, 2)
        for p, (s, n) in enumerate(pre):
            for r in range(max_q):
                j = r - (max_q - n)
                want = q[s + j] if j >= 0 else torch.zeros(3, 2)
                assert torch.equal(qpad[p, r], want), (p, r)
    else:
        assert qpad is None


@pytest.mark.parametrize("lens", _MIXES)
def test_mixed_unpack_inverts_pack(lens):
    T = sum(lens)
    q = _rand(T, 4, 8, dtype=torch.bfloat16, seed=T)
    q_dec, qpad = ref.mixed_pack(q, lens)
    out = torch.full_like(q, float("nan"))
    ref.mixed_unpack(out, q_dec, qpad, lens)
    assert_bitexact(out, q, "unpack(pack(q))")


def test_moe_gate_up_silu_oracle_rows_and_experts():
    """All tokens routed to one expert equal gate_up_silu with that expert's weight; rows
    follow t * k + c; the expert is picked by index."""
    x, w0 = gen.gate_up_inputs(4, 32, 8, torch.bfloat16, seed=21)
    _, w1 = gen.gate_up_inputs(4, 32, 8, torch.bfloat16, seed=22)
    w = torch.stack([w0, w1])
    same = ref.moe_gate_up_silu(x, torch.zeros(4, 1, dtype=torch.long), w)
    assert torch.equal(same, ref.gate_up_silu(x, w0))
    ids = torch.tensor([[1, 0]] * 4)
    got = ref.moe_gate_up_silu(x, ids, w)
    assert torch.equal(got[0::2], ref.gate_up_silu(x, w1)) and torch.equal(got[1::2], ref.gate_up_silu(x, w0))


# ---- moe_align layout ---------------------------------------------------------------------
def test_moe_align_oracle_reference_case():
    """tests/test_moe_triton.py:34-48's case (N=4, k=2, E=4, block 4), slot by slot:
    flat ids [1,3,3,0,1,1,3,2] -> expert 0 {3}, 1 {0,4,5}, 2 {7}, 3 {1,2,6}."""
    ids = torch.tensor([[1, 3], [3, 0], [1, 1], [3, 2]])
    s, b, nv = ref.moe_align(ids, 4, 4)
    assert nv == 8
    assert s == [3, 8, 8, 8, 0, 4, 5, 8, 7, 8, 8, 8, 1, 2, 6, 8, 8, 8, 8, 8]
    assert b == [0, 1, 2, 3, 4]


def test_moe_align_oracle_closed_forms():
    # every assignment to one expert: one run 0..nv-1, then padding; that expert's blocks
    ids = torch.full((5, 3), 2)
    s, b, nv = ref.moe_align(ids, 8, 4)
    assert nv == 15 and len(s) == (15 + 8 * 3 + 3) // 4 * 4
    assert s[:15] == list(range(15)) and all(v == 15 for v in s[15:])
    assert b[:4] == [2] * 4 and all(v == 8 for v in b[4:])
    # no assignments: all sentinels
    s, b, nv = ref.moe_align(torch.zeros((0, 6), dtype=torch.long), 64, 16)
    assert nv == 0 and s == [0] * 960 and b == [64] * 60
    # block 1: every assignment is its own block, in expert then id order
    s, b, nv = ref.moe_align(torch.tensor([[2, 0], [2, 1]]), 3, 1)
    assert s == [1, 3, 0, 2] and b == [0, 1, 2, 2]


@pytest.mark.parametrize("n,e,k,bm", [(1, 64, 6, 16), (7, 8, 2, 16), (50, 16, 4, 16), (3, 4, 4, 4), (40, 5, 3, 8)])
def test_moe_align_oracle_properties(n, e, k, bm):
    """Each assignment exactly once; runs ascending, one expert each, starting on a block
    boundary; blocks in ascending expert order; block counts ceil(count / bm)."""
    ids = torch.randint(0, e, (n, k), generator=torch.Generator().manual_seed(n * e + k))
    s, b, nv = ref.moe_align(ids, e, bm)
    flat = ids.reshape(-1).tolist()
    assert len(s) == -(-(nv + e * (bm - 1)) // bm) * bm and len(b) == len(s) // bm
    assert sorted(v for v in s if v < nv) == list(range(nv))
    used = [x for x in b if x < e]
    assert used == sorted(used) and all(x == e for x in b[len(used):])
    for x in range(e):
        assert used.count(x) == -(-flat.count(x) // bm)
    for blk, x in enumerate(b):
        rows = [v for v in s[blk * bm:(blk + 1) * bm] if v < nv]
        if x >= e:
            assert not rows
        else:
            assert rows == sorted(rows) and all(flat[v] == x for v in rows)


@pytest.mark.parametrize("groups", [1, 3, 4, 7, 100])
def test_pack_gate_up_weight_index_definition(groups):
    """Element by element against the layout's closed form: unit (slab, j) of U units holds
    W[part I + 64 slab + 16 wave + lane % 16][64 j + 32 h + 8 (lane // 16) + e] at
    ((h * 4 + wave) * 2 + part) * 64 + lane, and the t-th unit of workgroup b's run is stored at
    t G + b while t < U // G, the extra units of longer runs after those in workgroup order
    (G = min(groups, U); runs of 3 and 4 units at G 7, a clamp at 100)."""
    i, h = 128, 128
    w = torch.arange(2 * i * h, dtype=torch.float64).view(2 * i, h)
    p = ref.pack_gate_up_weight(w, groups)
    assert p.numel() == w.numel()
    total = (i // 64) * (h // 64)
    g = min(groups, total)
    q = total // g
    pos = {}
    for b in range(g):
        start = b * total // g
        for t in range((b + 1) * total // g - start):
            pos[start + t] = t * g + b if t < q else q * g + (start - b * q)
    assert sorted(pos.values()) == list(range(total))
    for slab in range(i // 64):
        for j in range(h // 64):
            base = pos[slab * (h // 64) + j] * 8192
            for idx in range(0, 8192, 29):
                e, lane, part, wave, hh = idx % 8, idx // 8 % 64, idx // 512 % 2, idx // 1024 % 4, idx // 4096
                row = part * i + 64 * slab + 16 * wave + lane % 16
                col = 64 * j + 32 * hh + 8 * (lane // 16) + e
                assert float(p[base + idx]) == float(w[row, col]), (groups, slab, j, idx)
    assert sorted(p.tolist()) == list(range(w.numel()))  # a permutation


def test_pack_moe_gate_up_weight_index_definition():
    """Element by element: expert e at e * 2 I H, unit (j, slab) at (j * I / 64 + slab) * 8192,
    holding W[e][part I + 64 slab + 16 wave + lane % 16][64 j + 32 h + 8 (lane // 16) + e8] at
    ((h * 4 + wave) * 2 + part) * 64 + lane."""
    ne, i, h = 3, 128, 192
    w = torch.arange(ne * 2 * i * h, dtype=torch.float64).view(ne, 2 * i, h)
    p = ref.pack_moe_gate_up_weight(w)
    slabs = i // 64
    for e in range(ne):
        for j in range(h // 64):
            for slab in range(slabs):
                base = e * 2 * i * h + (j * slabs + slab) * 8192
                for idx in range(0, 8192, 31):
                    e8, lane, part, wave, hh = idx % 8, idx // 8 % 64, idx // 512 % 2, idx // 1024 % 4, idx // 4096
                    row = part * i + 64 * slab + 16 * wave + lane % 16
                    col = 64 * j + 32 * hh + 8 * (lane // 16) + e8
                    assert float(p[base + idx]) == float(w[e, row, col]), (e, j, slab, idx)
    assert sorted(p.tolist()) == list(range(w.numel()))
