"""Parity of the gfx950 paged decode attention (emberserve_amd.paged_decode ->
ember_paged_decode) with the CPU oracle (oracle.ref_ops.paged_decode, the fp32 definition
of attn/paged_torch.py:87-98) on identical seeded inputs.

Tolerance, per output element, against the fp32 oracle o:
  MFMA path (fp16/bf16 q and cache, the reference's tl.dot numerics):
      |got - o| <= 1.1 * (u_p * mass + u_out * |o|) + 1e-4 * mass + 1e-6
    where mass = sum_j p_j |v_j| (oracle.ref_ops.paged_decode_prob_mass) and u = 2^-11
    (fp16) / 2^-8 (bf16) is the relative rounding of a probability to the cache dtype
    before P.V (u_p) and of the result to the output dtype (u_out); 1e-4 * mass covers fp32
    accumulation order over up to 4096 keys.
  fp32 path (fp32 caches, dtype mixes, variant="sum"):
      |got - o| <= 1.1 * u_out * |o| + 1e-5 * mass + 1e-6
The reference's own GPU test allows atol 2e-2, rtol 1e-2 (tests/test_paged_triton_gpu.py:46).
Cases mirror tests/test_paged_triton.py and tests/test_paged_triton_gpu.py (geometry
14q/2kv D=64, ragged contexts up to 2048 with 1, 2048 and a block boundary forced, block
16 and 256, splits 1 / 4 / default) plus Qwen3-8B's 32q/8kv D=128 and group sizes > 16.
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
from emberserve_amd.paged_decode import default_num_splits, paged_attention_decode  # noqa: E402
from oracle import inputs as gen  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402

DEV = "cuda"
U = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -24}


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield


def _ragged(batch: int, max_ctx: int, block: int, seed: int) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, max_ctx + 1, (batch,), generator=g).tolist()
    if batch >= 3:
        ctx[0], ctx[1], ctx[2] = 1, max_ctx, block  # test_paged_triton_gpu.py:58-59
    return ctx


def _to_dev(*ts):
    return [t.to(DEV) for t in ts]


def _check(got: torch.Tensor, q, kc, vc, bt, ctx, scale, mfma: bool, what: str, want=None) -> None:
    """`want` = (output, probability mass) from the oracle, when the caller reuses them."""
    if want is None:
        want = _want(q, kc, vc, bt, ctx, scale)
    o, mass = want
    u_out = U[q.dtype]
    if mfma:
        u_p = U[kc.dtype]
        tol = 1.1 * (u_p * mass + u_out * o.abs()) + 1e-4 * mass + 1e-6
    else:
        tol = 1.1 * u_out * o.abs() + 1e-5 * mass + 1e-6
    err = (got.float().cpu() - o).abs()
    bad = err > tol
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {err.numel()} elements out of tolerance; "
        f"max err {float(err.max()):.3e}, worst ratio {float((err / tol).max()):.2f}")


def _want(q, kc, vc, bt, ctx, scale):
    return (ref.paged_decode(q.float(), kc, vc, bt, ctx, scale),
            ref.paged_decode_prob_mass(q.float(), kc, vc, bt, ctx, scale))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("block", [16, 256])
@pytest.mark.parametrize("batch", [1, 7, 16])
def test_decode_matches_oracle_qwen25_05b_geometry(dtype, block, batch):
    """test_paged_triton_gpu.py:90-102: 14q/2kv, D=64, ragged contexts in [1, 2048]."""
    ctx = _ragged(batch, 2048, block, seed=batch * 31 + block)
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, 14, 2, 64, block, dtype, seed=batch + block)
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    for splits in (1, 4, None):
        _say(f"decode 14/2/64 {dtype} block={block} B={batch} splits={splits}")
        got = paged_attention_decode(dq, dkc, dvc, dbt, dcl, 64 ** -0.5, num_splits=splits)
        assert got.shape == q.shape and got.dtype == dtype
        _check(got, q, kc, vc, bt, cl, 64 ** -0.5, True, f"splits={splits}")
    assert _lib.read_errors() == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (28, 4, 128), (4, 4, 64), (6, 2, 64), (40, 2, 128),
                                      (64, 4, 64), (16, 1, 128)])
def test_decode_matches_oracle_geometries(dtype, hq, hkv, d):
    """Qwen3-8B (32/8, D=128), Qwen2.5-7B (28/4), MHA, padded groups (3), groups > 16 (20,
    split over two 16-head chunks), exactly 16."""
    ctx = _ragged(5, 700, 16, seed=hq + hkv + d)
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, hq, hkv, d, 16, dtype, seed=hq * d)
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    for splits in (1, 3):
        _say(f"decode {hq}/{hkv}/{d} {dtype} splits={splits}")
        got = paged_attention_decode(dq, dkc, dvc, dbt, dcl, d ** -0.5, num_splits=splits)
        _check(got, q, kc, vc, bt, cl, d ** -0.5, True, f"{hq}/{hkv}/{d} splits={splits}")


@pytest.mark.parametrize("qdt,cdt", [(torch.float32, torch.float32), (torch.float16, torch.float32),
                                     (torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16)])
def test_decode_fp32_path(qdt, cdt):
    """test_paged_triton.py:69-95 (fp32 caches, 4q/2kv, D=64, ragged 5/19/40 over scrambled
    tables) and dtype mixes; the last case forces variant="sum" on a bf16 cache."""
    ctx = [5, 19, 40, 1, 64]
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, 4, 2, 64, 16, cdt, seed=11)
    q = q.to(qdt)
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    for splits in (1, 2):
        got = paged_attention_decode(dq, dkc, dvc, dbt, dcl, 64 ** -0.5, num_splits=splits, variant="sum")
        assert got.dtype == qdt
        _check(got, q, kc, vc, bt, cl, 64 ** -0.5, False, f"{qdt}/{cdt} splits={splits}")


def test_decode_fp16_cache_and_padded_groups_reference_case():
    """test_paged_triton.py:116-133: Hq=6, Hk=2, tables [[3,1,0],[2,0,0]], contexts 30, 16."""
    g = torch.Generator().manual_seed(0)
    kc = torch.randn(4, 16, 2, 64, generator=g).half()
    vc = torch.randn(4, 16, 2, 64, generator=g).half()
    q = torch.randn(2, 6, 64, generator=g).half()
    bt = torch.tensor([[3, 1, 0], [2, 0, 0]], dtype=torch.int32)
    cl = torch.tensor([30, 16], dtype=torch.int32)
    got = paged_attention_decode(*_to_dev(q, kc, vc, bt, cl), 64 ** -0.5, num_splits=1)
    assert got.dtype == torch.float16
    _check(got, q, kc, vc, bt, cl, 64 ** -0.5, True, "reference case")


def test_decode_real_config_groups7_reference_case():
    """test_paged_triton.py:135-157: 14q/2kv D=64 fp16, contexts 17, 49, 1, splits 1 and 3."""
    g = torch.Generator().manual_seed(1)
    kc = torch.randn(6, 16, 2, 64, generator=g).half()
    vc = torch.randn(6, 16, 2, 64, generator=g).half()
    q = torch.randn(3, 14, 64, generator=g).half()
    bt = torch.tensor([[5, 2, 0, 0], [1, 4, 3, 0], [2, 0, 0, 0]], dtype=torch.int32)
    cl = torch.tensor([17, 49, 1], dtype=torch.int32)
    for splits in (1, 3):
        got = paged_attention_decode(*_to_dev(q, kc, vc, bt, cl), 64 ** -0.5, num_splits=splits)
        _check(got, q, kc, vc, bt, cl, 64 ** -0.5, True, f"splits={splits}")


@pytest.mark.parametrize("block", [16, 256])
def test_decode_is_deterministic_across_calls(block):
    """test_paged_triton_gpu.py:121-137."""
    ctx = _ragged(8, 1500, block, seed=5)
    q, kc, vc, bt, cl = _to_dev(*gen.decode_inputs(ctx, 14, 2, 64, block, torch.float16, seed=5))
    for splits in (1, 4):
        outs = [paged_attention_decode(q, kc, vc, bt, cl, 0.125, num_splits=splits) for _ in range(3)]
        for o in outs[1:]:
            assert torch.equal(o, outs[0]), f"num_splits={splits} not deterministic"


def test_decode_writes_into_provided_out_buffer_and_strided_q():
    """test_paged_triton_gpu.py:140-150, with q a strided view of a fused qkv row."""
    ctx = _ragged(6, 900, 16, seed=6)
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, 14, 2, 64, 16, torch.bfloat16, seed=6)
    qkv = torch.zeros(6, 18, 64, dtype=torch.bfloat16)
    qkv[:, :14] = q
    dqkv, dkc, dvc, dbt, dcl = _to_dev(qkv, kc, vc, bt, cl)
    dq = dqkv[:, :14]
    out = torch.full((6, 14, 64), float("nan"), dtype=torch.bfloat16, device=DEV)
    got = paged_attention_decode(dq, dkc, dvc, dbt, dcl, 0.125, num_splits=2, out=out)
    assert got.data_ptr() == out.data_ptr()
    _check(out, q, kc, vc, bt, cl, 0.125, True, "out= / strided q")


@pytest.mark.parametrize("batch", [1, 2, 40])
def test_decode_qwen3_small_and_full_grids(batch):
    """Qwen3-8B geometry (32q/8kv, D=128, bf16) on both sides of the workgroup-shape rule:
    grids of at most half as many workgroups as CUs run 8 waves per workgroup, larger
    grids 4. B = 1 and 2 at the default split (16) are small grids; B = 40 is full at any
    split. Contexts up to 3000 keys, one ending mid-block."""
    ctx = [3000] if batch == 1 else _ragged(batch, 3000, 16, seed=batch)
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, 32, 8, 128, 16, torch.bfloat16, seed=70 + batch)
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    for splits in (None, 1, 4):
        _say(f"decode qwen3 B={batch} splits={splits}")
        got = paged_attention_decode(dq, dkc, dvc, dbt, dcl, 128 ** -0.5, num_splits=splits)
        _check(got, q, kc, vc, bt, cl, 128 ** -0.5, True, f"B={batch} splits={splits}")
    assert _lib.read_errors() == 0


@pytest.mark.parametrize("hq,hkv,d,dtype,block", [(14, 2, 64, torch.float16, 16), (32, 8, 128, torch.bfloat16, 16),
                                                   (32, 8, 128, torch.bfloat16, 256)])
def test_decode_long_contexts_cross_block_id_windows(hq, hkv, d, dtype, block):
    """Each wave keeps the block ids of its next 32 key tiles in a register window and
    rereads the table every 32 tiles. One split over 20000 keys gives every wave 79 (8
    waves) or 157 (4 waves) tiles, so several windows; 3 splits and a 9001-key sequence
    move the window edges, and a 1-key sequence sits beside them."""
    ctx = [20000, 9001, 1]
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, hq, hkv, d, block, dtype, seed=hq + block)
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    want = _want(q, kc, vc, bt, cl, d ** -0.5)
    for splits in (1, 3):
        _say(f"decode long contexts {hq}q/{hkv}kv d{d} block {block} splits={splits}")
        got = paged_attention_decode(dq, dkc, dvc, dbt, dcl, d ** -0.5, num_splits=splits)
        _check(got, q, kc, vc, bt, cl, d ** -0.5, True, f"splits={splits}", want)
    assert _lib.read_errors() == 0


def test_decode_full_size_split_invariance_and_sampled_parity():
    """The bench size (128 sequences x 2048 keys, 14q/2kv D=64 fp16, block 16): the default
    split and one split agree within the split-K rounding; four sampled sequences are
    checked against the oracle on their own."""
    ctx = [2048] * 128
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, 14, 2, 64, 16, torch.float16, seed=12)
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    one = paged_attention_decode(dq, dkc, dvc, dbt, dcl, 0.125, num_splits=1)
    splits = default_num_splits(128, 2, bt.shape[1] * 16, dq.device, 14, 64)
    many = paged_attention_decode(dq, dkc, dvc, dbt, dcl, 0.125, num_splits=max(splits, 2))
    diff = (one.float() - many.float()).abs()
    assert float(diff.max()) <= 2 * 2.0 ** -11 * float(one.float().abs().max()) + 1e-3
    for b in (0, 41, 97, 127):
        sl = slice(b, b + 1)
        _check(one[sl], q[sl], kc, vc, bt[sl], cl[sl], 0.125, True, f"sequence {b}")


def test_decode_zero_context_gives_nan_like_the_reference():
    q, kc, vc, bt, cl = gen.decode_inputs([0, 20], 4, 2, 64, 16, torch.float16, seed=13)
    got = paged_attention_decode(*_to_dev(q, kc, vc, bt, cl), 0.125, num_splits=1).cpu()
    want = ref.paged_decode(q, kc, vc, bt, cl, 0.125)
    assert bool(torch.isnan(got[0]).all()) and bool(torch.isnan(want[0]).all())
    assert not bool(torch.isnan(got[1]).any())


def test_decode_bad_block_ids_and_contexts_set_error_bits():
    q, kc, vc, bt, cl = gen.decode_inputs([20, 40], 4, 2, 64, 16, torch.float16, seed=14)
    bt[1, 1] = 10_000
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    paged_attention_decode(dq, dkc, dvc, dbt, dcl, 0.125, num_splits=1)
    assert _lib.read_errors() & _lib.ERR_BLOCK_ID
    dcl2 = torch.tensor([20, 10_000], dtype=torch.int32, device=DEV)
    paged_attention_decode(dq, dkc, dvc, dbt, dcl2, 0.125, num_splits=1)
    assert _lib.read_errors() & _lib.ERR_DECODE_CTX
    os.environ["EMBERSERVE_CHECK_INDICES"] = "1"
    try:
        with pytest.raises(IndexError):
            paged_attention_decode(dq, dkc, dvc, dbt, dcl, 0.125, num_splits=1)
    finally:
        del os.environ["EMBERSERVE_CHECK_INDICES"]


def test_decode_after_kv_cache_write_matches_history():
    """The decode step as the backend drives it (paged_triton.py:465-477): this step's k/v go
    into the cache through ember_kv_cache_write, then the decode kernel reads them back."""
    ctx = [33, 64, 5]
    q, kc, vc, bt, cl = gen.decode_inputs(ctx, 14, 2, 64, 16, torch.float16, seed=15)
    g = torch.Generator().manual_seed(16)
    k_new = torch.randn(3, 2, 64, generator=g).half()
    v_new = torch.randn(3, 2, 64, generator=g).half()
    slots = torch.tensor([int(bt[b, (c - 1) // 16]) * 16 + (c - 1) % 16 for b, c in enumerate(ctx)])
    dq, dkc, dvc, dbt, dcl = _to_dev(q, kc, vc, bt, cl)
    ops.kv_cache_write(k_new.to(DEV), v_new.to(DEV), slots.to(DEV), dkc, dvc)
    got = paged_attention_decode(dq, dkc, dvc, dbt, dcl, 0.125)
    ref.kv_cache_write(k_new, v_new, slots, kc, vc)
    _check(got, q, kc, vc, bt, cl, 0.125, True, "after cache write")


def test_decode_graph_capture_replays_match_eager():
    ctx = _ragged(16, 1024, 16, seed=17)
    q, kc, vc, bt, cl = _to_dev(*gen.decode_inputs(ctx, 14, 2, 64, 16, torch.bfloat16, seed=17))
    eager = paged_attention_decode(q, kc, vc, bt, cl, 0.125, num_splits=4)
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        paged_attention_decode(q, kc, vc, bt, cl, 0.125, num_splits=4, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_attention_decode(q, kc, vc, bt, cl, 0.125, num_splits=4, out=out)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
