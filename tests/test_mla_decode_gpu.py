"""Parity of the gfx950 MLA decode (emberserve_amd.mla_decode -> ember_mla_decode) with the
CPU oracle (oracle.ref_ops.mla_decode: mla_attention_absorbed with identity W, the
definition tests/test_mla_triton_gpu.py:40-49 compares the reference kernel with) on
identical seeded inputs.

Tolerance, per output element, against the fp32 oracle o (as for paged decode):
  MFMA path (fp16/bf16, DL 512, DR 64: the reference kernel's tl.dot numerics):
      |got - o| <= 1.1 * (u_p * mass + u_out * |o|) + 1e-4 * mass + 1e-6
    mass = sum_j p_j |c_j| (oracle.ref_ops.mla_decode_prob_mass), u = 2^-11 (fp16) / 2^-8
    (bf16) the relative rounding of a probability before P.c (u_p) and of the result
    (u_out); 1e-4 * mass covers fp32 accumulation order.
  fp32 path (fp32 caches, other geometries):
      |got - o| <= 1.1 * u_out * |o| + 1e-5 * mass + 1e-6
The reference's own test allows atol = rtol = 2e-2 (fp16) and 5e-2 (bf16)
(tests/test_mla_triton_gpu.py:57-58); both bounds are asserted. Cases: the reference's
(Moonlight geometry H 16, DL 512, DR 64, block 16; contexts [1], [16, 17],
[300, 5, 1024, 77], [2048] * 8; splits 1, default, 4), its interpreter geometry (H 4, DL 32,
DR 16, fp32, splits 1 / 2 / 3), head counts that are not a multiple of 16, the pair form
of q with strided views, block size 64, bad contexts and block ids, and graph replay.
"""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib  # noqa: E402
from emberserve_amd.mla_decode import mla_decode, mla_num_splits  # noqa: E402
from emberserve_amd.paged_decode import num_sms  # noqa: E402
from oracle import inputs as gen  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402

DEV = "cuda"
U = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -24}
REF_TOL = {torch.float16: 2e-2, torch.bfloat16: 5e-2, torch.float32: 1e-4}
H, DL, DR = 16, 512, 64
SCALE = (128 + 64) ** -0.5


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield


def _check(got, q_c, q_pe, lat, bt, ctx, scale, dl, mfma: bool, what: str) -> None:
    o = ref.mla_decode(q_c.float(), q_pe.float(), lat, bt, ctx, scale, dl)
    mass = ref.mla_decode_prob_mass(q_c.float(), q_pe.float(), lat, bt, ctx, scale, dl)
    u_out = U[q_c.dtype]
    if mfma:
        tol = 1.1 * (U[lat.dtype] * mass + u_out * o.abs()) + 1e-4 * mass + 1e-6
    else:
        tol = 1.1 * u_out * o.abs() + 1e-5 * mass + 1e-6
    g = got.float().cpu()
    err = (g - o).abs()
    bad = err > tol
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {err.numel()} elements out of tolerance; "
        f"max err {float(err.max()):.3e}, worst ratio {float((err / tol).max()):.2f}")
    t = REF_TOL[q_c.dtype]
    torch.testing.assert_close(g, o, atol=t, rtol=t)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ctx_lens", [[1], [16, 17], [300, 5, 1024, 77], [2048] * 8])
def test_kernel_matches_reference(dtype, ctx_lens):
    q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, H, DL, DR, 16, dtype, seed=1)
    qd, latd, btd, ctxd = (t.to(DEV) for t in (q, lat, bt, ctx))
    for splits in (1, None, 4):
        _say(f"mla decode {dtype} ctx {ctx_lens[:4]} splits {splits}")
        got = mla_decode(qd, latd, btd, ctxd, SCALE, DL, num_splits=splits)
        torch.cuda.synchronize()
        _check(got, q[..., :DL], q[..., DL:], lat, bt, ctx, SCALE, DL, True, f"splits {splits}")
    assert _lib.read_errors() == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_full_grid_two_stream_workgroups(dtype):
    """160 sequences of ragged contexts (1..700 keys) at one and two splits: a grid of more
    than half the CUs, which runs two tile streams per workgroup (small grids run four)."""
    g = torch.Generator().manual_seed(11)
    ctx_lens = torch.randint(1, 701, (160,), generator=g).tolist()
    ctx_lens[:3] = [1, 700, 16]
    q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, H, DL, DR, 16, dtype, seed=12)
    for splits in (1, 2):
        _say(f"mla decode full grid {dtype} splits {splits}")
        got = mla_decode(q.to(DEV), lat.to(DEV), bt.to(DEV), ctx.to(DEV), SCALE, DL, num_splits=splits)
        torch.cuda.synchronize()
        _check(got, q[..., :DL], q[..., DL:], lat, bt, ctx, SCALE, DL, True, f"splits {splits}")
    assert _lib.read_errors() == 0


def test_long_contexts_cross_block_id_windows():
    """Contexts of 9000 and 5000 keys at one and two splits: each wave walks 40-71 tiles,
    crossing the 32-tile windows of prefetched block ids; block size 32 (two halves per
    block)."""
    q, lat, bt, ctx = gen.mla_decode_inputs([9000, 5000, 33], H, DL, DR, 32, torch.bfloat16, seed=10)
    for splits in (1, 2):
        _say(f"mla decode long contexts splits {splits}")
        got = mla_decode(q.to(DEV), lat.to(DEV), bt.to(DEV), ctx.to(DEV), SCALE, DL, num_splits=splits)
        torch.cuda.synchronize()
        _check(got, q[..., :DL], q[..., DL:], lat, bt, ctx, SCALE, DL, True, f"splits {splits}")
    assert _lib.read_errors() == 0


def test_full_size_sampled_parity_at_every_split_count():
    """The bench's largest row (256 sequences x 2048 keys, bf16, block 16) at one split,
    the default and 8: five sampled sequences of each match the oracle on their own, and
    no error bit is set."""
    ctx = [2048] * 256
    q, lat, bt, cl = gen.mla_decode_inputs(ctx, H, DL, DR, 16, torch.bfloat16, seed=13, spare_blocks=1)
    dq, dlat, dbt, dcl = (t.to(DEV) for t in (q, lat, bt, cl))
    for splits in (1, None, 8):
        _say(f"mla decode full size splits {splits}")
        got = mla_decode(dq, dlat, dbt, dcl, SCALE, DL, num_splits=splits).cpu()
        for b in (0, 77, 128, 201, 255):
            sl = slice(b, b + 1)
            _check(got[sl], q[sl, :, :DL], q[sl, :, DL:], lat, bt[sl], cl[sl], SCALE, DL, True,
                   f"splits {splits} sequence {b}")
    assert _lib.read_errors() == 0


def test_small_grids_back_to_back_split_counts():
    """Small grids (the staged kernel) at 4 to 32 splits, merged by k_mla_merge: calls
    alternate between split counts, batch 1 and 2, and head counts 16 and 32 (one and two
    chunks), with no synchronisation in between, and every call must match the oracle
    (splits past the context publish empty partials)."""
    cases = []
    for heads, ctx_lens in ((16, [320]), (16, [333, 17]), (32, [320])):
        q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, heads, DL, DR, 16, torch.bfloat16, seed=20 + heads)
        cases.append((heads, ctx_lens, q, lat, bt, ctx, tuple(t.to(DEV) for t in (q, lat, bt, ctx))))
    outs = []
    for rnd in range(2):
        for splits in (4, 6, 8, 10, 16, 20, 32):
            for heads, ctx_lens, q, lat, bt, ctx, dev_in in cases:
                outs.append((heads, ctx_lens, splits, q, lat, bt, ctx,
                             mla_decode(*dev_in[:2], dev_in[2], dev_in[3], SCALE, DL, num_splits=splits)))
    torch.cuda.synchronize()
    for heads, ctx_lens, splits, q, lat, bt, ctx, got in outs:
        _check(got, q[..., :DL], q[..., DL:], lat, bt, ctx, SCALE, DL, True,
               f"spread merge heads {heads} ctx {ctx_lens} splits {splits}")
    assert _lib.read_errors() == 0


@pytest.mark.parametrize("splits", [1, 2, 3])
def test_interpreter_geometry_fp32(splits):
    """tests/test_mla_triton.py's geometry (H 4, DL 32, DR 16, fp32), its contexts and split
    counts: the fp32 kernel and its merge."""
    for ctx_lens in ([1], [16], [17, 5, 40], [33, 64, 3, 50], [70, 9, 48]):
        _say(f"mla decode fp32 small ctx {ctx_lens} splits {splits}")
        q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, 4, 32, 16, 16, torch.float32, seed=2, amp=1.0)
        got = mla_decode(q.to(DEV), lat.to(DEV), bt.to(DEV), ctx.to(DEV), 0.3, 32, num_splits=splits)
        torch.cuda.synchronize()
        _check(got, q[..., :32], q[..., 32:], lat, bt, ctx, 0.3, 32, False, f"ctx {ctx_lens}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fp32_cache_and_unaligned_strides_take_the_fp32_kernel(dtype):
    """fp32 at the MFMA geometry, and bf16 with a q row stride that is not a multiple of 8
    elements: both run the fp32 kernel and match at its tolerance."""
    ctx_lens = [40, 300, 17]
    q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, H, DL, DR, 16, dtype, seed=3)
    if dtype == torch.bfloat16:
        wide = torch.zeros(len(ctx_lens), H, DL + DR + 3, dtype=dtype)
        wide[..., :DL + DR] = q
        qd = wide.to(DEV)[..., :DL + DR]  # head stride 579: unaligned
    else:
        qd = q.to(DEV)
    for splits in (1, 3):
        _say(f"mla decode fp32 kernel {dtype} splits {splits}")
        got = mla_decode(qd, lat.to(DEV), bt.to(DEV), ctx.to(DEV), SCALE, DL, num_splits=splits)
        torch.cuda.synchronize()
        _check(got, q[..., :DL], q[..., DL:], lat, bt, ctx, SCALE, DL, False, f"splits {splits}")


@pytest.mark.parametrize("heads", [1, 20, 128])
def test_head_counts(heads):
    """One head (15 padded MFMA columns), 20 heads (a full and a partial 16-head chunk) and
    DeepSeek-V3's 128 heads (8 chunks re-reading each row), at one split, the default and
    5 (merged by its own launch; with one head, 15 partial rows put the partial block 8
    bytes past a 16-byte boundary)."""
    ctx_lens = [77, 513, 1]
    q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, heads, DL, DR, 16, torch.bfloat16, seed=4)
    for splits in (1, None, 5):
        _say(f"mla decode heads {heads} splits {splits}")
        got = mla_decode(q.to(DEV), lat.to(DEV), bt.to(DEV), ctx.to(DEV), SCALE, DL, num_splits=splits)
        torch.cuda.synchronize()
        _check(got, q[..., :DL], q[..., DL:], lat, bt, ctx, SCALE, DL, True, f"heads {heads}")


def test_pair_form_with_strided_views_and_block_64():
    """q as the backend passes it (mla_triton.py:226-229): q_c the transposed output of a
    bmm over heads ([H, B, DL] storage), q_pe a view into a wider rope'd row; block size
    64; an output buffer with a padded head stride."""
    ctx_lens = [129, 64, 1000, 3]
    B = len(ctx_lens)
    q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, H, DL, DR, 64, torch.float16, seed=5)
    q_c = q[..., :DL].transpose(0, 1).contiguous().to(DEV).transpose(0, 1)  # strides (DL, B*DL, 1)
    rows = torch.zeros(B, H, 192, dtype=torch.float16)
    rows[..., 128:] = q[..., DL:]
    q_pe = rows.to(DEV)[..., 128:]
    out = torch.full((B, H, DL + 8), float("nan"), dtype=torch.float16, device=DEV)
    for splits in (1, 5):
        _say(f"mla decode pair form block 64 splits {splits}")
        got = mla_decode((q_c, q_pe), lat.to(DEV), bt.to(DEV), ctx.to(DEV), SCALE, DL, num_splits=splits,
                         out=out[..., :DL])
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        _check(got, q[..., :DL], q[..., DL:], lat, bt, ctx, SCALE, DL, True, f"splits {splits}")
    assert bool(out[..., DL:].isnan().all())  # the padding past each head row is untouched


def test_padded_table_width_and_zero_context():
    """Tables padded to a wide width (graph-capture layout: the split partitions the real
    context) and a zero-length context, which yields NaN rows as the reference's 0/0."""
    ctx_lens = [300, 0, 45]
    q, lat, bt, ctx = gen.mla_decode_inputs(ctx_lens, H, DL, DR, 16, torch.bfloat16, seed=6, table_width=256)
    for splits in (1, None, 16):
        _say(f"mla decode padded table splits {splits}")
        got = mla_decode(q.to(DEV), lat.to(DEV), bt.to(DEV), ctx.to(DEV), SCALE, DL, num_splits=splits).cpu()
        assert bool(got[1].isnan().all())
        keep = [0, 2]
        _check(got[keep], q[keep, :, :DL], q[keep, :, DL:], lat, bt[keep], ctx[keep], SCALE, DL, True,
               f"splits {splits}")


def test_bad_context_and_block_id_raise(monkeypatch):
    q, lat, bt, ctx = gen.mla_decode_inputs([40, 20], H, DL, DR, 16, torch.bfloat16, seed=7)
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    bad_ctx = ctx.clone()
    bad_ctx[1] = 10_000  # past the table
    _say("mla decode bad context")
    with pytest.raises(IndexError):
        mla_decode(q.to(DEV), lat.to(DEV), bt.to(DEV), bad_ctx.to(DEV), SCALE, DL)
    bad_bt = bt.clone()
    bad_bt[0, 1] = lat.shape[0] + 7
    _say("mla decode bad block id")
    with pytest.raises(IndexError):
        mla_decode(q.to(DEV), lat.to(DEV), bad_bt.to(DEV), ctx.to(DEV), SCALE, DL)


def test_split_rule_shapes_only(monkeypatch):
    monkeypatch.delenv("EMBERSERVE_TRITON_SPLITS", raising=False)
    dev = torch.device(DEV)
    cus = num_sms(dev)
    assert mla_num_splits(128, dev) == max(1, cus // 128)
    assert mla_num_splits(1, dev, max_context=16) == 1
    assert mla_num_splits(1, dev, max_context=320) == min(8, cus)  # ~sqrt(context / 4)
    assert mla_num_splits(1, dev, max_context=4096) == min(32, cus)
    assert mla_num_splits(1, dev, max_context=1 << 20) == min(128, cus)
    assert mla_num_splits(4, dev, num_heads=128, max_context=1 << 20) == max(1, min(128, cus // 32))


def test_graph_replay_with_changing_contexts():
    """Captured once with a padded table (as CUDA-graph decode captures it), replayed with
    new q, contexts and table contents (eager work and syncs between replays): every replay
    equals the eager call."""
    B, width = 8, 64
    q, lat, bt, ctx = gen.mla_decode_inputs([200] * B, H, DL, DR, 16, torch.bfloat16, seed=8, table_width=width,
                                            spare_blocks=B * width)
    qd, latd = q.to(DEV), lat.to(DEV)
    btd, ctxd = bt.to(DEV), ctx.to(DEV)
    out = torch.empty(B, H, DL, dtype=torch.bfloat16, device=DEV)
    splits = mla_num_splits(B, torch.device(DEV), max_context=width * 16)

    def step():
        return mla_decode(qd, latd, btd, ctxd, SCALE, DL, num_splits=splits, out=out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    gsplit = torch.Generator().manual_seed(9)
    for rep in range(3):
        new_ctx = torch.randint(1, width * 16 + 1, (B,), generator=gsplit, dtype=torch.int32)
        perm = torch.randperm(lat.shape[0], generator=gsplit)[:B * width].view(B, width).to(torch.int32)
        qd.copy_((torch.randn(B, H, DL + DR, generator=gsplit) * 0.5).to(torch.bfloat16).to(DEV))
        ctxd.copy_(new_ctx.to(DEV))
        btd.copy_(perm.to(DEV))
        _say(f"mla decode graph replay {rep}")
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = step().clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"
