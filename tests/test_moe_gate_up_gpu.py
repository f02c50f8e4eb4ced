"""GPU parity of the routed experts' fused gate_up + silu_and_mul (ember_moe_gate_up_silu)
over the moe_align layout, against the oracle `moe_gate_up_silu` (per assignment, float64
dot products rounded to the dtype, then silu_and_mul), at the reference's MoE test geometry
(tests/test_moe_triton_gpu.py:22-29: Moonlight, H 2048, I 1408, 64 experts, top-6). The
tolerance is tests.helpers.check_gate_up's."""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib  # noqa: E402
from emberserve_amd.moe import (GEMM_FROM, fused_moe_gate_up, moe_align, moe_gate_up_silu,  # noqa: E402
                                moe_gate_up_silu_direct, moe_gate_up_silu_gemm, pack_moe_gate_up_weight)
from oracle import ref_ops as ref  # noqa: E402
from tests.helpers import check_gate_up  # noqa: E402

DEV = "cuda"
H, I, E, K = 2048, 1408, 64, 6


def _inputs(n, dtype, seed, experts=E):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, H, generator=g) * 0.5).to(dtype)
    w = (torch.randn(experts, 2 * I, H, generator=g) * 1.5 / H ** 0.5).to(dtype)
    ids = torch.stack([torch.randperm(experts, generator=g)[:K] for _ in range(n)])
    return x, w, ids


def _check(got, x, w, ids, what):
    rows = [(t, int(ids[t, c])) for t in range(ids.shape[0]) for c in range(ids.shape[1])]
    gu = torch.cat([(x[t:t + 1].double() @ w[e].double().T).to(x.dtype) for t, e in rows])
    absdot = torch.cat([x[t:t + 1].double().abs() @ w[e].double().abs().T for t, e in rows])
    check_gate_up(got, ref.moe_gate_up_silu(x, ids, w), gu, absdot, H, what, parts=0)


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield
    assert _lib.read_errors() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 8, 37])
def test_moe_gate_up_matches_oracle(dtype, n):
    """test_moe_triton_gpu.py:33-43's token counts (200 -> 37 to keep the oracle quick)."""
    print(f"moe gate_up n={n} {dtype}", flush=True)
    x, w, ids = _inputs(n, dtype, seed=n)
    dx, dids, dw = x.to(DEV), ids.to(DEV), w.to(DEV)
    rows = [(t, int(ids[t, c])) for t in range(n) for c in range(K)]
    want = ref.moe_gate_up_silu(x, ids, w)
    gu = torch.cat([(x[t:t + 1].double() @ w[e].double().T).to(x.dtype) for t, e in rows])
    absdot = torch.cat([x[t:t + 1].double().abs() @ w[e].double().abs().T for t, e in rows])
    for splits in ((None, 1, 2, 4) if n < 37 else (None, 4)):
        got = fused_moe_gate_up(dx, dids, dw, num_splits=splits)
        assert got.shape == (n * K, I)
        check_gate_up(got, want, gu, absdot, H, f"n={n} splits={splits}", parts=0)


def test_moe_gate_up_some_experts_get_no_tokens():
    """Every token routed to the same six experts: 58 experts idle, one expert's block
    holds all of a choice's rows (tests/test_moe.py:112-118's case)."""
    x, w, _ = _inputs(20, torch.bfloat16, seed=5)
    ids = torch.tensor([[3, 9, 17, 40, 41, 63]] * 20)
    got = fused_moe_gate_up(x.to(DEV), ids.to(DEV), w.to(DEV))
    _check(got, x, w, ids, "six experts")


def test_moe_gate_up_split_graph_replay():
    """Split partials and counters across captured replays, with other work in between:
    every replay matches the eager result (the counters return to zero)."""
    x, w, ids = _inputs(2, torch.bfloat16, seed=8)
    dx, dids, dw = x.to(DEV), ids.to(DEV), w.to(DEV)
    sorted_ids, block_expert, nv = moe_align(dids, E)
    want = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=4)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=4)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        got = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=4)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
        assert torch.equal(moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=4), want)


def test_moe_gate_up_bad_assignment_sets_error_bit():
    """An assignment id whose token row is past x reads row 0 and flags EMBER_ERR_ROW_INDEX
    (every kernel still exits normally)."""
    x, w, ids = _inputs(4, torch.bfloat16, seed=2)
    sorted_ids, block_expert, nv = moe_align(ids.to(DEV), E)
    moe_gate_up_silu(x[:2].to(DEV), w.to(DEV), sorted_ids, block_expert, nv, K)  # rows 2, 3 missing
    torch.cuda.synchronize()
    assert _lib.read_errors(clear=True) & _lib.ERR_ROW_INDEX


def test_moe_gemm_bad_assignment_sets_error_bit():
    """The prefill GEMM through the C ABI with num_tokens 2 while the layout holds the
    assignments of 4 tokens: rows 2 and 3 read token 0 and flag EMBER_ERR_ROW_INDEX."""
    from emberserve_amd.ops import _launch
    x, w, ids = _inputs(4, torch.bfloat16, seed=3)
    dx, dw = x.to(DEV), w.to(DEV)
    sorted_ids, block_expert, nv = moe_align(ids.to(DEV), E, 128)
    out = torch.empty((nv, I), dtype=dx.dtype, device=DEV)
    _launch("ember_moe_gate_up_silu_gemm", _lib.load().ember_moe_gate_up_silu_gemm, dx.device,
            dx.data_ptr(), dx.stride(0), 2, dw.data_ptr(), dw.stride(0), dw.stride(1), _lib.dtype_tag(dx.dtype),
            E, H, I, sorted_ids.data_ptr(), block_expert.data_ptr(), block_expert.numel(), 128, nv, K, 128,
            out.data_ptr(), out.stride(0))
    torch.cuda.synchronize()
    assert _lib.read_errors(clear=True) & _lib.ERR_ROW_INDEX


# ---- the packed expert layout (ember_moe_gate_up_silu_pack_weight / _packed) ----
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_moe_pack_weight_matches_the_oracle_permutation(dtype):
    g = torch.Generator().manual_seed(3)
    w = torch.randn(5, 2 * 192, 256, generator=g).to(dtype)
    got = pack_moe_gate_up_weight(w.to(DEV)).packed.cpu()
    assert torch.equal(got.view(torch.int16), ref.pack_moe_gate_up_weight(w).view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 2, 8, 37])
def test_moe_packed_equals_the_row_kernel(dtype, n):
    """Same grid, products and order: bit-identical to ember_moe_gate_up_silu at every split
    count, and within the oracle's tolerance."""
    print(f"moe packed n={n} {dtype}", flush=True)
    x, w, ids = _inputs(n, dtype, seed=100 + n)
    dx, dids, dw = x.to(DEV), ids.to(DEV), w.to(DEV)
    packed = pack_moe_gate_up_weight(dw)
    sorted_ids, block_expert, nv = moe_align(dids, E)
    for splits in (1, 2, 4):
        a = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=splits)
        b = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=splits, packed=packed)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"n={n} splits={splits}"
    if n <= 8:
        _check(fused_moe_gate_up(dx, dids, dw, packed=packed), x, w, ids, f"packed n={n}")


def test_moe_packed_bad_assignment_sets_error_bit():
    x, w, ids = _inputs(4, torch.bfloat16, seed=2)
    dw = w.to(DEV)
    sorted_ids, block_expert, nv = moe_align(ids.to(DEV), E)
    moe_gate_up_silu(x[:2].to(DEV), dw, sorted_ids, block_expert, nv, K, packed=pack_moe_gate_up_weight(dw))
    torch.cuda.synchronize()
    assert _lib.read_errors(clear=True) & _lib.ERR_ROW_INDEX


@pytest.mark.parametrize("n", [1, 3, 37])
def test_moe_packed_half_slabs_equal_full_slabs(n):
    """Two-wave workgroups over 32 columns run every wave's rows over the whole k range as the
    four-wave ones do: bit-identical (one split)."""
    x, w, ids = _inputs(n, torch.bfloat16, seed=300 + n)
    dx, dw = x.to(DEV), w.to(DEV)
    packed = pack_moe_gate_up_weight(dw)
    sorted_ids, block_expert, nv = moe_align(ids.to(DEV), E)
    a = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=1, packed=packed, half_slabs=False)
    b = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=1, packed=packed, half_slabs=True)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with pytest.raises(ValueError):
        moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=2, packed=packed, half_slabs=True)


@pytest.mark.parametrize("id_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("n", [1, 3, 8, 12])
@pytest.mark.parametrize("half", [False, True])
def test_moe_direct_equals_the_aligned_path(id_dtype, n, half):
    """Each expert's assignments in groups of 16, computed by the workgroups of each group's
    first assignment: the same rows and products as its aligned block, so bit-identical."""
    x, w, ids = _inputs(n, torch.bfloat16, seed=400 + n)
    dx, dw, dids = x.to(DEV), w.to(DEV), ids.to(DEV)
    packed = pack_moe_gate_up_weight(dw)
    sorted_ids, block_expert, nv = moe_align(dids, E)
    want = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=1, packed=packed, half_slabs=False)
    got = moe_gate_up_silu_direct(dx, dids.to(id_dtype), packed, half_slabs=half)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # fused_moe_gate_up takes this path up to DIRECT_MAX_TOKENS tokens over packed experts
    assert torch.equal(fused_moe_gate_up(dx, dids, dw, packed=packed).view(torch.int16), want.view(torch.int16))


def test_moe_direct_groups_longer_than_16():
    """40 tokens whose first two choices are experts 0 and 1: runs of 40 assignments, three
    groups each (16 + 16 + 8), every group's rows in assignment order."""
    n = 40
    x, w, ids = _inputs(n, torch.bfloat16, seed=41)
    ids[:, 0], ids[:, 1] = 0, 1
    ids[:, 2:] = torch.stack([torch.randperm(E - 2, generator=torch.Generator().manual_seed(t))[:K - 2] + 2
                              for t in range(n)])
    dx, dw, dids = x.to(DEV), w.to(DEV), ids.to(DEV)
    packed = pack_moe_gate_up_weight(dw)
    sorted_ids, block_expert, nv = moe_align(dids, E)
    want = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, K, num_splits=1, packed=packed, half_slabs=False)
    for half in (False, True):
        got = moe_gate_up_silu_direct(dx, dids, packed, half_slabs=half)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), half


def test_moe_direct_rejects_more_than_256_assignments():
    x, w, ids = _inputs(43, torch.bfloat16, seed=43)  # 258 assignments
    with pytest.raises(RuntimeError):
        moe_gate_up_silu_direct(x.to(DEV), ids.to(DEV), pack_moe_gate_up_weight(w.to(DEV)))


def test_fused_moe_gate_up_large_top_k_takes_the_aligned_path():
    """12 tokens at top-24 (288 assignments, past the direct kernel's 256): fused_moe_gate_up
    over packed experts must fall through to the aligned path rather than raise."""
    n, k = 12, 24
    x, w, _ = _inputs(n, torch.bfloat16, seed=44)
    g = torch.Generator().manual_seed(44)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(n)])
    dx, dw, dids = x.to(DEV), w.to(DEV), ids.to(DEV)
    packed = pack_moe_gate_up_weight(dw)
    sorted_ids, block_expert, nv = moe_align(dids, E)
    want = moe_gate_up_silu(dx, dw, sorted_ids, block_expert, nv, k, num_splits=1, packed=packed, half_slabs=False)
    got = fused_moe_gate_up(dx, dids, dw, packed=packed)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    _check(got.cpu(), x, w, ids, "top-24")


def test_moe_direct_bad_expert_sets_error_bit():
    x, w, ids = _inputs(1, torch.bfloat16, seed=5)
    dw = w.to(DEV)
    bad = ids.clone()
    bad[0, 2] = E + 3
    moe_gate_up_silu_direct(x.to(DEV), bad.to(DEV), pack_moe_gate_up_weight(dw))
    torch.cuda.synchronize()
    assert _lib.read_errors(clear=True) & _lib.ERR_EXPERT_ID


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 5, 37])
def test_moe_gemm_matches_oracle(dtype, n):
    """The prefill GEMM over 256-row blocks (mostly padding at these sizes) against the
    oracle, at both column tiles."""
    print(f"moe gemm n={n} {dtype}", flush=True)
    x, w, ids = _inputs(n, dtype, seed=100 + n)
    for rows, tile in ((256, 64), (256, 128), (128, 128)):
        got = moe_gate_up_silu_gemm(x.to(DEV), w.to(DEV), ids.to(DEV), column_tile=tile, block_rows=rows).cpu()
        _check(got, x, w, ids, f"moe gemm n={n} tile {rows}x{tile}")


@pytest.mark.parametrize("n,experts,skew", [(300, 64, False), (700, 64, False), (600, 8, True)])
def test_moe_gemm_equals_the_row_kernel(n, experts, skew):
    """Bit-identical to the 16-block row kernel at one k split (every accumulator over k in
    order): a few hundred tokens, runs spanning several 256-row blocks, and skewed routing
    whose runs cross many blocks."""
    print(f"moe gemm vs row n={n} E={experts} skew={skew}", flush=True)
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(n, H, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    w = (torch.randn(experts, 2 * I, H, generator=g) * 1.5 / H ** 0.5).to(torch.bfloat16).to(DEV)
    if skew:
        ids = torch.stack([torch.randperm(experts, generator=g)[:K] for _ in range(n)])
        ids[: n // 2] = torch.arange(K)  # half the tokens on experts 0-5
    else:
        ids = torch.stack([torch.randperm(experts, generator=g)[:K] for _ in range(n)])
    ids = ids.to(DEV)
    si, be, nv = moe_align(ids, experts)
    want = moe_gate_up_silu(x, w, si, be, nv, K, num_splits=1)
    packed = pack_moe_gate_up_weight(w)
    for rows, tile in ((256, 64), (256, 128), (128, 128)):
        got = moe_gate_up_silu_gemm(x, w, ids, column_tile=tile, block_rows=rows)
        assert torch.equal(got, want), (rows, tile)
        # over the packed experts (ember_moe_gate_up_silu_gemm_packed), no unpacked weight
        got = moe_gate_up_silu_gemm(x, None, ids, column_tile=tile, block_rows=rows, packed=packed)
        assert torch.equal(got, want), ("packed", rows, tile)


def test_fused_moe_gate_up_takes_the_gemm_at_prefill_sizes(monkeypatch):
    """From GEMM_FROM assignments fused_moe_gate_up runs the GEMM (bit-identical to the
    row kernel at one split); below it the 16-block kernels."""
    n = -(-GEMM_FROM // K)
    x, w, ids = _inputs(n, torch.bfloat16, seed=9)
    dx, dw, dids = x.to(DEV), w.to(DEV), ids.to(DEV)
    calls = []
    import emberserve_amd.moe as moe_mod
    real = moe_mod.moe_gate_up_silu_gemm
    monkeypatch.setattr(moe_mod, "moe_gate_up_silu_gemm", lambda *a, **k: calls.append(1) or real(*a, **k))
    got = fused_moe_gate_up(dx, dids, dw)
    assert calls == [1]
    si, be, nv = moe_align(dids, E)
    assert torch.equal(got, moe_gate_up_silu(dx, dw, si, be, nv, K, num_splits=1))
    fused_moe_gate_up(dx[:8], dids[:8], dw)
    assert calls == [1]


def test_prefill_path_graph_replay_with_fresh_ids():
    """fused_moe_gate_up at a prefill size (the two-launch alignment grid, then the
    expert-block GEMM) captured once and replayed with new routing ids copied into the
    captured input: every replay equals the eager call on the same ids."""
    n = 700  # 4200 assignments: the alignment's grid form and 128-row GEMM blocks
    x, w, ids = _inputs(n, torch.bfloat16, seed=21)
    dx, dw, dids = x.to(DEV), w.to(DEV), ids.to(DEV)
    fused_moe_gate_up(dx, dids, dw)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fused_moe_gate_up(dx, dids, dw)
    g = torch.Generator().manual_seed(22)
    for rep in range(3):
        new = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(n)])
        dids.copy_(new.to(DEV))
        out.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = fused_moe_gate_up(dx, new.to(DEV), dw)
        assert torch.equal(out, want), rep
