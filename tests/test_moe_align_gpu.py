"""GPU parity of the single-launch expert alignment (ember_moe_align) against the oracle's
slot-by-slot layout definition (oracle.ref_ops.moe_align), bit-exact, at the reference's
test cases (tests/test_moe_triton.py:34-48, 100-119; test_moe_triton_gpu.py:66-67) and at
decode and prefill sizes of the Moonlight (64 experts, top-6) and DeepSeek-V3 (256
experts, top-8) routers."""

from __future__ import annotations


import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib  # noqa: E402
from emberserve_amd.moe import moe_align  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402

DEV = "cuda"


def _check(ids, e, bm, dtype=torch.int64):
    print(f"moe_align ids {tuple(ids.shape)} E={e} block {bm} {dtype}", flush=True)
    s, b, nv = moe_align(ids.to(DEV, dtype), e, bm)
    want_s, want_b, want_nv = ref.moe_align(ids, e, bm)
    assert nv == want_nv
    assert s.dtype == torch.int32 and b.dtype == torch.int32
    assert s.cpu().tolist() == want_s
    assert b.cpu().tolist() == want_b


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield
    assert _lib.read_errors() == 0


def test_reference_layout_case():
    _check(torch.tensor([[1, 3], [3, 0], [1, 1], [3, 2]]), 4, 4)


@pytest.mark.parametrize("n", [1, 7, 40, 200])
def test_reference_kernel_cases(n):
    """test_moe_triton.py:105-113: E = 16, k = 4, block 16, seeds = n."""
    ids = torch.randint(0, 16, (n, 4), generator=torch.Generator().manual_seed(n))
    _check(ids, 16, 16)


def test_many_experts_few_tokens():
    _check(torch.tensor([[63, 0], [63, 5]]), 64, 16)


@pytest.mark.parametrize("n,e,k", [(1, 64, 6), (64, 64, 6), (683, 64, 6), (8192, 64, 6), (1, 256, 8),
                                   (128, 256, 8), (4096, 256, 8)])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_router_sizes(n, e, k, dtype):
    """Distinct experts per token (top-k of a router), decode to prefill sizes; 683 x 6 =
    4098 assignments is just past the reference's one-launch limit (moe_triton.py:94)."""
    g = torch.Generator().manual_seed(n + e)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    _check(ids, e, 16, dtype)


def test_skewed_and_block_sizes():
    g = torch.Generator().manual_seed(5)
    skew = (torch.rand(300, 4, generator=g) ** 4 * 32).long()  # most ids on the first experts
    for bm in (1, 4, 16, 64):
        _check(skew, 32, bm)
    _check(torch.full((100, 2), 7), 8, 16)      # every assignment on one expert
    _check(torch.zeros((0, 6), dtype=torch.long), 64, 16)  # no tokens: sentinels only
    _check(torch.randint(0, 1024, (50, 8), generator=g), 1024, 16)  # the most experts supported


def test_bad_expert_id_is_flagged_and_left_out(monkeypatch):
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    ids = torch.tensor([[0, 9], [1, 0]], device=DEV)
    with pytest.raises(IndexError, match="expert id"):
        moe_align(ids, 4, 4)
    monkeypatch.delenv("EMBERSERVE_CHECK_INDICES")
    s, b, nv = moe_align(ids, 4, 4)
    _lib.read_errors(clear=True)
    # assignment 1 (expert 9) is left out; the rest keep the layout of the valid ids
    assert s.cpu().tolist()[:8] == [0, 3, 4, 4, 2, 4, 4, 4] and b.cpu().tolist()[:2] == [0, 1]


def test_align_in_a_graph_replays_fresh_ids():
    """Captured once, replayed with new ids copied into the captured input: every replay
    equals the oracle (no memset nodes; the kernel writes every output slot)."""
    n, e, k = 16, 64, 6
    g = torch.Generator().manual_seed(3)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)]).to(DEV)
    moe_align(ids, e)  # warm up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s, b, _ = moe_align(ids, e)
    for rep in range(4):
        new = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
        ids.copy_(new.to(DEV))
        s.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_s, want_b, _ = ref.moe_align(new, e, 16)
        assert s.cpu().tolist() == want_s and b.cpu().tolist() == want_b, rep


@pytest.mark.parametrize("n,e,k,dtype", [(512, 64, 6, torch.int64), (513, 64, 6, torch.int64),
                                         (1366, 64, 6, torch.int64), (1366, 64, 6, torch.int32),
                                         (8192, 64, 6, torch.int64), (4096, 256, 8, torch.int32),
                                         (20000, 1024, 3, torch.int64), (70000, 64, 6, torch.int64)])
def test_grid_form_matches_one_workgroup_form(n, e, k, dtype):
    """Past 3072 assignments the layout comes from a count launch and a placement launch
    over up to 64 workgroups; it equals the one-workgroup form slot for slot and the oracle
    (512 x 6 is the last one-workgroup size at k = 6, 513 x 6 the first grid size; 70000 x 6
    spreads 420000 assignments over the 64-workgroup cap, past the register-held spans)."""
    g = torch.Generator().manual_seed(n * 7 + e)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    lib = _lib.load()
    print(f"moe_align grid ids {(n, k)} E={e} workspace {lib.ember_moe_align_workspace_bytes(n * k, e)} B",
          flush=True)
    s1, b1, _ = moe_align(ids.to(DEV, dtype), e, grid=True)
    s0, b0, _ = moe_align(ids.to(DEV, dtype), e, grid=False)
    assert torch.equal(s1, s0) and torch.equal(b1, b0)
    if n * k <= 50000:
        want_s, want_b, _ = ref.moe_align(ids, e, 16)
        assert s1.cpu().tolist() == want_s and b1.cpu().tolist() == want_b


def test_grid_form_skewed_and_bad_ids(monkeypatch):
    """All assignments on a few experts (long runs crossing segment boundaries) and an out-of-range
    id in the grid form: flagged, left out, the rest as the one-workgroup form places them."""
    g = torch.Generator().manual_seed(11)
    skew = (torch.rand(3000, 4, generator=g) ** 6 * 12).long()
    s1, b1, _ = moe_align(skew.to(DEV), 12, 16)
    want_s, want_b, _ = ref.moe_align(skew, 12, 16)
    assert s1.cpu().tolist() == want_s and b1.cpu().tolist() == want_b
    bad = skew.clone()
    bad[1234, 2] = 40
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    with pytest.raises(IndexError, match="expert id"):
        moe_align(bad.to(DEV), 12, 16)
    monkeypatch.delenv("EMBERSERVE_CHECK_INDICES")
    s1, b1, _ = moe_align(bad.to(DEV), 12, 16)
    s0, b0, _ = moe_align(bad.to(DEV), 12, 16, grid=False)
    _lib.read_errors(clear=True)
    assert torch.equal(s1, s0) and torch.equal(b1, b0)
    assert (s1 == 1234 * 4 + 2).sum().item() == 0  # assignment 4938 is left out
