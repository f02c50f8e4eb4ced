"""GPU parity of the mixed-step query pack / output unpack (emberserve_amd.mixed, the data
movement of paged_flash.py:242-289) against the oracle's restatement of the reference's
torch sequence. Index work: bit-exact."""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib  # noqa: E402
from emberserve_amd.mixed import MixedRows, pack_queries, prefill_kvcache, unpack_outputs  # noqa: E402
from emberserve_amd.paged_decode import paged_attention_decode  # noqa: E402
from oracle import inputs as gen  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402
from tests.helpers import assert_bitexact  # noqa: E402

DEV = "cuda"


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield


def _rand(*shape, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


MIXES = {
    "decode only": [1] * 39,
    "prefill only": [300],
    "39 decodes + one 300-token prompt": [1] * 39 + [300],
    "ragged prefills among decodes": [1, 17, 1, 1, 64, 3, 1, 2],
    "two prompts": [128, 5],
}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mix", list(MIXES))
def test_pack_unpack_match_the_reference_sequence(dtype, mix):
    """q as the strided view of a fused qkv buffer (Qwen2.5-7B heads: 28 q + 2 x 4 kv,
    D = 128): the pack equals index_select + new_zeros + slice copies, the unpack equals
    index_copy_ + slice copies, bit for bit."""
    lens = MIXES[mix]
    T, H, Hkv, D = sum(lens), 28, 4, 128
    _say(f"mixed pack/unpack {mix} {dtype}")
    qkv = _rand(T, (H + 2 * Hkv) * D, dtype=dtype, seed=T)
    q = qkv[:, :H * D].view(T, H, D)
    want_dec, want_pad = ref.mixed_pack(q, lens)
    plan = MixedRows(lens, DEV)
    qd = qkv.to(DEV)[:, :H * D].view(T, H, D)
    got_dec, got_pad = pack_queries(qd, plan)
    for got, want, name in ((got_dec, want_dec, "q_dec"), (got_pad, want_pad, "q_pad")):
        assert (got is None) == (want is None), name
        if want is not None:
            assert_bitexact(got, want, name)
    # attention outputs: any values; the unpack must put each row where the reference does
    o_dec = _rand(plan.num_dec, 1, H, D, dtype=dtype, seed=1) if plan.num_dec else None
    o_pad = _rand(plan.num_pre, plan.max_q, H, D, dtype=dtype, seed=2) if plan.num_pre else None
    want = ref.mixed_unpack(torch.zeros(T, H, D, dtype=dtype), o_dec, o_pad, lens)
    out = torch.full((T, H, D), float("nan"), dtype=dtype, device=DEV)
    unpack_outputs(out, None if o_dec is None else o_dec.to(DEV), None if o_pad is None else o_pad.to(DEV), plan)
    assert_bitexact(out, want, "out")
    assert _lib.read_errors() == 0


def test_row_kernels_unaligned_rows_and_bad_index(monkeypatch):
    """Rows of 7 fp16 elements (14 bytes: the 2-byte unit path), and an index past the end:
    a zero row for the gather, a dropped row for the scatter, EMBER_ERR_ROW_INDEX set and
    IndexError with index checks on."""
    lens = [1, 3, 1]
    src = _rand(5, 7, dtype=torch.float16, seed=3)
    plan = MixedRows(lens, DEV)
    got_dec, got_pad = pack_queries(src.to(DEV), plan)
    want_dec, want_pad = ref.mixed_pack(src, lens)
    assert_bitexact(got_dec, want_dec, "q_dec (2-byte units)")
    assert_bitexact(got_pad, want_pad, "q_pad (2-byte units)")
    plan.rows[1] = 99  # corrupt one slot: past the end of q
    monkeypatch.setenv("EMBERSERVE_CHECK_INDICES", "1")
    with pytest.raises(IndexError):
        pack_queries(src.to(DEV), plan)
    out = torch.zeros(5, 7, dtype=torch.float16, device=DEV)
    with pytest.raises(IndexError):
        unpack_outputs(out, got_dec, got_pad, plan)
    # the valid rows still landed; slot 1's row (index 99) went nowhere
    assert_bitexact(out[0], src[0], "row 0 still written")


def test_prefill_kvcache_with_the_decode_kernel():
    """The whole data path of one mixed layer: decode rows through paged_attention_decode
    (cache geometry of Qwen3-8B, 32q/8kv x 128), the padded prefill rows through a stand-in
    attention (scaled identity), outputs back in packed order."""
    lens = [1, 1, 6, 1]
    T, H, Hkv, D = sum(lens), 32, 8, 128
    dec_idx = [i for i, n in enumerate(lens) if n == 1]
    q = _rand(T, H, D, dtype=torch.bfloat16, seed=5).to(DEV)
    _, kc, vc, bt, cl = gen.decode_inputs([70, 33, 150], H, Hkv, D, 16, torch.bfloat16, seed=6)
    kc, vc, bt, cl = (t.to(DEV) for t in (kc, vc, bt, cl))
    plan = MixedRows(lens, DEV)

    def decode(qd):
        return paged_attention_decode(qd.view(-1, H, D), kc, vc, bt, cl, D ** -0.5).view(-1, 1, H, D)

    out = prefill_kvcache(q, plan, decode, lambda qp: qp * 2)
    starts = [sum(lens[:i]) for i in range(len(lens))]
    want_dec = paged_attention_decode(q[[starts[i] for i in dec_idx]], kc, vc, bt, cl, D ** -0.5)
    assert_bitexact(out[[starts[i] for i in dec_idx]], want_dec, "decode rows")
    assert_bitexact(out[2:8], q[2:8] * 2, "prefill rows")


def test_pack_unpack_in_a_graph_replay():
    """Recorded once with a per-step plan, replayed with new q values each time (eager work
    and syncs in between): every replay equals the eager launches."""
    lens = [1] * 7 + [20, 1, 9]
    T, H, D = sum(lens), 4, 64
    plan = MixedRows(lens, DEV)
    q = torch.empty(T, H, D, dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(q)
    q.copy_(_rand(T, H, D, dtype=torch.bfloat16, seed=9).to(DEV))

    def step():
        q_dec, q_pad = pack_queries(q, plan)
        return unpack_outputs(out, q_dec * 3, q_pad - 1, plan)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for seed in range(10, 13):
        q.copy_(_rand(T, H, D, dtype=torch.bfloat16, seed=seed).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = step().clone()
        torch.cuda.synchronize()
        assert_bitexact(got, want, f"replay {seed}")
