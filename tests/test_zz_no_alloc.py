"""The no-allocation paged decode entry point (ember_paged_decode_noalloc), called through the
C ABI, against ember_paged_decode with a caller-allocated workspace: bit-identical outputs
(same kernels, same split count), on two calls in a row, the second smaller, so the shared
scratch's counters and partials carry over from the first call."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib  # noqa: E402
from oracle import inputs as gen  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402

DEV = "cuda"


def _args(q, kc, vc, bt, cl, splits, out):
    return (q.data_ptr(), q.stride(0), q.stride(1), _lib.dtype_tag(q.dtype), kc.data_ptr(), vc.data_ptr(),
            kc.shape[0], kc.shape[1], kc.shape[2], kc.shape[3], kc.stride(0), kc.stride(1), kc.stride(2),
            vc.stride(0), vc.stride(1), vc.stride(2), _lib.dtype_tag(kc.dtype), bt.data_ptr(), bt.stride(0),
            bt.shape[1], cl.data_ptr(), q.shape[0], q.shape[1], float(q.shape[2] ** -0.5), splits, 0)


def _pair(ctx, hq, hkv, d, dtype, splits, seed):
    print(f"noalloc decode ctx={ctx[:4]}.. B={len(ctx)} {hq}q/{hkv}kv x{d} {dtype} splits={splits}", flush=True)
    lib = _lib.load()
    q, kc, vc, bt, cl = (t.to(DEV) for t in gen.decode_inputs(ctx, hq, hkv, d, 16, dtype, seed=seed))
    stream = torch.cuda.current_stream().cuda_stream
    need = lib.ember_paged_decode_workspace_bytes(q.shape[0], hq, d, splits)
    assert 0 <= need <= lib.ember_paged_decode_noalloc_max_bytes()
    ws = torch.zeros(max(need, 16) // 4, dtype=torch.float32, device=DEV)
    want = torch.full_like(q, float("nan"))
    got = torch.full_like(q, float("nan"))
    a = _args(q, kc, vc, bt, cl, splits, want)
    assert lib.ember_paged_decode(*a, ws.data_ptr(), ws.numel() * 4, want.data_ptr(), want.stride(0),
                                  want.stride(1), stream) == 0
    assert lib.ember_paged_decode_noalloc(*a, got.data_ptr(), got.stride(0), got.stride(1), stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # and both are the decode: the fp32 oracle within the bf16/fp16 probability budget
    o = ref.paged_decode(q.float().cpu(), kc.cpu(), vc.cpu(), bt.cpu(), cl.cpu(), d ** -0.5)
    mass = ref.paged_decode_prob_mass(q.float().cpu(), kc.cpu(), vc.cpu(), bt.cpu(), cl.cpu(), d ** -0.5)
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err = (got.float().cpu() - o).abs()
    assert bool((err <= 1.1 * u * (mass + o.abs()) + 1e-4 * mass + 1e-6).all())


def test_noalloc_matches_the_workspace_entry_point_on_consecutive_calls():
    # first call: Qwen3-8B geometry, 8 sequences, 16 splits; second: smaller (3 sequences,
    # 4 splits, ragged contexts) on the scratch the first left behind
    _pair([2048] * 8, 32, 8, 128, torch.bfloat16, 16, seed=1)
    _pair([300, 17, 1025], 32, 8, 128, torch.bfloat16, 4, seed=2)
    # head_dim 64 fp16 (Qwen2.5-0.5B geometry), then one split (no scratch at all)
    _pair([777, 2048], 14, 2, 64, torch.float16, 8, seed=3)
    _pair([512], 14, 2, 64, torch.float16, 1, seed=4)


def test_noalloc_rejects_calls_past_its_scratch():
    lib = _lib.load()
    cap = lib.ember_paged_decode_noalloc_max_bytes()
    q = torch.zeros((1024, 32, 128), dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros((4, 16, 8, 128), dtype=torch.bfloat16, device=DEV)
    bt = torch.zeros((1024, 4), dtype=torch.int32, device=DEV)
    cl = torch.full((1024,), 64, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    assert lib.ember_paged_decode_workspace_bytes(1024, 32, 128, 4) > cap
    st = lib.ember_paged_decode_noalloc(*_args(q, kc, kc, bt, cl, 4, out), out.data_ptr(), out.stride(0),
                                        out.stride(1), torch.cuda.current_stream().cuda_stream)
    assert st == 5 and b"no-allocation" in lib.ember_status_string(5)
