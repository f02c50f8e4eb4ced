"""The `torch.ops.emberserve.*` registrations (emberserve_amd.torch_ops): schema and
mutation declarations, fake kernels and AOT dispatch checked by `torch.library.opcheck`,
results against the oracle, and a `torch.compile` trace through the fake kernels. CPU
tensors here (the eager forms); the GPU tests at the bottom run the same checks on the
HIP library."""

from __future__ import annotations

import pytest
import torch

from emberserve_amd import torch_ops  # noqa: F401  (registers torch.ops.emberserve)
from oracle import inputs as gen
from oracle import ref_ops as ref

OPS = torch.ops.emberserve


def _cases(device: str):
    """(op, args) for every registered op at small shapes, on `device`."""
    d = device
    bf = torch.bfloat16
    x, r, w = gen.add_rmsnorm_inputs(6, 64, bf, seed=1)
    q, k, pos = gen.rope_inputs(5, 4, 2, 64, 128, bf, seed=2)
    cos, sin = ref.rope_tables(64, 128, 1e4)
    g = gen.silu_inputs(3, 32, bf, seed=3)
    ids, tab = gen.embedding_inputs(7, 50, 32, bf, seed=4)
    qkv, qw, kw, pos2 = gen.qkv_inputs(5, 4, 2, 64, 128, bf, seed=5)
    kv_a, qm, wm, pos3 = gen.mla_inputs(4, 2, 32, 64, 128, 128, bf, seed=6)
    mcos, msin = ref.rope_tables(64, 128, 5e4)
    kc = torch.zeros(4, 16, 2, 64, dtype=bf)
    slots = torch.tensor([3, 17, 40, 9, 60], dtype=torch.int64)
    lat_cache = torch.zeros(4, 16, 192, dtype=bf)
    latent = gen.normal((5, 192), bf, 7)
    qd, kcd, vcd, bt, cl = gen.decode_inputs([5, 19], 4, 2, 64, 16, torch.float32, seed=8)
    qa, lat, bt2, cl2 = gen.mla_decode_inputs([5, 40], 4, 32, 16, 16, torch.float32, seed=9)
    gx, gw = gen.gate_up_inputs(3, 128, 64, bf, seed=10)
    from emberserve_amd.moe import moe_align
    mw = torch.stack([gen.gate_up_inputs(1, 128, 64, bf, seed=11 + e)[1] for e in range(4)])
    mids = torch.tensor([[0, 2], [3, 2], [1, 0]])
    sid, bex, nv = moe_align(mids, 4)

    def dev(*ts):
        return tuple(t.to(d) for t in ts)
    xq = qkv.to(d)
    return [
        ("rmsnorm", dev(x, w) + (1e-6,)),
        ("fused_add_rmsnorm", dev(x, r, w) + (1e-6,)),
        ("rope", dev(q.clone(), k.clone(), cos, sin, pos)),
        ("silu_and_mul", dev(g)),
        ("embedding", dev(ids, tab)),
        ("qk_norm_rope", (xq[:, :256].view(5, 4, 64).clone(), xq[:, 256:384].view(5, 2, 64).clone())
         + dev(qw, kw) + (1e-6,) + dev(cos, sin, pos2)),
        ("mla_latent_rope", dev(kv_a[:, :128].contiguous(), kv_a[:, 128:].contiguous().view(4, 1, 64),
                                qm[..., 32:].contiguous(), wm) + (1e-6,) + dev(mcos, msin, pos3)),
        ("kv_cache_write", dev(k, k.clone(), slots, kc, kc.clone())),
        ("latent_cache_write", dev(latent, slots, lat_cache)),
        ("paged_attention_decode", dev(qd, kcd, vcd, bt, cl) + (0.125, None)),
        ("mla_decode", dev(qa[..., :32].contiguous(), qa[..., 32:].contiguous(), lat, bt2, cl2) + (0.3, 32, None)),
        ("gate_up_silu", dev(gx, gw)),
        ("moe_gate_up_silu", dev(gx, mw, sid, bex) + (nv, 2)),
        ("moe_align", dev(mids) + (4, 16)),
        ("fused_moe_gate_up", dev(gx, mids, mw)),
    ]


@pytest.mark.parametrize("name", [c[0] for c in _cases("cpu")])
def test_opcheck_cpu(name):
    op, args = next((getattr(OPS, n), a) for n, a in _cases("cpu") if n == name)
    torch.library.opcheck(op, args)


def test_registered_ops_match_the_oracle_cpu():
    c = dict(_cases("cpu"))
    x, w, eps = c["rmsnorm"]
    torch.testing.assert_close(torch_ops.rmsnorm(x, w, eps), ref.rmsnorm(x, w, eps), rtol=0, atol=0)
    q, k, cos, sin, pos = c["rope"]
    want_q, want_k = ref.rope(q.clone(), k.clone(), cos, sin, pos)
    got_q, got_k = torch_ops.rope(q, k, cos, sin, pos)
    assert got_q is q and got_k is k  # in place, returned as the reference's rope does
    torch.testing.assert_close(q, want_q, rtol=0, atol=0)
    torch.testing.assert_close(k, want_k, rtol=0, atol=0)
    qa, qp, lat, bt, cl, scale, dl, _ = c["mla_decode"]
    torch.testing.assert_close(torch_ops.mla_decode(qa, qp, lat, bt, cl, scale, dl),
                               ref.mla_decode(qa, qp, lat, bt, cl, scale, dl), rtol=0, atol=1e-6)
    kk, vv, slots, kc, vc = c["kv_cache_write"]
    torch_ops.kv_cache_write(kk, vv, slots, kc, vc)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    ref.kv_cache_write(kk, vv, slots, kc2, vc2)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)


def test_compile_traces_through_the_fake_kernels():
    """aot_eager: Dynamo + AOTAutograd functionalize the in-place ops from their schemas
    and size every output from the fake kernels; the compiled function equals eager."""
    c = dict(_cases("cpu"))
    x, r, w, eps = c["fused_add_rmsnorm"]
    q, k, cos, sin, pos = c["rope"]

    def layer(x, r, q, k):
        n, r2 = torch_ops.fused_add_rmsnorm(x, r, w, eps)
        q, k = torch_ops.rope(q, k, cos, sin, pos)
        return n, r2, q * 2, k

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    got = compiled(x, r, q.clone(), k.clone())
    want = layer(x, r, q.clone(), k.clone())
    for a, b in zip(got, want):
        assert torch.equal(a, b)


# ---- the same on the GPU --------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("name", [c[0] for c in _cases("cpu")])
def test_opcheck_gpu(name):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    print(f"opcheck {name} on the GPU", flush=True)
    op, args = next((getattr(OPS, n), a) for n, a in _cases("cuda") if n == name)
    torch.library.opcheck(op, args)


@pytest.mark.gpu
def test_registered_ops_run_the_hip_library_and_capture():
    """On GPU tensors the registered ops reach libember_ops.so (a raising stand-in for the
    eager forms proves it), and a HIP graph of them replays to the eager result."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from emberserve_amd import eager, ops
    c = dict(_cases("cuda"))
    x, r, w, eps = c["fused_add_rmsnorm"]
    q, k, cos, sin, pos = c["rope"]
    saved = (ops.fused_add_rmsnorm_torch, ops.rope_torch)

    def boom(*a, **kw):
        raise AssertionError("eager fallback ran on a GPU tensor")
    ops.fused_add_rmsnorm_torch = ops.rope_torch = boom
    try:
        def step():
            n, r2 = torch_ops.fused_add_rmsnorm(x, r, w, eps)
            torch_ops.rope(q, k, cos, sin, pos)
            return n, r2
        n0, r0 = step()
        q0, k0 = q.clone(), k.clone()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        q.copy_(q0)
        k.copy_(k0)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            n1, r1 = step()
        for _ in range(3):
            q.copy_(q0)
            k.copy_(k0)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(n1, n0) and torch.equal(r1, r0)
        want_q, want_k = eager.rope_torch(q0, k0, cos, sin, pos)
    finally:
        ops.fused_add_rmsnorm_torch, ops.rope_torch = saved
    torch.testing.assert_close(q.cpu(), want_q.cpu(), rtol=0, atol=0)
    assert q.data_ptr() != q0.data_ptr()
