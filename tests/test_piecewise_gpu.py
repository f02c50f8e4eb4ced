"""Segment-graph replay at padded token buckets (emberserve_amd.piecewise; the role of the
reference's PiecewiseGraphRunner, emberserve/attn/piecewise_graphs.py:12-15, 166-184).

Two Qwen3-8B-shaped layers (hidden 4096, 32 q + 8 kv heads x 128, intermediate 12288,
bf16). Pre piece: add + RMSNorm, then qk-norm + rope + paged KV write; post piece: add +
RMSNorm, silu_and_mul, and the row copy that feeds the next layer. Captured at buckets 16,
256 and 8192; the embedding gather runs before the graphs and a stand-in attention (a
copy of the rotated q rows) eagerly between them, on the real rows only. Every step stages
fresh inputs, runs with fewer real rows than its bucket, and must leave the real rows of
every buffer and the whole KV cache bit-identical to the same pieces launched eagerly at
the real row count: cache slots outside the step's real slots keep their old bytes."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib, ops  # noqa: E402
from emberserve_amd.piecewise import SegmentGraphs, stage_rows  # noqa: E402
from emberserve_amd.rope import RotaryEmbedding  # noqa: E402

DEV = torch.device("cuda")
BF = torch.bfloat16
H, HQ, HK, D, I, V = 4096, 32, 8, 128, 12288, 151936
LAYERS = 2
BUCKETS = (16, 256, 8192)
BLOCKS, BLOCK = 1200, 16  # 19200 cache slots


class Buffers:
    """One set of static rows at the largest bucket, plus per-layer weights and caches."""

    def __init__(self, t: int, g: torch.Generator, weights=None, caches=None):
        z = lambda *s: torch.zeros(s, dtype=BF, device=DEV)  # noqa: E731
        self.hidden, self.residual, self.normed, self.attn, self.normed2 = (z(t, H) for _ in range(5))
        self.act = z(t, I)
        self.qkv = [z(t, (HQ + 2 * HK) * D) for _ in range(LAYERS)]
        self.gate_up = [z(t, 2 * I) for _ in range(LAYERS)]
        self.positions = torch.zeros(t, dtype=torch.int64, device=DEV)
        self.slots = torch.zeros(t, dtype=torch.int64, device=DEV)
        if weights is None:
            def w(n):
                return (torch.randn(n, generator=g, device=DEV) * 0.1 + 1).to(BF)
            weights = [dict(w1=w(H), w2=w(H), qw=w(D), kw=w(D)) for _ in range(LAYERS)]
        self.weights = weights
        if caches is None:
            caches = [tuple(torch.randn((BLOCKS, BLOCK, HK, D), generator=g, device=DEV).to(BF) for _ in range(2))
                      for _ in range(LAYERS)]
        self.caches = caches

    def pre(self, i: int, t: int, cos, sin) -> None:
        w = self.weights[i]
        ops.fused_add_rmsnorm_hip(self.hidden[:t], self.residual[:t], w["w1"], 1e-6, out=self.normed[:t],
                                  residual_out=self.residual[:t])
        qkv = self.qkv[i]
        ops.rope_kv_cache_hip(qkv[:t, :HQ * D].view(t, HQ, D), qkv[:t, HQ * D:(HQ + HK) * D].view(t, HK, D),
                              qkv[:t, (HQ + HK) * D:].view(t, HK, D), cos, sin, self.positions[:t], self.slots[:t],
                              self.caches[i][0], self.caches[i][1], w["qw"], w["kw"], 1e-6)

    def attend(self, i: int, n: int) -> None:
        self.attn[:n].copy_(self.qkv[i][:n, :HQ * D])

    def post(self, i: int, t: int) -> None:
        w = self.weights[i]
        ops.fused_add_rmsnorm_hip(self.attn[:t], self.residual[:t], w["w2"], 1e-6, out=self.normed2[:t],
                                  residual_out=self.residual[:t])
        ops.silu_and_mul_hip(self.gate_up[i][:t], out=self.act[:t])
        self.hidden[:t].copy_(self.act[:t, :H])


def _step_inputs(n: int, g: torch.Generator, table: torch.Tensor):
    ids = torch.randint(0, V, (n,), generator=g, device=DEV)
    pos = torch.randint(0, 40960, (n,), generator=g, device=DEV)
    slots = torch.randperm(BLOCKS * BLOCK, generator=g, device=DEV)[:n]
    qkv = [torch.randn((n, (HQ + 2 * HK) * D), generator=g, device=DEV).to(BF) for _ in range(LAYERS)]
    gu = [torch.randn((n, 2 * I), generator=g, device=DEV).to(BF) for _ in range(LAYERS)]
    res = torch.randn((n, H), generator=g, device=DEV).to(BF)
    return ids, pos, slots, qkv, gu, res


def _stage(b: Buffers, n: int, bucket: int, inputs, table, rows: bool = True) -> None:
    ids, pos, slots, qkv, gu, res = inputs
    b.hidden[:n].copy_(ops.embedding_hip(ids, table))  # the embedding runs outside the graphs
    b.residual[:n].copy_(res)
    if rows:
        stage_rows(n, bucket, b.positions, b.slots, pos, slots)
    for i in range(LAYERS):
        b.qkv[i][:n].copy_(qkv[i])
        b.gate_up[i][:n].copy_(gu[i])


def test_piecewise_replay_at_padded_buckets_matches_eager():
    print("piecewise: 2 Qwen3-8B layers, buckets 16/256/8192", flush=True)
    _lib.read_errors(clear=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    table = (torch.randn((V, H), generator=g, device=DEV) * 0.02).to(BF)
    cos, sin = RotaryEmbedding(D, 40960, 1e6).full_tables(DEV)
    top = max(BUCKETS)
    gb = Buffers(top, g)
    # the eager side: its own rows, the same weights, its own copy of the caches
    eb = Buffers(top, g, weights=gb.weights, caches=[tuple(c.clone() for c in kv) for kv in gb.caches])
    runner = SegmentGraphs(LAYERS, BUCKETS, lambda i, t: gb.pre(i, t, cos, sin), gb.post, DEV)
    assert runner.num_segments == LAYERS + 1
    gb.positions, gb.slots = runner.rows.positions, runner.rows.slots  # the runner owns the step rows
    # warm-up and capture run the pieces with every slot PAD_SLOT: the caches must not change
    saved = [tuple(c.clone() for c in kv) for kv in gb.caches]
    runner.capture()
    for (k, v), (k0, v0) in zip(gb.caches, saved):
        assert torch.equal(k, k0) and torch.equal(v, v0), "capture wrote the KV cache"
    del saved
    assert all(torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) for a, b in zip(gb.caches, eb.caches))
    for j, n in enumerate((1, 9, 16, 200, 256, 5000)):
        bucket = runner.bucket(n)
        via_step = j % 2 == 1  # odd steps hand the rows to step(), even ones stage them first
        print(f"piecewise step n={n} bucket={bucket}", flush=True)
        inputs = _step_inputs(n, g, table)
        # stale, different padding rows in the graph side's buffers: they must not matter
        for buf in [gb.hidden, gb.residual, *gb.qkv, *gb.gate_up]:
            buf[n:bucket].normal_(generator=g)
        _stage(gb, n, bucket, inputs, table, rows=not via_step)
        _stage(eb, n, n, inputs, table)
        used = runner.step(n, gb.attend, inputs[1], inputs[2]) if via_step else runner.step(n, gb.attend)
        assert used == bucket
        for i in range(LAYERS):  # the same pieces, launched eagerly at the real row count
            eb.pre(i, n, cos, sin)
            eb.attend(i, n)
            eb.post(i, n)
        torch.cuda.synchronize()
        for name in ("hidden", "residual", "normed", "attn", "normed2", "act"):
            a, b = getattr(gb, name)[:n], getattr(eb, name)[:n]
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"n={n}: {name} rows differ"
        for i in range(LAYERS):
            assert torch.equal(gb.qkv[i][:n].view(torch.int16), eb.qkv[i][:n].view(torch.int16)), f"n={n}: qkv {i}"
            for c in range(2):  # whole caches: real slots written alike, every other slot untouched
                assert torch.equal(gb.caches[i][c].view(torch.int16), eb.caches[i][c].view(torch.int16)), \
                    f"n={n}: layer {i} cache {c} differs"
    assert _lib.read_errors() == 0  # padding slots are skipped without an error
    runner.release()


def test_padding_slot_is_skipped_by_every_cache_write():
    """Slot -1 marks a padding row: the KV write, the fused rope + KV write and the latent
    write store nothing for it and raise no error; other bad slots still set the bit."""
    _lib.read_errors(clear=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(9)
    n = 64
    k = torch.randn((n, HK, D), generator=g, device=DEV).to(BF)
    v = torch.randn((n, HK, D), generator=g, device=DEV).to(BF)
    kc = torch.randn((8, BLOCK, HK, D), generator=g, device=DEV).to(BF)
    vc = torch.randn_like(kc)
    slots = torch.arange(n, device=DEV)
    slots[1::2] = -1
    k0, v0 = kc.clone(), vc.clone()
    ops.kv_cache_write_hip(k, v, slots, kc, vc)
    want_k, want_v = k0.clone(), v0.clone()
    ops.kv_cache_write_torch(k, v, slots, want_k, want_v)  # the eager form skips them too
    assert torch.equal(kc, want_k) and torch.equal(vc, want_v)
    assert torch.equal(kc.view(-1, HK, D)[1::2][:n // 2], k0.view(-1, HK, D)[1::2][:n // 2])
    lat = torch.randn((n, 576), generator=g, device=DEV).to(BF)
    lc = torch.randn((n, 576), generator=g, device=DEV).to(BF)
    l0 = lc.clone()
    ops.latent_cache_write_hip(lat, slots, lc)
    assert torch.equal(lc[0::2], lat[0::2]) and torch.equal(lc[1::2], l0[1::2])
    assert _lib.read_errors() == 0
    slots[3] = 10 ** 6
    ops.kv_cache_write_hip(k, v, slots, kc, vc)
    assert _lib.read_errors() & _lib.ERR_KV_SLOT
