"""Host-side checks that need no GPU: the C-ABI library loads and exports every entry
point include/ember_ops.h declares, argument validation rejects bad calls before any
launch, the Python drop-in keeps the reference's API, and CPU tensors take the eager path
exactly as the reference's dispatch does (emberserve/model/ops.py:43-46, 92-115)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from emberserve_amd import _lib, layers, ops, rope
from oracle import inputs as gen
from oracle import ref_ops as ref
from tests.helpers import assert_bitexact

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ember_ops.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(ember_\w+)\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    names = _declared()
    for n in ["ember_rmsnorm", "ember_fused_add_rmsnorm", "ember_rope", "ember_silu_and_mul",
              "ember_embedding", "ember_qk_norm_rope", "ember_mla_latent_rope", "ember_kv_cache_write",
              "ember_latent_cache_write"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_status_strings():
    lib = _lib.load()
    assert lib.ember_abi_version() == _lib.ABI_VERSION
    assert lib.ember_status_string(0) == b"ok"
    assert b"invalid" in lib.ember_status_string(1)
    assert lib.ember_status_string(99) == b"unknown status"


def test_argument_validation_happens_before_any_launch():
    """Bad shapes and dtypes return EMBER_EINVAL (1) without touching HIP, so these run
    without a GPU; a zero-row call is a successful no-op."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: the calls are rejected first
    assert lib.ember_rmsnorm(p, 64, p, 1, p, 64, -1, 64, 1e-6, 1, None) == 1  # rows < 0
    assert lib.ember_rmsnorm(p, 64, p, 1, p, 64, 4, 0, 1e-6, 1, None) == 1  # cols == 0
    assert lib.ember_rmsnorm(p, 64, p, 2, p, 64, 4, 64, 1e-6, 1, None) == 1  # bf16 weight, fp16 x
    assert lib.ember_rmsnorm(p, 64, p, 7, p, 64, 4, 64, 1e-6, 7, None) == 1  # dtype tag
    assert lib.ember_rmsnorm(p, 64, p, 1, p, 64, 0, 64, 1e-6, 1, None) == 0  # nothing to do
    assert lib.ember_fused_add_rmsnorm(p, 64, None, 64, p, 1, p, 64, p, 64, 4, 64, 1e-6, 1, None) == 1
    assert lib.ember_silu_and_mul(p, 10, p, 5, 4, 8, 1, None) == 1  # row stride < 2*inter
    assert lib.ember_silu_and_mul(p, 16, p, 8, 0, 8, 1, None) == 0
    assert lib.ember_embedding(p, 4, p, 10, 64, 64, p, 64, 3, None) == 1  # elem_bytes 3
    assert lib.ember_embedding(p, 0, p, 10, 64, 64, p, 64, 2, None) == 0
    assert lib.ember_rope(p, 64, 64, 1, p, 64, 64, 1, 63, p, p, 8, 64, p, 4, 2, None) == 1  # odd D
    assert lib.ember_rope(p, 64, 64, 1, p, 64, 64, 1, 64, p, p, 8, 16, p, 4, 2, None) == 1  # table too narrow
    assert lib.ember_rope(p, 64, 64, 1, p, 64, 64, 1, 64, p, p, 8, 64, p, 0, 2, None) == 0
    assert lib.ember_mla_latent_rope(p, 576, 512, p, 576, p, 192, 192, 16, 64, p, 2, 1e-6, p, p, 8, 64,
                                     p, 4, p, 500, 2, None) == 1  # latent row too short
    assert lib.ember_kv_cache_write(p, 1024, 128, p, 1024, 128, 8, 128, p, 4, p, p, 64, 1024, 128, 3,
                                    None) == 1  # elem_bytes 3
    assert lib.ember_kv_cache_write(p, 1024, 128, p, 1024, 128, 8, 128, p, 0, p, p, 64, 1024, 128, 2,
                                    None) == 0  # no tokens
    assert lib.ember_latent_cache_write(p, 576, 0, p, 4, p, 64, 576, 2, None) == 1  # latent_dim 0
    assert lib.ember_latent_cache_write(p, 576, 576, p, 0, p, 64, 576, 2, None) == 0


def test_ops_api_mirrors_the_reference():
    for name in ["fused_enabled", "rmsnorm", "fused_add_rmsnorm", "rope", "silu_and_mul",
                 "rmsnorm_torch", "fused_add_rmsnorm_torch", "rope_torch", "silu_and_mul_torch",
                 "qk_norm_rope", "mla_latent_rope", "embedding"]:
        assert callable(getattr(ops, name)), name
    assert callable(rope.RotaryEmbedding) and callable(rope.rotate_half)


def test_cache_writes_on_cpu_match_the_oracle():
    g = torch.Generator().manual_seed(0)
    k = torch.randn(5, 2, 32, generator=g)
    v = torch.randn(5, 2, 32, generator=g)
    slots = torch.tensor([3, 9, 0, 15, 4])
    a = [torch.zeros(4, 4, 2, 32) for _ in range(2)]
    b = [torch.zeros(4, 4, 2, 32) for _ in range(2)]
    ops.kv_cache_write(k, v, slots, *a)
    ref.kv_cache_write(k, v, slots, *b)
    assert_bitexact(a[0], b[0])
    assert_bitexact(a[1], b[1])
    lat = torch.randn(5, 48, generator=g)
    c1, c2 = torch.zeros(4, 4, 48), torch.zeros(4, 4, 48)
    ops.latent_cache_write(lat, slots, c1)
    ref.latent_cache_write(lat, slots, c2)
    assert_bitexact(c1, c2)


def test_dispatch_uses_torch_off_gpu():
    """ops.py:100-104 of the reference's test: CPU tensors stay on the eager path."""
    x = torch.randn(2, 64)
    w = torch.ones(64)
    assert not ops.fused_enabled(x)
    torch.testing.assert_close(ops.rmsnorm(x, w, 1e-6), ops.rmsnorm_torch(x, w, 1e-6))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_eager_path_equals_the_oracle(dtype):
    """The package's eager forms (CPU tensors) give the oracle's bits."""
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(5, 128, generator=g) * 2).to(dtype)
    r = torch.randn(5, 128, generator=g).to(dtype)
    w = (torch.randn(128, generator=g) * 0.1 + 1).to(dtype)
    assert_bitexact(ops.rmsnorm(x, w, 1e-6), ref.rmsnorm(x, w, 1e-6))
    a, b = ops.fused_add_rmsnorm(x, r, w, 1e-6)
    c, d = ref.fused_add_rmsnorm(x, r, w, 1e-6)
    assert_bitexact(a, c)
    assert_bitexact(b, d)
    assert_bitexact(ops.silu_and_mul(x), ref.silu_and_mul(x))
    cos, sin = ref.rope_tables(64, 32, 1e4)
    q = x.view(5, 2, 64)
    pos = torch.tensor([0, 3, 31, 7, 1])
    for got, want in zip(ops.rope(q, q[:, :1], cos, sin, pos), ref.rope(q, q[:, :1], cos, sin, pos)):
        assert_bitexact(got, want)
    ids = torch.tensor([3, 1, 4])
    assert_bitexact(ops.embedding(ids, x), ref.embedding(ids, x))
    for got, want in zip(ops.qk_norm_rope(q, q[:, :1], w[:64], w[64:], 1e-6, cos, sin, pos),
                         ref.qk_norm_rope(q, q[:, :1], w[:64], w[64:], 1e-6, cos, sin, pos)):
        assert_bitexact(got, want)


def test_rotary_module_tables_match_oracle_and_forward_on_cpu():
    mod = rope.RotaryEmbedding(64, 256, 1e6)
    pos = torch.tensor([0, 5, 255])
    cos, sin = mod.tables(pos)
    rc, rs = ref.rope_tables(64, 256, 1e6)
    assert_bitexact(cos, rc[pos])
    assert_bitexact(sin, rs[pos])
    q = torch.randn(3, 2, 64)
    qo, _ = mod(q, q[:, :1], pos)
    assert_bitexact(qo, ref.rope(q, q[:, :1], rc, rs, pos)[0])


def test_layers_on_cpu():
    norm = layers.RMSNorm(64, 1e-6)
    x = torch.randn(3, 64)
    assert_bitexact(norm(x), ref.rmsnorm(x, norm.weight.detach(), 1e-6))
    emb = layers.Embedding(10, 8)
    ids = torch.tensor([1, 9])
    assert_bitexact(emb(ids).detach(), emb.weight.detach()[ids])
    # Qwen3 pre-attention tail on a fused qkv buffer
    n, hq, hk, d = 4, 4, 2, 64
    qkv = torch.randn(n, (hq + 2 * hk) * d)
    qn, kn = layers.RMSNorm(d, 1e-6), layers.RMSNorm(d, 1e-6)
    rot = rope.RotaryEmbedding(d, 64, 1e6)
    pos = torch.tensor([0, 1, 2, 63])
    q, k, v = layers.qwen3_pre_attention_rope(qkv, hq, hk, d, qn, kn, rot, pos)
    cos, sin = ref.rope_tables(d, 64, 1e6)
    wq, wk = ref.qk_norm_rope(qkv[:, :hq * d].view(n, hq, d), qkv[:, hq * d:(hq + hk) * d].view(n, hk, d),
                              qn.weight.detach(), kn.weight.detach(), 1e-6, cos, sin, pos)
    assert_bitexact(q.detach(), wq)
    assert_bitexact(k.detach(), wk)
    assert_bitexact(v, qkv[:, (hq + hk) * d:].view(n, hk, d))


def test_hip_wrappers_refuse_host_tensors():
    """A host pointer must never reach a kernel: every *_hip wrapper checks devices before
    it loads the library or launches (runs without a GPU)."""
    x = torch.randn(4, 64)
    w = torch.ones(64)
    cos, sin = ref.rope_tables(64, 16, 1e4)
    pos = torch.arange(4)
    q = x.view(4, 1, 64)
    with pytest.raises(ValueError):
        ops.rmsnorm_hip(x, w, 1e-6)
    with pytest.raises(ValueError):
        ops.fused_add_rmsnorm_hip(x, x, w, 1e-6)
    with pytest.raises(ValueError):
        ops.rope_hip(q, q, cos, sin, pos)
    with pytest.raises(ValueError):
        ops.silu_and_mul_hip(x)
    with pytest.raises(ValueError):
        ops.embedding_hip(pos, x)
    with pytest.raises(ValueError):
        ops.qk_norm_rope_hip(q, q, w, w, 1e-6, cos, sin, pos)
    with pytest.raises(ValueError):
        ops.mla_latent_rope_hip(x, x[:, :16], q[..., :16], w, 1e-6, cos, sin, pos)
    with pytest.raises(ValueError):
        ops.kv_cache_write_hip(q, q, pos, torch.zeros(2, 4, 1, 64), torch.zeros(2, 4, 1, 64))
    with pytest.raises(ValueError):
        ops.latent_cache_write_hip(x, pos, torch.zeros(2, 4, 64))


def test_silu_and_mul_rejects_odd_width():
    with pytest.raises(RuntimeError):  # torch eager: the two halves differ in size
        ops.silu_and_mul(torch.randn(2, 7))
    if torch.cuda.is_available():
        with pytest.raises(ValueError):
            ops.silu_and_mul_hip(torch.randn(2, 7, device="cuda"))


# ---- paged decode attention (host side) ----------------------------------------------------
def test_paged_decode_cpu_path_matches_oracle_and_asserts_like_the_reference():
    from emberserve_amd.paged_decode import paged_attention_decode
    q, kc, vc, bt, cl = gen.decode_inputs([5, 19, 40], 4, 2, 64, 16, torch.float32, seed=0)
    got = paged_attention_decode(q, kc, vc, bt, cl, 64 ** -0.5, num_splits=1)
    torch.testing.assert_close(got, ref.paged_decode(q, kc, vc, bt, cl, 64 ** -0.5), rtol=0, atol=1e-6)
    bad = torch.randn(2, 8, 1, 64)  # block_size 8: test_paged_triton.py:272-277
    with pytest.raises(AssertionError, match="block_size"):
        paged_attention_decode(torch.randn(1, 2, 64), bad, bad, torch.zeros(1, 1, dtype=torch.int32),
                               torch.ones(1, dtype=torch.int32), 1.0)
    with pytest.raises(AssertionError, match="head_dim"):
        kc48 = torch.randn(2, 16, 1, 48)
        paged_attention_decode(torch.randn(1, 2, 48), kc48, kc48, torch.zeros(1, 1, dtype=torch.int32),
                               torch.ones(1, dtype=torch.int32), 1.0)


def test_paged_decode_abi_rejects_bad_arguments_before_any_device_call():
    lib = _lib.load()
    assert lib.ember_paged_decode_workspace_bytes(2, 4, 64, 1) == 0
    assert lib.ember_paged_decode_workspace_bytes(2, 4, 64, 3) == 3 * 2 * 4 * 66 * 4 + 32
    assert lib.ember_paged_decode_workspace_bytes(2, 4, 64, 0) == -1
    base = dict(block_size=16, flags=0, heads=4, kv=2, d=64, splits=1)

    def call(block_size, flags, heads, kv, d, splits):
        return lib.ember_paged_decode(None, 0, 0, 1, None, None, 4, block_size, kv, d, 0, 0, 0, 0, 0, 0, 1,
                                      None, 0, 1, None, 1, heads, 1.0, splits, flags, None, 0, None, 0, 0, None)
    for bad in (dict(block_size=8), dict(flags=2), dict(heads=5), dict(d=300), dict(splits=0)):
        assert call(**{**base, **bad}) == 1, bad
    assert call(**base) == 1  # null pointers


def test_paged_decode_default_splits_follow_the_grid_rule(monkeypatch):
    from emberserve_amd import paged_decode as pd
    monkeypatch.delenv("EMBERSERVE_TRITON_SPLITS", raising=False)
    monkeypatch.setattr(pd, "num_sms", lambda device: 256)
    dev = torch.device("cpu")
    assert pd.default_num_splits(128, 8, 2048, dev, 32, 128) == 1      # 1024 programs
    assert pd.default_num_splits(8, 8, 8192, dev, 32, 128) == 4        # 64 programs -> 256
    assert pd.default_num_splits(128, 2, 8192, dev, 14, 64) == 1       # 256 programs
    assert pd.default_num_splits(32, 2, 2048, dev, 14, 64) == 4        # 64 programs -> 256
    assert pd.default_num_splits(1, 8, 8192, dev, 32, 128) == 16       # < 512 keys per split at 32
    assert pd.default_num_splits(1, 8, 16384, dev, 32, 128) == 32      # 512 keys per split at 32
    assert pd.default_num_splits(1, 8, 32768, dev, 32, 128) == 32      # capped at MAX_SPLITS
    assert pd.default_num_splits(1, 2, 8192, dev, 14, 64) == 16
    assert pd.default_num_splits(1, 8, 512, dev, 32, 128) == 2         # >= 256 keys per split
    assert pd.default_num_splits(4, 2, 100000, dev, 40, 64) == 16      # 20 heads/kv: 2 chunks
    monkeypatch.setenv("EMBERSERVE_TRITON_SPLITS", "3")
    assert pd.default_num_splits(128, 8, 2048, dev, 32, 128) == 3


# ---- MLA decode (host side) ----------------------------------------------------------------
def test_mla_decode_cpu_path_matches_oracle_and_asserts_like_the_reference():
    from emberserve_amd.mla_decode import mla_decode
    q, lat, bt, cl = gen.mla_decode_inputs([5, 19, 40], 4, 32, 16, 16, torch.float32, seed=0)
    want = ref.mla_decode(q[..., :32], q[..., 32:], lat, bt, cl, 0.3, 32)
    torch.testing.assert_close(mla_decode(q, lat, bt, cl, 0.3, 32), want, rtol=0, atol=1e-6)
    got = mla_decode((q[..., :32], q[..., 32:]), lat, bt, cl, 0.3, 32)  # the pair form
    torch.testing.assert_close(got, want, rtol=0, atol=1e-6)
    with pytest.raises(AssertionError):  # DR not a power of two >= 16 (mla_triton.py:155)
        mla_decode(torch.randn(1, 4, 40), torch.randn(2, 16, 40), bt[:1], cl[:1], 0.3, 32)
    with pytest.raises(AssertionError, match="block_size"):
        mla_decode(torch.randn(1, 4, 48), torch.randn(2, 8, 48), bt[:1, :1], torch.ones(1, dtype=torch.int32),
                   0.3, 32)


def test_mla_decode_abi_and_split_rule(monkeypatch):
    from emberserve_amd import mla_decode as md
    lib = _lib.load()
    assert lib.ember_mla_decode_workspace_bytes(2, 16, 512, 1) == 0
    assert lib.ember_mla_decode_workspace_bytes(2, 16, 512, 3) == 3 * 2 * 16 * 514 * 4 + 128
    assert lib.ember_mla_decode_workspace_bytes(2, 16, 512, 0) == -1

    def call(block_size=16, dl=512, dr=64, splits=1, heads=16):
        return lib.ember_mla_decode(None, 0, 0, None, 0, 0, 1, None, 4, block_size, dl, dr, 0, 0, 1, None, 0, 1,
                                    None, 1, heads, 1.0, splits, None, 0, None, 0, 0, None)
    for bad in (dict(block_size=8), dict(dl=1024), dict(splits=0), dict(heads=0)):
        assert call(**bad) == 1, bad
    assert call() == 1  # null pointers
    monkeypatch.delenv("EMBERSERVE_TRITON_SPLITS", raising=False)
    monkeypatch.setattr(md, "num_sms", lambda device: 256)
    dev = torch.device("cpu")
    assert md.mla_num_splits(128, dev) == 2                          # 128 workgroups -> 256
    assert md.mla_num_splits(1, dev) == md.MAX_SPLITS
    assert md.mla_num_splits(1, dev, max_context=320) == 8           # ~sqrt(context / 4)
    assert md.mla_num_splits(1, dev, max_context=4096) == 32
    assert md.mla_num_splits(1, dev, max_context=32768) == 90
    assert md.mla_num_splits(1, dev, max_context=48) == 3            # at least 16 keys a split
    assert md.mla_num_splits(1, dev, max_context=16) == 1
    assert md.mla_num_splits(8, dev, num_heads=128, max_context=4096) == 4   # 64 workgroups -> 256
    assert md.mla_num_splits(128, dev, max_context=320) == 2
    assert md.mla_num_splits(512, dev) == 1
    monkeypatch.setenv("EMBERSERVE_TRITON_SPLITS", "5")
    assert md.mla_num_splits(128, dev) == 5


def test_mixed_rows_plan_and_layout_checks():
    """MixedRows on the host: slot order (decode rows first, then each prefill row
    left-padded to max_q), the reference plan's dec_tokens, and refusals before launch."""
    from emberserve_amd.mixed import MixedRows, pack_queries
    plan = MixedRows([1, 3, 1, 2], "cpu")
    assert plan.num_tokens == 7 and plan.num_dec == 2 and plan.num_pre == 2 and plan.max_q == 3
    assert plan.rows.tolist() == [0, 4, 1, 2, 3, -1, 5, 6]
    assert plan.dec_tokens.tolist() == [0, 4]
    assert MixedRows([1, 1], "cpu").rows.tolist() == [0, 1]
    assert MixedRows([4], "cpu").rows.tolist() == [0, 1, 2, 3]
    with pytest.raises(ValueError):
        MixedRows([1, 0], "cpu")
    with pytest.raises(ValueError):  # host tensors never reach a kernel
        pack_queries(torch.zeros(7, 2, 4), plan)


# ---- gate_up + silu_and_mul (host side) ------------------------------------------------------
def test_gate_up_silu_cpu_path_is_the_unfused_pair():
    from emberserve_amd.gate_up_silu import gate_up_silu
    x, w = gen.gate_up_inputs(6, 128, 96, torch.bfloat16, seed=4)
    got = gate_up_silu(x, w)
    assert torch.equal(got, ref.silu_and_mul(torch.nn.functional.linear(x, w)))
    assert gate_up_silu(x.view(2, 3, 128), w).shape == (2, 3, 96)
    with pytest.raises(ValueError):
        gate_up_silu(x, w[:, :64])
    with pytest.raises(ValueError):
        gate_up_silu(x, w[:95])


def test_gate_up_silu_workspace_plan():
    """Units are (64-column slab, 64-k step) pairs in slab-major order; workgroup b runs
    units [floor(b total / G), floor((b + 1) total / G)). The workspace holds, per slab, one
    partial slot per workgroup whose run meets it (counted here by brute force over the
    units), plus a counter per slab."""
    lib = _lib.load()

    def expected(tokens, hidden, inter, programs):
        nk, slabs = hidden // 64, inter // 64
        total = nk * slabs
        G = min(programs, total)
        owner = []
        for b in range(G):
            owner += [b] * ((b + 1) * total // G - b * total // G)
        parts = max(len(set(owner[s * nk:(s + 1) * nk])) for s in range(slabs))
        tiles = 1
        while tiles < -(-tokens // 16):  # token tiles rounded up to a power of two
            tiles *= 2
        floats = 4 * tiles * 2 * 64 * 4
        return slabs * parts * floats * 4 + (slabs * 4 + 255) // 256 * 256
    for args in [(16, 4096, 12288, 256), (64, 3584, 18944, 256), (1, 896, 4864, 256), (5, 128, 64, 256),
                 (33, 4096, 12288, 512), (16, 1024, 1024, 7), (40, 4096, 12288, 256)]:
        assert lib.ember_gate_up_silu_workspace_bytes(*args) == expected(*args), args
    assert lib.ember_gate_up_silu_workspace_bytes(65, 4096, 12288, 256) == -1
    assert lib.ember_gate_up_silu_workspace_bytes(16, 4096, 100, 256) == -1
    assert lib.ember_gate_up_silu_workspace_bytes(16, 100, 128, 256) == -1
    assert lib.ember_gate_up_silu_workspace_bytes(16, 4096, 128, 0) == -1


def test_moe_align_workspace_and_abi_validation():
    """The grid form's count table: [segments][E] int32 over ceil(num_valid / 2048) segments,
    at most 64, used past 3072 assignments (0 bytes below); argument checks before any launch."""
    lib = _lib.load()
    assert lib.ember_moe_align_workspace_bytes(3072, 64) == 0
    assert lib.ember_moe_align_workspace_bytes(3073, 64) == 2 * 64 * 4
    assert lib.ember_moe_align_workspace_bytes(8193, 64) == 5 * 64 * 4
    assert lib.ember_moe_align_workspace_bytes(49152, 64) == 24 * 64 * 4
    assert lib.ember_moe_align_workspace_bytes(10 ** 7, 256) == 64 * 256 * 4
    assert lib.ember_moe_align_workspace_bytes(-1, 64) == -1
    assert lib.ember_moe_align_workspace_bytes(100, 1025) == -1
    mp = lib.ember_moe_align_padded_size(100, 8, 16)

    def call(nv=100, e=8, bm=16, padded=mp, blocks=mp // 16, ws=None, ws_bytes=0, id_bytes=8):
        return lib.ember_moe_align(None, id_bytes, nv, e, bm, None, padded, None, blocks, ws, ws_bytes, None)
    for bad in (dict(id_bytes=2), dict(e=0), dict(e=1025), dict(bm=0), dict(padded=mp + 16), dict(blocks=1),
                dict(ws_bytes=-1), dict(ws_bytes=64)):
        assert call(**bad) == 1, bad
    assert call() == 1  # null pointers


def test_moe_direct_half_slab_rule(monkeypatch):
    """Two-wave half-slab workgroups while min(assignments, experts) x slabs is 1-5x the CUs."""
    import emberserve_amd.moe as moe
    monkeypatch.setattr(moe, "num_sms", lambda device: 256)
    dev = torch.device("cpu")
    assert not moe.moe_direct_half_slabs(6, 64, 1408, dev)      # 132 workgroups
    assert moe.moe_direct_half_slabs(12, 64, 1408, dev)         # 264
    assert moe.moe_direct_half_slabs(48, 64, 1408, dev)         # 1056
    assert not moe.moe_direct_half_slabs(72, 64, 1408, dev)     # 64 experts: 1408


def test_gemm_column_tile_rule(monkeypatch):
    """The tile with the fewest rows streamed per CU: ceil(tiles / CUs) x (256 + 2 x cols)."""
    import emberserve_amd.gate_up_silu as gu
    monkeypatch.setattr(gu, "num_sms", lambda device: 256)
    dev = torch.device("cpu")
    assert gu.gemm_column_tile(256, 12288, dev) == 64      # Qwen3-8B: 1 round of 192 tiles
    assert gu.gemm_column_tile(512, 12288, dev) == 96      # 2 x 384 | 1 x 416 | 1 x 512
    assert gu.gemm_column_tile(8192, 12288, dev) == 128    # 24 x 384 | 16 x 448 | 12 x 512
    assert gu.gemm_column_tile(256, 18944, dev) == 96      # Qwen2.5-7B: 2 x 384 | 1 x 448
    assert gu.gemm_column_tile(512, 18944, dev) == 96      # 3 x 384 | 2 x 448 | 2 x 512
    assert gu.gemm_column_tile(8192, 18944, dev) == 128    # 37 x 384 | 25 x 448 | 19 x 512
    assert gu.gemm_column_tile(8192, 4864 + 64, dev) == 96  # 128 does not divide inter
    assert gu.gemm_column_tile(8192, 192, dev) == 64       # 96 tiles of 64 fit one round
    with pytest.raises(ValueError):
        gu.gemm_column_tile(256, 40, dev)


def test_moe_gate_up_silu_gemm_abi_validation():
    lib = _lib.load()

    def call(blocks=4, rows=256, valid=10, tokens=5, top_k=2, experts=8, hidden=2048, inter=1408, tile=64, dtype=2):
        return lib.ember_moe_gate_up_silu_gemm(None, hidden, tokens, None, 2 * inter * hidden, hidden, dtype, experts,
                                               hidden, inter, None, None, blocks, rows, valid, top_k, tile, None,
                                               inter, None)
    assert call(blocks=0) == 0 and call(valid=0) == 0  # nothing to do
    for bad in (dict(tokens=0), dict(top_k=0), dict(experts=0), dict(hidden=100), dict(tile=32),
                dict(tile=128, inter=1344), dict(rows=128), dict(rows=64, tile=128), dict(dtype=0)):
        assert call(**bad) == 1, bad
    assert call() == 1  # null pointers


def test_gate_up_silu_abi_validation():
    lib = _lib.load()

    def call(tokens=16, hidden=4096, inter=12288, programs=256, dtype=2):
        return lib.ember_gate_up_silu(None, hidden, None, hidden, dtype, tokens, hidden, inter, programs, None, 0,
                                      None, inter, None)
    assert call(tokens=0) == 0
    for bad in (dict(tokens=65), dict(hidden=100), dict(inter=100), dict(programs=0), dict(dtype=0)):
        assert call(**bad) == 1, bad
    assert call() == 1  # null pointers


def test_packed_gemm_abi_validation():
    """The packed prefill GEMMs reject bad shapes and tiles (no 96-column tile: slabs are
    64 rows) before any device call."""
    lib = _lib.load()

    def dense(tokens=300, hidden=4096, inter=12288, programs=256, rows=256, tile=128, dtype=2):
        return lib.ember_gate_up_silu_gemm_packed(None, hidden, None, dtype, tokens, hidden, inter, programs, rows, tile,
                                                  None, inter, None)
    assert dense(tokens=0) == 0
    for bad in (dict(tile=96), dict(rows=128, tile=64), dict(inter=4864 + 64), dict(hidden=100), dict(programs=0),
                dict(dtype=0), dict(tokens=-1)):
        assert dense(**bad) == 1, bad
    assert dense() == 1  # null pointers

    def moe(blocks=4, rows=256, valid=10, tokens=5, top_k=2, experts=8, hidden=2048, inter=1408, tile=64, dtype=2):
        return lib.ember_moe_gate_up_silu_gemm_packed(None, hidden, tokens, None, dtype, experts, hidden, inter, None,
                                                      None, blocks, rows, valid, top_k, tile, None, inter, None)
    assert moe(blocks=0) == 0 and moe(valid=0) == 0
    for bad in (dict(tile=96), dict(rows=128, tile=64), dict(tile=128, inter=1344), dict(top_k=0), dict(dtype=0)):
        assert moe(**bad) == 1, bad
    assert moe() == 1


def test_gate_up_silu_without_the_unpacked_weight():
    """weight None needs the packed copy, and cannot take the unfused pair."""
    from emberserve_amd.gate_up_silu import gate_up_silu
    x = torch.zeros(4, 64)
    with pytest.raises(ValueError):
        gate_up_silu(x, None)
    with pytest.raises(ValueError):
        gate_up_silu(x, None, packed=object(), fused=False)


# ---- MoE gate_up + silu_and_mul (host side) -------------------------------------------------
@pytest.mark.parametrize("n,e,k", [(1, 64, 6), (7, 8, 2), (50, 16, 4), (3, 4, 4)])
def test_moe_align_layout(n, e, k):
    """moe_triton.py:215-254's layout: every assignment exactly once, each expert's run in
    ascending id order starting on a block boundary, padding = num_valid, block_expert the
    expert of each block (num_experts past the used blocks), sizes as the reference's."""
    from emberserve_amd.moe import BLOCK_M, moe_align
    ids = torch.randint(0, e, (n, k), generator=torch.Generator().manual_seed(n * e))
    sorted_ids, block_expert, nv = moe_align(ids, e)
    assert nv == n * k
    want_s, want_b, _ = ref.moe_align(ids, e, BLOCK_M)
    assert sorted_ids.tolist() == want_s and block_expert.tolist() == want_b
    max_padded = -(-(nv + e * (BLOCK_M - 1)) // BLOCK_M) * BLOCK_M
    assert sorted_ids.shape == (max_padded,) and block_expert.shape == (max_padded // BLOCK_M,)
    s = sorted_ids.tolist()
    assert sorted(v for v in s if v < nv) == list(range(nv))
    assert all(v == nv for v in s if v >= nv)
    flat = ids.reshape(-1).tolist()
    used_blocks = 0
    for b, be in enumerate(block_expert.tolist()):
        blk = [v for v in s[b * BLOCK_M:(b + 1) * BLOCK_M] if v < nv]
        if be >= e:
            assert not blk
            continue
        used_blocks = b + 1
        assert all(flat[v] == be for v in blk) and blk == sorted(blk)
    assert all(be >= e for be in block_expert.tolist()[used_blocks:])
    assert used_blocks == sum(-(-flat.count(x) // BLOCK_M) for x in range(e))


def test_moe_gate_up_cpu_path_follows_the_assignments():
    """The eager form computes silu_and_mul(F.linear(x[t], w[e])) for row t * k + c with
    e = topk_ids[t, c], bit for bit against the same ops row by row."""
    from emberserve_amd.moe import fused_moe_gate_up
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 64, generator=g).to(torch.bfloat16)
    w = (torch.randn(6, 2 * 32, 64, generator=g) * 0.2).to(torch.bfloat16)
    ids = torch.randint(0, 6, (5, 3), generator=g)
    got = fused_moe_gate_up(x, ids, w)
    for t in range(5):
        for c in range(3):
            want = ref.silu_and_mul(torch.nn.functional.linear(x[t:t + 1], w[int(ids[t, c])]))
            assert torch.equal(got[t * 3 + c:t * 3 + c + 1], want), (t, c)


def test_moe_split_rule_and_workspace(monkeypatch):
    from emberserve_amd import moe
    monkeypatch.setattr(moe, "num_sms", lambda device: 256)
    dev = torch.device("cpu")
    # row kernel: one split under the CUs, else two
    assert moe.moe_num_splits(6, 64, 2048, 1408, dev) == 1     # one token: 6 x 22 slabs = 132
    assert moe.moe_num_splits(12, 64, 2048, 1408, dev) == 2    # two tokens: 264
    assert moe.moe_num_splits(384, 64, 2048, 1408, dev) == 2   # 64 tokens: 1408
    # packed kernel: one split
    assert moe.moe_num_splits(6, 64, 2048, 1408, dev, packed=True) == 1
    assert moe.moe_num_splits(12, 64, 2048, 1408, dev, packed=True) == 1
    # packed, half-slab workgroups: from one to 1.5 times the CUs of four-wave ones
    assert not moe.moe_half_slabs(6, 64, 1408, dev)    # 132
    assert moe.moe_half_slabs(12, 64, 1408, dev)       # 264
    assert moe.moe_half_slabs(17, 64, 1408, dev)       # 374 < 384
    assert not moe.moe_half_slabs(18, 64, 1408, dev)   # 396
    assert not moe.moe_half_slabs(24, 64, 1408, dev)   # 528
    assert moe.moe_num_splits(12, 64, 64 * 3, 1408, dev) == 1  # three k steps: no even split
    lib = _lib.load()
    assert lib.ember_moe_gate_up_silu_workspace_bytes(6, 1408, 61, 1) == 0
    assert lib.ember_moe_gate_up_silu_workspace_bytes(6, 1408, 61, 4) == (4 * 6 * 2816 * 4 + 255) // 256 * 256 + (61 * 22 * 4 + 255) // 256 * 256
    assert lib.ember_moe_gate_up_silu_workspace_bytes(6, 1408, 61, 5) == -1
    assert lib.ember_moe_gate_up_silu_workspace_bytes(6, 100, 61, 2) == -1


def test_swiglu_mlp_module_matches_the_reference_composition():
    """layers.SwiGLUMLP has Qwen2MLP's parameters and computes down(silu_and_mul(gate_up(x)))."""
    mlp = layers.SwiGLUMLP(64, 96).to(torch.bfloat16)
    assert mlp.gate_up_proj.weight.shape == (192, 64) and mlp.down_proj.weight.shape == (64, 96)
    x = torch.randn(5, 64, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    with torch.no_grad():
        want = mlp.down_proj(ref.silu_and_mul(mlp.gate_up_proj(x)))
        assert torch.equal(mlp(x), want)


def test_noalloc_decode_rejects_oversize_calls_before_any_launch():
    """ember_paged_decode_noalloc refuses, with EMBER_ETOOBIG and no HIP call, a call whose
    split-K workspace would not fit beside its counters in the library's scratch array."""
    lib = _lib.load()
    cap = lib.ember_paged_decode_noalloc_max_bytes()
    assert cap == 15 * 2 ** 20
    assert lib.ember_paged_decode_workspace_bytes(1024, 32, 128, 4) > cap
    p = ctypes.c_void_p(16)  # never dereferenced
    st = lib.ember_paged_decode_noalloc(p, 4096, 128, 2, p, p, 4, 16, 8, 128, 16384, 1024, 128, 16384, 1024, 128,
                                        2, p, 4, 4, p, 1024, 32, 0.088, 4, 0, p, 4096, 128, None)
    assert st == 5 and b"no-allocation" in lib.ember_status_string(5)
