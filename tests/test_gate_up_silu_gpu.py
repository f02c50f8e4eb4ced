"""GPU parity of the fused gate_up projection + silu_and_mul (ember_gate_up_silu) against
the oracle `gate_up_silu` (float64 dot products rounded to the dtype, then silu_and_mul).

The tolerance is tests.helpers.check_gate_up's: the first-order bound on the fp32
accumulation error (n 2^-24 sum|x w|) carried through the activation, and at least 98% of
the elements bit-identical to the oracle."""

from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

from emberserve_amd import _lib  # noqa: E402
from emberserve_amd.gate_up_silu import gate_up_silu, gate_up_silu_torch  # noqa: E402
from oracle import inputs as gen  # noqa: E402
from oracle import ref_ops as ref  # noqa: E402
from tests.helpers import check_gate_up  # noqa: E402

DEV = "cuda"


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _check(got: torch.Tensor, x: torch.Tensor, w: torch.Tensor, what: str, min_exact: float = 0.98) -> None:
    gu = (x.double() @ w.double().T).to(x.dtype)
    absdot = x.double().abs() @ w.double().abs().T
    check_gate_up(got, ref.gate_up_silu(x, w), gu, absdot, x.shape[1], what, min_exact)


@pytest.fixture(autouse=True)
def _clear_errors():
    _lib.read_errors(clear=True)
    yield
    assert _lib.read_errors() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [1, 5, 16, 17, 33, 64])
def test_gate_up_silu_small_model(dtype, tokens):
    """Qwen2.5-0.5B MLP (H 896, I 4864): every token-tile count; one workgroup per CU (runs
    of about 4 units, so most slabs merge partials), 7 workgroups (runs of many whole slabs
    and a shared one), and one workgroup (everything written directly)."""
    x, w = gen.gate_up_inputs(tokens, 896, 4864, dtype, seed=tokens)
    dx, dw = x.to(DEV), w.to(DEV)
    for programs in (None, 7, 1):
        _say(f"gate_up_silu 0.5B T={tokens} {dtype} workgroups={programs}")
        _check(gate_up_silu(dx, dw, num_workgroups=programs, fused=True), x, w, f"T={tokens} workgroups={programs}")


@pytest.mark.parametrize("tokens", [1, 32, 64])
def test_gate_up_silu_qwen3_8b(tokens):
    """Qwen3-8B MLP (H 4096, I 12288), bf16: one and two workgroups per CU."""
    x, w = gen.gate_up_inputs(tokens, 4096, 12288, torch.bfloat16, seed=100 + tokens)
    dx, dw = x.to(DEV), w.to(DEV)
    for programs in (None, 512):
        _say(f"gate_up_silu Qwen3-8B T={tokens} workgroups={programs}")
        _check(gate_up_silu(dx, dw, num_workgroups=programs, fused=True), x, w, f"T={tokens} workgroups={programs}")


def test_gate_up_silu_qwen25_7b_strided_rows():
    """Qwen2.5-7B MLP (H 3584, I 18944), x a row-strided view (rows of a wider buffer)."""
    xb, w = gen.gate_up_inputs(9, 3584 + 64, 18944, torch.bfloat16, seed=7)
    w = w[:, :3584].contiguous()
    x = xb[:, :3584]
    dx = xb.to(DEV)[:, :3584]
    assert dx.stride(0) == 3584 + 64
    _say("gate_up_silu Qwen2.5-7B strided x")
    _check(gate_up_silu(dx, w.to(DEV), fused=True), x, w, "strided x")


def test_gate_up_silu_partition_invariance_and_determinism():
    """Any workgroup count (runs shorter than, equal to and longer than a slab's 16 k
    steps, and more workgroups than units) gives results within the tolerance; repeated
    calls are identical."""
    x, w = gen.gate_up_inputs(20, 1024, 1024, torch.bfloat16, seed=3)
    dx, dw = x.to(DEV), w.to(DEV)
    for programs in (1, 3, 16, 100, 256, 300):
        outs = [gate_up_silu(dx, dw, num_workgroups=programs, fused=True) for _ in range(3)]
        assert all(torch.equal(o, outs[0]) for o in outs), f"workgroups={programs} not deterministic"
        _check(outs[0], x, w, f"workgroups={programs}")


def test_gate_up_silu_unfused_fallbacks():
    """Shapes the kernel does not take run the unfused pair (torch linear + silu_and_mul):
    more than 64 tokens, a hidden size that is not a multiple of 64, fp32; and by default
    more than FUSED_TOKENS tokens."""
    for tokens, hidden, inter, dtype in [(65, 256, 128, torch.bfloat16), (4, 200, 128, torch.bfloat16),
                                         (4, 256, 100, torch.float16), (4, 256, 128, torch.float32),
                                         (17, 256, 128, torch.bfloat16)]:
        x, w = gen.gate_up_inputs(tokens, hidden, inter, dtype, seed=tokens + hidden)
        got = gate_up_silu(x.to(DEV), w.to(DEV), fused=None if tokens == 17 else True)
        torch.testing.assert_close(got.cpu(), gate_up_silu_torch(x.to(DEV), w.to(DEV)).cpu(), rtol=0, atol=0)


def test_gate_up_silu_bad_workgroups_raise():
    x, w = gen.gate_up_inputs(4, 512, 128, torch.bfloat16, seed=1)
    with pytest.raises(ValueError):
        gate_up_silu(x.to(DEV), w.to(DEV), num_workgroups=0)


def test_gate_up_silu_default_dispatch_runs_the_kernel():
    """Up to FUSED_TOKENS tokens the default path is the kernel: with the unfused pair
    replaced by a raising stand-in it still returns the right result."""
    from emberserve_amd import gate_up_silu as gus
    x, w = gen.gate_up_inputs(16, 1024, 512, torch.bfloat16, seed=9)
    saved = gus.gate_up_silu_torch

    def boom(*a, **kw):
        raise AssertionError("unfused pair ran")
    gus.gate_up_silu_torch = boom
    try:
        got = gus.gate_up_silu(x.to(DEV), w.to(DEV))
    finally:
        gus.gate_up_silu_torch = saved
    _check(got, x, w, "default dispatch")


def test_gate_up_silu_graph_replay():
    """A captured call replays to the eager result, with other work between replays (the
    split counters must be back at zero after every call)."""
    x, w = gen.gate_up_inputs(12, 2048, 2048, torch.bfloat16, seed=5)
    dx, dw = x.to(DEV), w.to(DEV)
    programs = 37  # runs of 27-28 units, shorter than a slab's 32 k steps: slabs merge partials
    want = gate_up_silu(dx, dw, num_workgroups=programs, fused=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        gate_up_silu(dx, dw, num_workgroups=programs, fused=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = gate_up_silu(dx, dw, num_workgroups=programs, fused=True)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
        assert torch.equal(gate_up_silu(dx, dw, num_workgroups=programs, fused=True), want)


def test_swiglu_mlp_module_on_the_gpu():
    """layers.SwiGLUMLP on a decode batch runs the fused kernel: its output equals
    down_proj of gate_up_silu's result."""
    from emberserve_amd import layers
    torch.manual_seed(0)
    mlp = layers.SwiGLUMLP(1024, 512).to(DEV, torch.bfloat16)
    x = torch.randn(8, 1024, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        got = mlp(x)
        want = mlp.down_proj(gate_up_silu(x, mlp.gate_up_proj.weight))
    assert torch.equal(got, want)


# ---- the packed weight layout (ember_gate_up_silu_pack_weight / ember_gate_up_silu_packed) ----
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("programs", [1, 7, 256, 5000])
def test_pack_weight_matches_the_oracle_permutation(dtype, programs):
    """H 192, I 320: 15 units, so 7 workgroups give runs of 2 and 3 units and 256 or 5000
    clamp to 15."""
    from emberserve_amd.gate_up_silu import pack_gate_up_weight
    g = torch.Generator().manual_seed(11)
    w = torch.randn(2 * 320, 192, generator=g).to(dtype)
    packed = pack_gate_up_weight(w.to(DEV), programs)
    assert torch.equal(packed.packed.cpu().view(torch.int16), ref.pack_gate_up_weight(w, programs).view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [1, 7, 16, 17, 33, 40, 64])
@pytest.mark.parametrize("programs", [7, 19, 76, 256, 300])
def test_packed_kernel_equals_the_row_kernel(dtype, tokens, programs):
    """Same products in the same order: bit-identical to ember_gate_up_silu (Qwen2.5-0.5B
    MLP, H 896, I 4864: 76 slabs), including runs that split slabs and merge partials, and
    whole-slab runs (19 and 76 workgroups), where up to 16 tokens keep x resident in LDS."""
    from emberserve_amd.gate_up_silu import pack_gate_up_weight
    _say(f"packed gate_up {dtype} T={tokens} G={programs}")
    g = torch.Generator().manual_seed(tokens)
    x = (torch.randn(tokens, 896, generator=g) * 0.5).to(dtype).to(DEV)
    w = (torch.randn(2 * 4864, 896, generator=g) / 896 ** 0.5).to(dtype).to(DEV)
    packed = pack_gate_up_weight(w, programs)
    a = gate_up_silu(x, w, num_workgroups=programs, fused=True)
    b = gate_up_silu(x, w, fused=True, packed=packed)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("tokens", [1, 16])
def test_packed_kernel_qwen3_8b_against_oracle(tokens):
    """Qwen3-8B MLP (H 4096, I 12288) bf16 on sampled output columns against the oracle."""
    from emberserve_amd.gate_up_silu import pack_gate_up_weight
    _say(f"packed gate_up qwen3-8b T={tokens}")
    g = torch.Generator().manual_seed(40 + tokens)
    x = (torch.randn(tokens, 4096, generator=g) * 0.5).to(torch.bfloat16)
    w = (torch.randn(2 * 12288, 4096, generator=g) / 64).to(torch.bfloat16)
    wd = w.to(DEV)
    got = gate_up_silu(x.to(DEV), wd, fused=True, packed=pack_gate_up_weight(wd)).cpu()
    cols = torch.randperm(12288, generator=g)[:512]
    ws = torch.cat([w[cols], w[12288 + cols]])
    _check(got[:, cols], x, ws, "packed qwen3-8b")


def test_packed_weight_rejects_another_grid():
    from emberserve_amd.gate_up_silu import pack_gate_up_weight
    w = torch.randn(2 * 128, 64, device=DEV).to(torch.bfloat16)
    x = torch.randn(1, 64, device=DEV).to(torch.bfloat16)
    packed = pack_gate_up_weight(w, 3)
    with pytest.raises(ValueError, match="packed for 3"):
        gate_up_silu(x, w, num_workgroups=4, fused=True, packed=packed)


def test_swiglu_mlp_packed_weights():
    """SwiGLUMLP.pack_weights: the packed path gives the unpacked module's output bit for bit,
    and an in-place change of the weight drops the stale copy."""
    from emberserve_amd import layers
    torch.manual_seed(1)
    mlp = layers.SwiGLUMLP(1024, 512).to(DEV, torch.bfloat16)
    x = torch.randn(4, 1024, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        want = mlp(x)
        mlp.pack_weights()
        assert mlp._packed is not None
        assert torch.equal(mlp(x), want)
        mlp.gate_up_proj.weight.mul_(2)
        changed = mlp(x)
        assert mlp._packed is None
        assert torch.equal(changed, mlp.down_proj(gate_up_silu(x, mlp.gate_up_proj.weight)))


# ---- prefill sizes: the MFMA GEMM with the activation as its epilogue ----
@pytest.mark.parametrize("token_tile,tile", [(256, 64), (256, 96), (256, 128), (128, 128)])
@pytest.mark.parametrize("tokens", [1, 16, 64, 300])
def test_gemm_equals_the_packed_kernel(token_tile, tile, tokens):
    """Every accumulator runs over k in order in one chain, as the packed kernel's over
    whole-slab runs (76 workgroups for Qwen2.5-0.5B's 76 slabs): bit-identical per token,
    in 64-token chunks past 64 (token tiles padded, a partial last tile)."""
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm, pack_gate_up_weight
    _say(f"gemm gate_up tile={token_tile}x{tile} T={tokens}")
    g = torch.Generator().manual_seed(900 + tokens)
    x = (torch.randn(tokens, 896, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    w = (torch.randn(2 * 4864, 896, generator=g) / 896 ** 0.5).to(torch.bfloat16).to(DEV)
    got = gate_up_silu_gemm(x, w, column_tile=tile, token_tile=token_tile)
    packed = pack_gate_up_weight(w, 76)
    for t0 in range(0, tokens, 64):
        want = gate_up_silu(x[t0:t0 + 64], w, fused=True, packed=packed)
        assert torch.equal(got[t0:t0 + 64].view(torch.int16), want.view(torch.int16)), t0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [256, 777])
def test_gemm_against_oracle(dtype, tokens):
    """Qwen3-8B MLP shape (H 4096, I 12288) on sampled columns against the oracle."""
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm
    _say(f"gemm gate_up oracle {dtype} T={tokens}")
    g = torch.Generator().manual_seed(950 + tokens)
    x = (torch.randn(tokens, 4096, generator=g) * 0.5).to(dtype)
    w = (torch.randn(2 * 12288, 4096, generator=g) / 64).to(dtype)
    got = gate_up_silu_gemm(x.to(DEV), w.to(DEV), column_tile=128).cpu()
    cols = torch.randperm(12288, generator=g)[:128]
    rows = torch.randperm(tokens, generator=g)[:64]
    _check(got[rows][:, cols], x[rows], torch.cat([w[cols], w[12288 + cols]]), f"gemm T={tokens}")


@pytest.mark.parametrize("inter", [112, 176, 4880])
@pytest.mark.parametrize("tokens", [7, 300])
def test_gemm_ragged_96_column_tile(inter, tokens):
    """The 96-column tile needs I only a multiple of 16 (and >= 96): its last tile is ragged
    (I = 112 is one whole tile and 16 columns, 176 one and 80, 4880 fifty and 80).
    Every column against the oracle, and the default dispatch picks a tile that fits."""
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm, gemm_column_tile
    _say(f"gemm gate_up ragged 96 I={inter} T={tokens}")
    g = torch.Generator().manual_seed(960 + inter + tokens)
    x = (torch.randn(tokens, 512, generator=g) * 0.5).to(torch.bfloat16)
    w = (torch.randn(2 * inter, 512, generator=g) / 512 ** 0.5).to(torch.bfloat16)
    got = gate_up_silu_gemm(x.to(DEV), w.to(DEV), column_tile=96).cpu()
    _check(got, x, w, f"gemm 96 I={inter} T={tokens}")
    if inter % 64 != 0:
        assert gemm_column_tile(tokens, inter, torch.device(DEV)) == 96
        fused = gate_up_silu(x.to(DEV), w.to(DEV), fused=True).cpu()
        if tokens > 64:
            assert torch.equal(fused, got)


@pytest.mark.parametrize("token_tile,tile", [(256, 64), (256, 128), (128, 128)])
@pytest.mark.parametrize("programs", [76, 256, 1000])
def test_gemm_packed_equals_the_gemm(token_tile, tile, programs):
    """The prefill GEMM over the packed weight (packed for 76, 256 or 1000 decode workgroups:
    runs that split slabs at different k, and more workgroups than units) gives the unpacked
    GEMM's bits at every token (300 tokens: a partial token tile)."""
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm, gate_up_silu_gemm_packed, pack_gate_up_weight
    _say(f"gemm packed tile={token_tile}x{tile} programs={programs}")
    g = torch.Generator().manual_seed(1100 + programs + tile)
    x = (torch.randn(300, 1024, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    w = (torch.randn(2 * 1280, 1024, generator=g) / 32).to(torch.bfloat16).to(DEV)
    packed = pack_gate_up_weight(w, programs)
    got = gate_up_silu_gemm_packed(x, packed, column_tile=tile, token_tile=token_tile)
    want = gate_up_silu_gemm(x, w, column_tile=tile, token_tile=token_tile)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_packed_qwen3_8b_against_oracle(dtype):
    """Qwen3-8B's MLP (H 4096, I 12288) at 777 tokens over a weight packed for the default
    grid: equal to the unpacked GEMM, and sampled rows and columns against the oracle."""
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm, gate_up_silu_gemm_packed, pack_gate_up_weight
    _say(f"gemm packed qwen3-8b {dtype}")
    g = torch.Generator().manual_seed(1200)
    x = (torch.randn(777, 4096, generator=g) * 0.5).to(dtype)
    w = (torch.randn(2 * 12288, 4096, generator=g) / 64).to(dtype)
    dx, dw = x.to(DEV), w.to(DEV)
    got = gate_up_silu_gemm_packed(dx, pack_gate_up_weight(dw))
    assert torch.equal(got.view(torch.int16), gate_up_silu_gemm(dx, dw, column_tile=128).view(torch.int16))
    got = got.cpu()
    cols = torch.randperm(12288, generator=g)[:128]
    rows = torch.randperm(777, generator=g)[:64]
    _check(got[rows][:, cols], x[rows], torch.cat([w[cols], w[12288 + cols]]), "packed gemm")


def test_swiglu_mlp_keeps_one_weight_copy():
    """pack_weights(keep_weight=False): the module holds only the packed copy and gives the
    unpacked module's output bit for bit at decode sizes (the packed decode kernel) and at
    prefill sizes (the packed GEMM against the unpacked GEMM)."""
    from emberserve_amd import layers
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm
    torch.manual_seed(2)
    mlp = layers.SwiGLUMLP(1024, 1280).to(DEV, torch.bfloat16)
    w = mlp.gate_up_proj.weight.detach().clone()
    xs = [torch.randn(t, 1024, device=DEV, dtype=torch.bfloat16) for t in (1, 16, 64, 65, 600)]
    with torch.no_grad():
        mlp.pack_weights()
        packed = mlp._packed
        want = {x.shape[0]: mlp.down_proj(gate_up_silu(x, w, fused=True, packed=packed) if x.shape[0] <= 64
                                          else gate_up_silu_gemm(x, w, column_tile=64)) for x in xs}
        mlp.pack_weights(keep_weight=False)
        assert mlp.gate_up_proj.weight.numel() == 0 and mlp._packed is not None
        for x in xs:
            assert torch.equal(mlp(x), want[x.shape[0]]), x.shape[0]
        with pytest.raises(RuntimeError):
            mlp.pack_weights()


def test_gemm_rejects_bad_tiles():
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm
    x = torch.randn(4, 128, device=DEV).to(torch.bfloat16)
    w = torch.randn(2 * 96, 128, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError):
        gate_up_silu_gemm(x, w, column_tile=64)  # I = 96 is not a multiple of 64


def test_fused_true_past_64_tokens_runs_the_gemm():
    """gate_up_silu(..., fused=True) above the decode kernels' limit is the GEMM at the
    column tile gemm_column_tile picks (its rule is pinned in test_host.py); the default
    keeps the unfused pair."""
    from emberserve_amd.gate_up_silu import gate_up_silu_gemm, gemm_column_tile
    g = torch.Generator().manual_seed(77)
    w = (torch.randn(2 * 256, 512, generator=g) / 512 ** 0.5).to(torch.bfloat16).to(DEV)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = set()
    for tokens in (100, 600, 256 * (cus // 2 + 1)):
        x = (torch.randn(tokens, 512, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
        tile = gemm_column_tile(tokens, 256, x.device)
        tiles.add(tile)
        assert torch.equal(gate_up_silu(x, w, fused=True), gate_up_silu_gemm(x, w, column_tile=tile))
        assert torch.equal(gate_up_silu(x, w), gate_up_silu_torch(x, w))
    assert len(tiles) >= 2
    # I = 48: no GEMM tile fits, so the fused form falls back to the pair
    w48 = (torch.randn(2 * 48, 512, generator=g) / 512 ** 0.5).to(torch.bfloat16).to(DEV)
    x = (torch.randn(100, 512, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    assert torch.equal(gate_up_silu(x, w48, fused=True), gate_up_silu_torch(x, w48))