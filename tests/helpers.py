"""Shared checks for the parity tests: ulp distance in the storage dtype."""

from __future__ import annotations

import torch

from tests.sum_order import torch_order_holds

_INT_VIEW = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}


def ordered_bits(t: torch.Tensor) -> torch.Tensor:
    """Maps floats to integers whose difference is the ulp distance (sign-magnitude to
    two's complement; +0 and -0 both map to 0)."""
    b = t.contiguous().view(_INT_VIEW[t.dtype]).to(torch.int64)
    mag_mask = 0x7FFF if t.dtype != torch.float32 else 0x7FFFFFFF
    return torch.where(b < 0, -(b & mag_mask), b)


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    assert a.dtype == b.dtype and a.shape == b.shape, (a.dtype, b.dtype, a.shape, b.shape)
    return (ordered_bits(a.cpu()) - ordered_bits(b.cpu())).abs()


def assert_ulp(got: torch.Tensor, want: torch.Tensor, max_ulp: int, what: str = "") -> None:
    d = ulp_diff(got, want)
    worst = int(d.max()) if d.numel() else 0
    assert worst <= max_ulp, (
        f"{what}: max ulp diff {worst} > {max_ulp} "
        f"({int((d > max_ulp).sum())} of {d.numel()} elements)")


def assert_bitexact(got: torch.Tensor, want: torch.Tensor, what: str = "") -> None:
    g, w = got.cpu(), want.cpu()
    assert g.dtype == w.dtype and g.shape == w.shape, (what, g.dtype, w.dtype, g.shape, w.shape)
    same = g.contiguous().view(_INT_VIEW.get(g.dtype, g.dtype)) == w.contiguous().view(_INT_VIEW.get(w.dtype, w.dtype))
    assert bool(same.all()), f"{what}: {int((~same).sum())} of {same.numel()} elements differ"


_MANT_BITS = {torch.float16: 10, torch.bfloat16: 7, torch.float32: 23}
_MIN_ULP = {torch.float16: 2.0 ** -24, torch.bfloat16: 2.0 ** -133, torch.float32: 2.0 ** -149}


def ulp_of(v: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The spacing of `dtype` at |v| (float64 result)."""
    _, e = torch.frexp(v.double().abs())
    u = torch.ldexp(torch.ones_like(v, dtype=torch.float64), (e - 1 - _MANT_BITS[dtype]).to(torch.int32))
    u = torch.where(v == 0, torch.zeros_like(u), u)
    return torch.clamp(u, min=_MIN_ULP[dtype])


def assert_rope_of_norm_close(got: torch.Tensor, want: torch.Tensor, y_ref: torch.Tensor,
                              cos_rows: torch.Tensor, sin_rows: torch.Tensor, norm_ulp: int,
                              what: str = "") -> None:
    """Checks a norm-then-rope output against the oracle's, allowing the norm its stated
    ulp budget and propagating it exactly through the rotation:
        |got - want| <= norm_ulp * (|c| ulp(y1) + |s| ulp(y2)) + ulp(want)
    for o1 = y1 c - y2 s (and the mirror for o2). `y_ref` is the oracle's normalised head
    rows [..., D], `cos_rows`/`sin_rows` the per-token table rows [N, D/2] (broadcast over
    heads). A plain ulp bound on the output would be meaningless where the rotation cancels
    to near zero: one ulp of y there is many ulp of the result."""
    dt = got.dtype
    half = y_ref.shape[-1] // 2
    c = cos_rows.double().unsqueeze(1).abs()
    s = sin_rows.double().unsqueeze(1).abs()
    u1 = ulp_of(y_ref[..., :half], dt)
    u2 = ulp_of(y_ref[..., half:], dt)
    prop1 = norm_ulp * (c * u1 + s * u2)
    prop2 = norm_ulp * (c * u2 + s * u1)
    bound = torch.cat((prop1, prop2), dim=-1) + ulp_of(want, dt)
    diff = (got.cpu().double() - want.double()).abs()
    bad = diff > bound
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {bad.numel()} elements outside the propagated norm "
        f"tolerance (worst excess {float((diff - bound).max()):.3g})")


_MANT = {torch.float16: 10, torch.bfloat16: 7}


def _ulp_of(v: torch.Tensor, dtype) -> torch.Tensor:
    a = v.abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - _MANT[dtype])


def check_gate_up(got: torch.Tensor, want: torch.Tensor, gu: torch.Tensor, absdot: torch.Tensor, hidden: int,
                  what: str, min_exact: float = 0.98, parts: int = 64) -> None:
    """A fused gate_up + silu_and_mul result against the oracle. `gu` [rows, 2I] holds the
    projections rounded to the dtype (float64 dot products), `absdot` the matching sums of
    |x_k w_k|. The kernel's fp32 sums differ from the exact dot product by at most
    n 2^-24 sum|x w| (n = hidden / 32 + 32 + parts roundings on any path; products of two
    fp16/bf16 values are exact in fp32), plus their own rounding to the dtype (one ulp).
    Those projection errors are carried through the activation; two ulp of round(silu(g))
    times |u| (a rounding flip, and the activation's own exp against torch's silu) and two
    ulp of the output are added. At least `min_exact` of the elements must be
    bit-identical."""
    dtype = want.dtype
    gu = gu.double()
    inter = gu.shape[1] // 2
    dgu = _ulp_of(gu, dtype) + (hidden / 32 + 32 + parts) * 2.0 ** -24 * absdot.double()
    g, u = gu[:, :inter], gu[:, inter:]
    dg, du = dgu[:, :inter], dgu[:, inter:]
    sig = torch.sigmoid(g)
    dsilu = (sig * (1 + g * (1 - sig))).abs().clamp_max(1.1)
    act = g * sig
    tol = (dsilu * u.abs() * dg + act.abs() * du + dg * du + 2 * _ulp_of(act, dtype) * u.abs()
           + 2 * _ulp_of(want.double(), dtype))
    gotd = got.cpu().double()
    err = (gotd - want.double()).abs()
    bad = err > tol
    if bool(bad.any()):
        i = int((err / tol).flatten().argmax())
        t, j = divmod(i, inter)
        raise AssertionError(f"{what}: {int(bad.sum())} of {err.numel()} out of tolerance, worst ratio "
                             f"{float((err / tol).max()):.2f} at [{t}, {j}]: g {float(g[t, j])!r} "
                             f"u {float(u[t, j])!r} got {float(gotd[t, j])!r} want {float(want[t, j])!r}")
    exact = float((gotd == want.double()).float().mean())
    assert exact >= min_exact, f"{what}: only {exact:.4f} of the elements bit-exact"


def norm_bitexact_expected(dtype: torch.dtype, cols: int) -> bool:
    """The gfx950 norm kernels sum rows of <= 512 half-precision elements (a multiple of 32)
    in the order of PyTorch's CPU sum, so their normalised rows are bit-identical to the
    oracle's wherever this host's torch really sums in that order."""
    return dtype in (torch.float16, torch.bfloat16) and cols % 32 == 0 and cols <= 512 and \
        torch_order_holds(cols)
