"""Parity criteria shared by the tests (the tolerances the HIP backend is held to).

fp32 outputs:  max|got - ref| / max|ref| <= 1e-5           (north star: 1e-5 relative)
bf16 outputs:  |got - ref| <= 2e-2 absolute for every element, where ref is the oracle's bf16
               result; an element may exceed 2e-2 only as a rounding-boundary flip, i.e. when
               got is within half a bf16 ulp (+ fp32 accumulation noise) of the oracle's fp32
               value before its cast. Both roundings are then correct roundings of values that
               differ by fp32 summation-order noise only; the count of such flips is reported
               and bounded.
"""
from __future__ import annotations

import torch

FP32_REL = 1e-5
BF16_ABS = 2e-2


def rel_err(got, ref) -> float:
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-300)).item()


def assert_fp32(got, ref, rel=FP32_REL, what=""):
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    assert torch.isfinite(got.cpu()).all(), f"{what}: non-finite output"
    e = rel_err(got, ref)
    assert e <= rel, f"{what}: rel err {e:.3e} > {rel:.1e}"
    return e


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (8 significant bits)."""
    a = x.abs().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(a)) - 7)


def assert_bf16(got, ref32, what="", max_flip_frac=1e-3):
    """got: bf16 result; ref32: the oracle's fp32 value before the cast to bf16."""
    assert got.dtype == torch.bfloat16, f"{what}: dtype {got.dtype}"
    assert got.shape == ref32.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref32.shape)}"
    g = got.double().cpu()
    r32 = ref32.double().cpu()
    rb = ref32.to(torch.bfloat16).double().cpu()
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    d = (g - rb).abs()
    over = d > BF16_ABS
    n_over = int(over.sum())
    if n_over:
        # every element beyond 2e-2 must be a correct rounding of ref32 up to fp32 noise
        slack = 0.5 * bf16_ulp(r32) * (1 + 1e-3) + 1e-5 * r32.abs()
        flip_ok = ((g - r32).abs() <= slack) | ~over
        assert bool(flip_ok.all()), (f"{what}: {int((~flip_ok).sum())} elements beyond 2e-2 that are not "
                                     f"rounding flips; max |d| {d.max().item():.3e}")
        assert n_over <= max(1, max_flip_frac * d.numel()), f"{what}: {n_over} rounding flips"
    return d.max().item(), n_over


def assert_abs(got, ref32, tol=BF16_ABS, what="", ulps=0.5):
    """The bf16 tolerance stated against the fp32 oracle: |got - ref32| <= tol absolute for every
    element, on top of the output's own rounding when got is bf16 (`ulps` bf16 ulps of ref32:
    half an ulp for one rounding of the output; no rounding of a bf16 output can stay within 2e-2
    of an fp32 value above 8, whose bf16 neighbours are 1/16 apart). Returns max|got - ref32|."""
    assert got.shape == ref32.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref32.shape)}"
    g = got.reshape(-1).cpu()
    r = ref32.reshape(-1).cpu()
    worst, excess = 0.0, 0
    step = 1 << 24
    for i in range(0, g.numel(), step):  # float64 in chunks: the full-size cases hold 10^8 elements
        gi, ri = g[i:i + step].double(), r[i:i + step].double()
        assert torch.isfinite(gi).all(), f"{what}: non-finite output"
        d = (gi - ri).abs()
        lim = tol + (ulps * bf16_ulp(ri) if got.dtype == torch.bfloat16 else 0.0)
        excess += int((d > lim).sum())
        worst = max(worst, d.max().item())
    assert excess == 0, f"{what}: {excess} elements beyond {tol:.0e} absolute; max|d| {worst:.3e}"
    return worst
