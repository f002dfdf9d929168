"""EVSSM's selective scan (the reference's TorchOps.selective_scan, python/clarus/ops/torch_ref.py:
312-341; its Triton scan8_kernel / carry_kernel, kernels/ssm.py:28-190).

CPU: the oracle's chunked closed form against the definition run as a float64 sequential
recurrence (h_l = exp(delta_l A) h_{l-1} + delta_l B_l u_l, y_l = C_l . h_l + D u_l), on small
crops with chunk boundaries inside them and a slowly decaying state.
GPU: clarus_hip_selective_scan (segments scanned in parallel, joined by their start states)
against the oracle at the reference's own test shapes (tools/test_kernels.py:264-268: u bf16 /
fp32, dbl N(0, 1), dt_w 0.5 N, dt_bias N - 2, D N, A = -U(0.5, 4.5)), within 1e-5 of the output
scale (the reference holds its kernel to 1e-3); and at EVSSM's level-0 crop (384 x 384 = 147456
steps, 96 channels, r = 3) against the float64 recurrence, where the segment joins matter.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.torch_ref import TorchRef

REF = TorchRef(torch.float32, "cpu")


def scan_inputs(t, h, w, d, r, seed, u_dtype=torch.float32, slow=False):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(t, h, w, d, generator=g).to(u_dtype)
    dbl = torch.randn(t, h, w, r + 16, generator=g)
    dtw = torch.randn(d, r, generator=g) * 0.5
    dtb = torch.randn(d, generator=g) - 2
    dsk = torch.randn(d, generator=g)
    A = -torch.rand(d, 8, generator=g) * 4 - 0.5
    if slow:  # long memory: decays close to 1 per step
        A = -torch.rand(d, 8, generator=g) * 0.02 - 0.001
    return u, dbl, dtw, dtb, A, dsk


def recurrence64(u, dbl, dtw, dtb, A, dsk):
    """The definition, float64, one step at a time (vectorised over crops, channels, states)."""
    t, hh, ww, d = u.shape
    r = dtw.shape[1]
    u = u.reshape(t, -1, d).double().numpy()
    dbl = dbl.reshape(t, -1, dbl.shape[-1]).double().numpy()
    dt = dbl[..., :r] @ dtw.double().numpy().T + dtb.double().numpy()
    delta = np.where(dt <= 20.0, np.log1p(np.exp(np.minimum(dt, 20.0))), dt)
    a = A.double().numpy()
    h = np.zeros((t, d, 8))
    y = np.empty_like(u)
    for l in range(u.shape[1]):
        dl = delta[:, l][..., None]
        h = np.exp(dl * a) * h + (dl[..., 0] * u[:, l])[..., None] * dbl[:, l, None, r:r + 8]
        y[:, l] = np.einsum("tdn,tn->td", h, dbl[:, l, r + 8:r + 16]) + dsk.double().numpy() * u[:, l]
    return torch.from_numpy(y.reshape(t, hh, ww, d))


def rel(got, ref):
    return ((got.double() - ref.double()).abs().max() / ref.double().abs().max()).item()


@pytest.mark.parametrize("t,h,w,d,r,slow", [(2, 7, 13, 16, 3, False), (1, 9, 10, 24, 6, True), (3, 5, 5, 8, 2, False)])
def test_oracle_scan_vs_float64_recurrence(t, h, w, d, r, slow):
    args = scan_inputs(t, h, w, d, r, seed=h * w, slow=slow)
    got = REF.selective_scan(*args)
    assert got.dtype == torch.float32 and got.shape == (t, h, w, d)
    e = rel(got, recurrence64(*args))
    assert e < 2e-6, e


@pytest.mark.gpu
@pytest.mark.parametrize("t,h,w,d,r", [(2, 48, 64, 96, 3), (8, 96, 96, 192, 6), (1, 300, 300, 32, 2)])
@pytest.mark.parametrize("udt", [torch.bfloat16, torch.float32])
def test_hip_scan_reference_shapes(t, h, w, d, r, udt, gpu_device):
    from clarus_amd import _lib
    from clarus_amd.hip_ops import HipOps
    hip = HipOps(torch.bfloat16 if udt == torch.bfloat16 else torch.float32, gpu_device)
    args = scan_inputs(t, h, w, d, r, seed=d + r, u_dtype=udt)
    print(f"[scan] {t}x{h}x{w} d{d} r{r} u {udt}", flush=True)
    got = hip.selective_scan(*[a.to(gpu_device) for a in args]).cpu()
    print(f"[scan] kernel: {_lib.last_kernel()}")
    ref = REF.selective_scan(args[0].float(), *args[1:])
    e = rel(got, ref)
    print(f"[scan] rel err vs oracle {e:.2e}")
    assert got.dtype == torch.float32 and e < 1e-5, e


@pytest.mark.gpu
def test_hip_scan_evssm_level0_crop(gpu_device):
    """Two 384 x 384 crops (L = 147456), 96 channels, r = 3: many segments, joined by the carry
    pass; against the float64 recurrence (the oracle's closed form would take minutes here)."""
    from clarus_amd import _lib
    from clarus_amd.hip_ops import HipOps
    hip = HipOps(torch.bfloat16, gpu_device)
    args = scan_inputs(2, 384, 384, 96, 3, seed=5, u_dtype=torch.bfloat16)
    got = hip.selective_scan(*[a.to(gpu_device) for a in args]).cpu()
    kernel = _lib.last_kernel()
    assert "nseg=1 " not in kernel, kernel
    e = rel(got, recurrence64(*args))
    print(f"[scan] EVSSM level 0: {kernel}, rel err vs float64 {e:.2e}")
    assert e < 1e-5, e


@pytest.mark.gpu
def test_hip_scan_bench_workload(gpu_device):
    """The bench's EVSSM row as timed: all 8 crops of 384 x 384, 96 channels, r = 3 (the seeded
    inputs of workloads.evssm_scan_case), against the float64 recurrence on every crop."""
    from clarus_amd import _lib, workloads as wl
    from clarus_amd.hip_ops import HipOps
    case = wl.evssm_scan_case(HipOps(torch.bfloat16, gpu_device), gpu_device)
    print(f"[scan] bench workload {case.name}", flush=True)
    got = case.run().cpu()
    kernel = _lib.last_kernel()
    h = case.cpu
    e = rel(got, recurrence64(h["u"], h["dbl"], h["dtw"], h["dtb"], h["A"], h["dsk"]))
    print(f"[scan] bench workload: {kernel}, rel err vs float64 {e:.2e}")
    assert got.shape == (8, 384, 384, 96) and e < 1e-5, e
