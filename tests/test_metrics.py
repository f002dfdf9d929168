"""PSNR / SSIM (the reference's on-device metrics, python/clarus/metrics.py).

CPU: the float64 oracle (oracle/metrics_ref.py) pinned by
  * values the reference itself wrote (tests/golden/metrics.safetensors): its host psnr() (basicsr
    rule) bit for bit, and its TorchMetrics (fp32 SSIM) within its own fp32 accuracy;
  * a brute-force 11 x 11 x 11 Gaussian convolution with replicate padding (no separability);
  * closed forms: identical images (SSIM 1, PSNR inf), two constant images
    (SSIM = (2 u v + C1) / (u^2 + v^2 + C1)), the peak rule (max(pred) <= 1 -> peak 1).
GPU: HipMetrics (clarus_hip_psnr_ssim) against the oracle on the same fixtures and at 720p:
PSNR within 1e-12, SSIM within 1e-9 (fp64 moments); also captured in a HIP graph.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file

from oracle import metrics_ref as mr

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "metrics.safetensors")


def metric_cases():
    with safe_open(GOLDEN, "pt") as f:
        names = [c[0] for c in json.loads(f.metadata()["cases"])]
    t = load_file(GOLDEN)
    return {n: {k.split(".", 1)[1]: v for k, v in t.items() if k.startswith(n + ".")} for n in names}


def test_oracle_matches_reference_metrics():
    for name, c in metric_cases().items():
        a, b = c["pred"].numpy(), c["gt"].numpy()
        p = mr.psnr(a, b)
        assert p == c["psnr"].item(), (name, p, c["psnr"].item())
        assert p == c["torch_metrics"][0].item() or (math.isinf(p) and math.isinf(c["torch_metrics"][0].item()))
        s = mr.ssim(a, b)
        # the reference's TorchMetrics runs its SSIM in fp32 with moments about 128: about 1e-7 of
        # the float64 value on 0..255 images; on a peak-1 image (values 0 / 1) the centred squares
        # (~128^2) cancel to variances of ~0.25 in fp32, which moves its SSIM by ~1e-3 there (the
        # float64 definition, basicsr's, is what the oracle and the HIP kernels compute)
        tol = 2e-6 if mr.psnr_peak(a) == 255.0 else 5e-3
        assert abs(s - c["torch_metrics"][1].item()) < tol, (name, s, c["torch_metrics"][1].item())


def test_oracle_ssim_vs_brute_force_3d():
    g = np.random.default_rng(3)
    a = g.integers(0, 256, (13, 17, 3)).astype(np.float64)
    b = np.clip(a + g.normal(0, 20, a.shape), 0, 255).round()
    k1 = mr.gaussian_1d()
    k3 = k1[:, None, None] * k1[None, :, None] * k1[None, None, :]

    def conv(x):  # the 3-D kernel applied directly, replicate padding on every axis
        xp = np.pad(x, 5, mode="edge")
        out = np.zeros_like(x)
        for i in range(x.shape[0]):
            for j in range(x.shape[1]):
                for c in range(3):
                    out[i, j, c] = (xp[i:i + 11, j:j + 11, c:c + 11] * k3).sum()
        return out
    mu1, mu2 = conv(a), conv(b)
    s11, s22, s12 = conv(a * a) - mu1 ** 2, conv(b * b) - mu2 ** 2, conv(a * b) - mu1 * mu2
    c1, c2 = (0.01 * 255) ** 2, (0.03 * 255) ** 2
    ref = (((2 * mu1 * mu2 + c1) * (2 * s12 + c2)) / ((mu1 ** 2 + mu2 ** 2 + c1) * (s11 + s22 + c2))).mean()
    assert abs(mr.ssim(a, b) - ref) < 1e-13


def test_oracle_closed_forms():
    g = np.random.default_rng(4)
    a = g.integers(0, 256, (9, 14, 3))
    assert mr.ssim(a, a) == pytest.approx(1.0, abs=1e-15) and math.isinf(mr.psnr(a, a))
    u, v = 200.0, 31.0
    c1 = (0.01 * 255) ** 2
    assert mr.ssim(np.full((12, 10, 3), u), np.full((12, 10, 3), v)) == pytest.approx(
        (2 * u * v + c1) / (u * u + v * v + c1), rel=1e-14)
    # peak 1 for max(pred) <= 1: one differing element of 3 * 4 * 5 -> MSE 1 / 60
    p, q = np.zeros((4, 5, 3)), np.zeros((4, 5, 3))
    p[0, 0, 0] = 1
    assert mr.psnr(p, q) == pytest.approx(10 * math.log10(60.0), abs=1e-12)
    assert mr.psnr(p * 255, q) == pytest.approx(10 * math.log10(60.0), abs=1e-12)  # peak 255, MSE 255^2 / 60
    assert mr.psnr(p * 2, q) == pytest.approx(20 * math.log10(255.0 / math.sqrt(4 / 60.0)), abs=1e-12)


# --------------------------------------------------------------------- GPU
@pytest.fixture(scope="module")
def hipm(gpu_device):
    from clarus_amd.metrics import make_metrics
    return make_metrics(gpu_device, "hip")


def _check(m, a, b, dev, what):
    res = torch.zeros(2, dtype=torch.float64, device=dev)
    m.compute(torch.from_numpy(np.ascontiguousarray(a)).to(dev), torch.from_numpy(np.ascontiguousarray(b)).to(dev),
              res)
    p, s = res.tolist()
    rp, rs = mr.psnr(a, b), mr.ssim(a, b)
    print(f"[metrics] {what}: psnr {p:.12f} (oracle {rp:.12f}) ssim {s:.12f} (oracle {rs:.12f})")
    assert (math.isinf(p) and math.isinf(rp)) or abs(p - rp) < 1e-12, (what, p, rp)
    assert abs(s - rs) < 1e-9, (what, s, rs)
    return p, s


@pytest.mark.gpu
def test_hip_metrics_on_reference_fixtures(hipm, gpu_device):
    for name, c in metric_cases().items():
        _check(hipm, c["pred"].numpy(), c["gt"].numpy(), gpu_device, name)


@pytest.mark.gpu
def test_hip_metrics_720p_and_graph(hipm, gpu_device):
    """A restored / ground-truth pair at 720p (smooth content, noise, blur-like shift); then the
    same compute captured in a HIP graph on a side stream, replayed after the inputs change."""
    g = np.random.default_rng(7)
    yy, xx = np.mgrid[0:720, 0:1280]
    base = np.stack([127 + 100 * np.sin(xx / (5 + 3 * c) + yy / (7 + c)) for c in range(3)], -1)
    gt = np.clip(base + g.normal(0, 12, base.shape), 0, 255).astype(np.uint8)
    pred = np.clip(0.6 * gt + 0.4 * np.roll(gt, 2, axis=1) + g.normal(0, 3, gt.shape), 0, 255).astype(np.uint8)
    _check(hipm, pred, gt, gpu_device, "720p")
    a = torch.from_numpy(pred).to(gpu_device)
    b = torch.from_numpy(gt).to(gpu_device)
    res = torch.zeros(2, dtype=torch.float64, device=gpu_device)
    sc = hipm.scratch(720, 1280)
    side = torch.cuda.Stream(gpu_device)
    side.wait_stream(torch.cuda.current_stream(gpu_device))
    with torch.cuda.stream(side):
        hipm.compute(a, b, res, sc)
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            hipm.compute(a, b, res, sc)
    torch.cuda.synchronize()
    for k in range(3):
        new = np.clip(pred.astype(np.int32) + k * 5, 0, 255).astype(np.uint8)
        a.copy_(torch.from_numpy(new))
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            graph.replay()
        side.synchronize()
        p, s = res.tolist()
        assert abs(p - mr.psnr(new, gt)) < 1e-12 and abs(s - mr.ssim(new, gt)) < 1e-9, (k, p, s)
