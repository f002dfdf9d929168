"""TEST ORACLE: basicsr's PSNR and 3-D SSIM in float64 numpy (the definitions the reference's
on-device metrics match, python/clarus/metrics.py:1-56). Only tests/ and bench.py's CPU leg use it.

  psnr(pred, gt)  python/clarus/metrics.py:41-56 (psnr_peak, psnr)
  ssim(pred, gt)  the 11 x 11 x 11 Gaussian (sigma 1.5, cv2.getGaussianKernel(11, 1.5)) over
                  (H, W, C) with replicate padding, C1 = (0.01 L)^2, C2 = (0.03 L)^2, L the PSNR
                  peak, mean of the map; applied as three separable 1-D passes with edge padding
                  (python/clarus/metrics.py:1-9, :164-199)
"""
from __future__ import annotations

import math

import numpy as np


def gaussian_1d(size: int = 11, sigma: float = 1.5) -> np.ndarray:
    """metrics.py:27-32: normalised exp(-(i - half)^2 / (2 sigma^2)) in float64."""
    half = size // 2
    g = np.array([math.exp(-((i - half) ** 2) / (2 * sigma * sigma)) for i in range(size)])
    return g / g.sum()


def psnr_peak(pred) -> float:
    """metrics.py:41-43: 1.0 if max(pred) <= 1 else 255.0."""
    return 1.0 if np.asarray(pred, dtype=np.float64).max() <= 1 else 255.0


def psnr(pred, gt) -> float:
    """metrics.py:46-56: float64 MSE, inf when identical."""
    a, b = np.asarray(pred, dtype=np.float64), np.asarray(gt, dtype=np.float64)
    mse = np.mean((a - b) ** 2)
    if mse == 0:
        return float("inf")
    return float(20.0 * np.log10(psnr_peak(a) / np.sqrt(mse)))


def _filter3(x: np.ndarray, g: np.ndarray) -> np.ndarray:
    """The separable 11-tap Gaussian along H, W and C of [H, W, C], edge (replicate) padding."""
    r = len(g) // 2
    for axis in range(3):
        pad = [(0, 0)] * 3
        pad[axis] = (r, r)
        xp = np.pad(x, pad, mode="edge")
        out = np.zeros_like(x)
        n = x.shape[axis]
        for t in range(len(g)):
            sl = [slice(None)] * 3
            sl[axis] = slice(t, t + n)
            out += g[t] * xp[tuple(sl)]
        x = out
    return x


def ssim(pred, gt) -> float:
    a, b = np.asarray(pred, dtype=np.float64), np.asarray(gt, dtype=np.float64)
    peak = psnr_peak(a)
    c1, c2 = (0.01 * peak) ** 2, (0.03 * peak) ** 2
    g = gaussian_1d()
    mu1, mu2 = _filter3(a, g), _filter3(b, g)
    s11 = _filter3(a * a, g) - mu1 * mu1
    s22 = _filter3(b * b, g) - mu2 * mu2
    s12 = _filter3(a * b, g) - mu1 * mu2
    m = ((2 * mu1 * mu2 + c1) * (2 * s12 + c2)) / ((mu1 * mu1 + mu2 * mu2 + c1) * (s11 + s22 + c2))
    return float(m.mean())
