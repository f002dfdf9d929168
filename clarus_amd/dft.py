"""Real matrices of the 8x8 patch rfft2 / irfft2 pair (FFTformer's patch DFT as a GEMM).

A p x p patch is the vector x[y * p + x] (row-major). Coefficient j = 2 b + part holds the real
(part 0) or imaginary (part 1) component of rfft2 bin b = u * (p // 2 + 1) + v:

  Fwd[j, :]  so that Fwd . x = rfft2(x)  (unnormalised forward transform)
  Inv[:, j]  = irfft2(e_j, s=(p, p))      (e_j the unit coefficient, 1 or i at bin b)

irfft2 is ifft over u followed by a complex-to-real transform over v that keeps only the real
part of the v = 0 and v = p/2 bins after the u transform, so for every coefficient
  y[yy, xx] = w_v / p^2 * Re(c * exp(2 pi i (u yy + v xx) / p)),  w_v = 1 (v = 0, p/2) else 2,
with c = 1 (Re) or i (Im). This is exactly what the reference computes through torch.fft for
spectra that are not Hermitian in the v = 0 / p/2 columns (python/clarus/kernels/freq.py:79-93);
tests pin both matrices against numpy.fft and torch.fft.
"""
from __future__ import annotations

import functools

import numpy as np


@functools.lru_cache(maxsize=None)
def dft_matrices(p: int = 8) -> tuple[np.ndarray, np.ndarray]:
    """(Fwd [2 nb, p*p], Inv [p*p, 2 nb]) in float64, nb = p * (p // 2 + 1)."""
    nv = p // 2 + 1
    nb = p * nv
    yy, xx = np.meshgrid(np.arange(p), np.arange(p), indexing="ij")
    yy, xx = yy.ravel(), xx.ravel()
    fwd = np.zeros((2 * nb, p * p))
    inv = np.zeros((p * p, 2 * nb))
    for u in range(p):
        for v in range(nv):
            b = u * nv + v
            theta = 2.0 * np.pi * (u * yy + v * xx) / p
            # forward: sum x exp(-i theta) -> Re = sum x cos, Im = -sum x sin
            fwd[2 * b] = np.cos(theta)
            fwd[2 * b + 1] = -np.sin(theta)
            wv = 1.0 if v in (0, p // 2) else 2.0
            # inverse: Re(1 * e^{i theta}) = cos, Re(i * e^{i theta}) = -sin
            inv[:, 2 * b] = wv / (p * p) * np.cos(theta)
            inv[:, 2 * b + 1] = -wv / (p * p) * np.sin(theta)
    return fwd, inv


def filter_gains(f: np.ndarray) -> np.ndarray:
    """Real filter f [C, p, p//2+1] -> per-coefficient gains [C, 2 nb] (both parts of a bin
    get the bin's gain)."""
    c = f.shape[0]
    g = np.asarray(f, dtype=np.float64).reshape(c, -1)
    return np.repeat(g, 2, axis=1)
