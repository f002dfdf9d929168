"""On-device PSNR / SSIM for clarus's evaluation loop, on HIP kernels (clarus_hip_psnr_ssim).

`HipMetrics` has the interface of the reference's TritonMetrics (python/clarus/metrics.py:164-246):
`scratch(h, w)` returns the device buffers for one image shape (shared by the callers holding
one, freed with the last), and `compute(out_u8, gt_u8, res, scratch)` writes res[0] = PSNR and
res[1] = SSIM (float64, on the device) without a host synchronisation, so it can be captured in
the worker's graph (python/clarus/worker.py:98-111). Definitions are basicsr's: PSNR from the
exact integer sum of squared differences with peak 1 if max(pred) <= 1 else 255; SSIM the 3-D
11 x 11 x 11 Gaussian (sigma 1.5) over (H, W, C) with replicate padding, moments in fp64.

    m = make_metrics(device, "hip")
    res = torch.zeros(2, device=device, dtype=torch.float64)
    m.compute(out_u8, gt_u8, res, m.scratch(h, w))
"""
from __future__ import annotations

import weakref

import torch

from . import _lib


class _Scratch:
    """Device workspace of clarus_hip_psnr_ssim for one image shape (a class so that it can be
    weakly cached)."""

    def __init__(self, lib, h: int, w: int, device):
        self.h, self.w = h, w
        self.nbytes = lib.clarus_hip_psnr_ssim_workspace(h, w)
        self.buf = torch.empty(max(self.nbytes, 16), dtype=torch.uint8, device=device)


class HipMetrics:
    def __init__(self, device):
        dev = torch.device(device)
        if torch.version.hip is None or dev.type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError("HipMetrics needs a HIP device")
        self.device = dev
        self.lib = _lib.load()
        self._live = weakref.WeakValueDictionary()

    def scratch(self, h: int, w: int) -> _Scratch:
        """Device scratch for [h, w, 3] images (about 1.4 bytes per pixel). The caller keeps it
        alive as long as anything (e.g. a captured graph) may use it; callers asking for the same
        shape while one is alive share it (they must run on one stream)."""
        s = self._live.get((h, w))
        if s is None:
            s = _Scratch(self.lib, h, w, self.device)
            self._live[(h, w)] = s
        return s

    def compute(self, out_u8: torch.Tensor, gt_u8: torch.Tensor, res: torch.Tensor, scratch=None):
        """out_u8, gt_u8: contiguous [H, W, 3] uint8 on the device. Writes res[0] = PSNR, res[1] =
        SSIM (res float64 on the device, contiguous, at least 2 elements)."""
        if out_u8.dtype != torch.uint8 or gt_u8.dtype != torch.uint8 or out_u8.shape != gt_u8.shape:
            raise ValueError("metrics: uint8 images of one shape")
        if out_u8.dim() != 3 or out_u8.shape[-1] != 3 or not (out_u8.is_contiguous() and gt_u8.is_contiguous()):
            raise ValueError("metrics: contiguous [H, W, 3] images")
        if res.dtype != torch.float64 or not res.is_contiguous() or res.numel() < 2 or res.device != out_u8.device:
            raise ValueError("metrics: res must be a contiguous float64 device tensor of >= 2 elements")
        h, w, _ = out_u8.shape
        b = scratch if scratch is not None else self.scratch(h, w)
        if (b.h, b.w) != (h, w):
            raise ValueError(f"metrics scratch is for {b.h}x{b.w}, image is {h}x{w}")
        _lib.check(self.lib.clarus_hip_psnr_ssim(out_u8.data_ptr(), gt_u8.data_ptr(), h, w, res.data_ptr(),
                                                 b.buf.data_ptr(), b.nbytes,
                                                 torch.cuda.current_stream(out_u8.device).cuda_stream), "psnr_ssim")


def make_metrics(device, backend: str = "hip"):
    """The metrics object of this backend ("hip"); the reference's make_metrics
    (python/clarus/metrics.py:272-280) would return it for backend "hip"."""
    if backend != "hip":
        raise ValueError(f"clarus_amd provides the 'hip' metrics backend, not {backend!r}")
    return HipMetrics(device)
