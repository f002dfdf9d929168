"""PyTorch backend for the NON-GEMM ops the NAFNet harness needs (depthwise conv, TLC local
mean, scaled add, pixel (un)shuffle), run on the device with torch.

These ops are outside the HIP hot path; in clarus they fall through to the reference torch
backend (python/clarus/ops/torch_ref.py:133-218), whose semantics this follows. Registered as
"torch" only when clarus itself is not installed (a clarus installation provides its own full
"torch" backend). It deliberately implements no GEMM-family op: a GEMM call the `hip`
backend declines raises `Unsupported` instead of silently running on torch.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .dispatch import Backend, _host, register_backend
from .geometry import Small, box_geometry


class TorchSpatialOps(Backend):
    name = "torch"

    def boxmean(self, x, k) -> Small:
        """Valid (kh, kw) local mean from a 2-D prefix sum, cast to the compute dtype
        (torch_ref.py:133-141)."""
        n, h, w, c = x.shape
        k1, k2, oh, ow, pt, pl = box_geometry(h, w, k)
        s = F.pad(x.float().cumsum(dim=2).cumsum(dim=1), (0, 0, 1, 0, 1, 0))
        win = s[:, k1:, k2:] + s[:, :-k1, :-k2] - s[:, :-k1, k2:] - s[:, k1:, :-k2]
        return Small((win / (k1 * k2)).to(self.dtype), pt, pl, h, w)

    def dwconv(self, x, w, b, dil=1, gate=False, act=None):
        """Depthwise conv, 'same' padding, optional SimpleGate / GELU gate / GELU
        (torch_ref.py:143-155)."""
        kh, kw = w.shape[-2:]
        y = F.conv2d(x.permute(0, 3, 1, 2).float(), w.float(), b, padding=(dil * (kh // 2), dil * (kw // 2)),
                     dilation=dil, groups=x.shape[-1]).permute(0, 2, 3, 1)
        if gate:
            half = y.shape[-1] // 2
            first = F.gelu(y[..., :half]) if gate == "gelu" else y[..., :half]
            y = first * y[..., half:]
        if act == "gelu":
            y = F.gelu(y)
        return y.contiguous().to(self.dtype)

    def add_scaled(self, a, b, alpha, out_dtype=None, out=None):
        """a * alpha + b (torch_ref.py:201-207)."""
        y = a.float() * alpha + b.float()
        if out is not None:
            out.copy_(y)
            return out
        return y.to(out_dtype or self.dtype)

    def pixel_unshuffle(self, x, r=2):
        n, h, w, c = x.shape
        return x.view(n, h // r, r, w // r, r, c).permute(0, 1, 3, 5, 2, 4).reshape(n, h // r, w // r, r * r * c)

    def pixel_shuffle(self, x):
        n, h, w, c4 = x.shape
        c = c4 // 4
        return x.view(n, h, w, c, 2, 2).permute(0, 1, 4, 2, 5, 3).reshape(n, 2 * h, 2 * w, c)


if _host is None:
    register_backend("torch")(TorchSpatialOps)
