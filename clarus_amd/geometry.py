"""Shared argument types of the operator interface.

`Small` is the TLC local-mean map handed to `linear(..., mul=...)` and accepted as `linear`'s
input (python/clarus/ops/torch_ref.py:18-33); `box_geometry` gives the valid-window geometry
of a (kh, kw) local mean (torch_ref.py:36-41). The HIP backend accepts any object with the
same attributes, so clarus's own `Small` instances work unchanged.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Small:
    """Local-mean map before replicate padding: data [N, oh, ow, C]; the full-resolution
    value at (y, x) is data[clamp(y - pt, 0, oh - 1), clamp(x - pl, 0, ow - 1)]."""

    data: torch.Tensor
    pt: int
    pl: int
    H: int
    W: int

    def with_data(self, data):
        return Small(data, self.pt, self.pl, self.H, self.W)


try:  # inside a clarus installation, return clarus's own Small (its torch backend checks the type)
    from clarus.ops.torch_ref import Small as _HostSmall  # type: ignore
except ImportError:
    _HostSmall = None


def make_small(data, pt: int, pl: int, H: int, W: int):
    """A local-mean map of the host's Small type when clarus is installed, else the local one."""
    return (_HostSmall or Small)(data, pt, pl, H, W)


def is_small(x) -> bool:
    return all(hasattr(x, a) for a in ("data", "pt", "pl", "H", "W", "with_data")) and not torch.is_tensor(x)


def box_geometry(h: int, w: int, k):
    """(k1, k2, oh, ow, pt, pl) of a k (int: square) local mean over an h x w map."""
    kh, kw = (k, k) if isinstance(k, int) else k
    k1, k2 = min(h, kh), min(w, kw)
    oh, ow = h - k1 + 1, w - k2 + 1
    return k1, k2, oh, ow, (h - oh) // 2, (w - ow) // 2
