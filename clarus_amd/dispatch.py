"""Per-operator backend dispatch: the contract the `hip` backend plugs into.

This restates clarus's dispatcher (python/clarus/ops/__init__.py:27-138) so the HIP backend
can be registered, exercised and tested without the reference package on the GPU box.

Contract (same names, arguments and error behaviour as the reference):
  * `Unsupported` raised by a backend op hands the call to the next backend in the chain;
    any other exception propagates (ops/__init__.py:27-28,112-121).
  * `BackendUnavailable` raised by a backend constructor makes `Ops` log and skip that
    backend (ops/__init__.py:31-32,90-97).
  * `register_backend(name, "pkg.mod:Class")` or `@register_backend(name)` (:41-51).
  * `Backend.cached(t, tag, fn)` memoises a weight re-layout per (data_ptr, shape, tag)
    (:74-80).
  * `Ops(backends, dtype, device, overrides, log)`: ordered chain per op, `op_overrides`
    pin an op to one backend, `served[(op, backend)]` counts eager calls, `report()`
    summarises (:83-138).

Inside a clarus installation (`clarus.ops` importable) the names exported here ARE clarus's
own classes and registry, so `HipOps` subclasses clarus's `Backend`, raises clarus's
`Unsupported` and registers as "hip" in clarus's dispatcher.
"""
from __future__ import annotations

import collections
import importlib

import torch


class _Unsupported(Exception):
    """A backend op declines these arguments; the dispatcher tries the next backend."""


class _BackendUnavailable(Exception):
    """A backend cannot run on this device / dtype (raised by its constructor)."""


# name -> class, or "module:Class" resolved on first use
_REGISTRY: dict[str, object] = {
    "hip": "clarus_amd.hip_ops:HipOps",
}


def _register_backend(name: str, path: str | None = None):
    """Register a backend by 'module:Class' path, or use as a class decorator."""
    if path is not None:
        _REGISTRY[name] = path
        return None

    def deco(cls):
        cls.name = name
        _REGISTRY[name] = cls
        return cls
    return deco


def backend_class(name: str):
    entry = _REGISTRY.get(name)
    if entry is None:
        raise ValueError(f"{name!r} is not a registered backend (registered: {', '.join(sorted(_REGISTRY))})")
    if isinstance(entry, str):
        module, cls = entry.split(":")
        entry = getattr(importlib.import_module(module), cls)
        _REGISTRY[name] = entry
    return entry


class _Backend:
    """Base of op backends; `dtype` is the activation (compute) dtype."""

    name = "base"

    def __init__(self, dtype: torch.dtype, device: torch.device):
        self.dtype = dtype
        self.device = device
        self._cache: dict = {}

    def cached(self, t: torch.Tensor, tag: str, fn):
        """fn(t) computed once per (tensor storage, shape, tag): weight re-layouts."""
        key = (t.data_ptr(), tuple(t.shape), tag)
        hit = self._cache.get(key)
        if hit is None:
            hit = fn(t)
            self._cache[key] = hit
        return hit


def linear_ln_linear_unfused(self, x, w, bias=None, scale=None, residual=None, mul=None, out_dtype=None,
                      w2=None, bias2=None, gate2=False, ln=True, ln_eps=1e-6):
    """y = linear(x, w, ...) followed by u = linear(y, w2, bias2, ln=ln, gate=gate2): the
    residual GEMM and the LayerNorm GEMM that reads its output (NAFNet conv3 -> conv4 at
    python/clarus/models/nafnet.py's block). Returns (y, u). Backends without a fused kernel
    run the two ops."""
    y = self.linear(x, w, bias, scale=scale, residual=residual, mul=mul, out_dtype=out_dtype)
    return y, self.linear(y, w2, bias2, ln=ln, gate=gate2, ln_eps=ln_eps)


def linear_gate_linear_unfused(self, x, w1, b1=None, w2=None, b2=None, scale=None, ln=False, ln_eps=1e-6,
                               out_dtype=None):
    """u = linear(x, w1, b1, ln=ln, gate=True) followed by linear(u, w2, b2, scale=scale,
    residual=x): the feed-forward half of a NAFNet block (conv4 -> SimpleGate -> conv5 scaled by
    gamma on the block's running sum, python/clarus/models/nafnet/__init__.py:159-161) and the
    pointwise chain of BASELINE config 1. Returns the second op's output. Backends without a fused
    kernel run the two ops."""
    u = self.linear(x, w1, b1, ln=ln, gate=True, ln_eps=ln_eps)
    return self.linear(u, w2, b2, scale=scale, residual=x, out_dtype=out_dtype)


def linear_dwconv_unfused(self, x, w, bias=None, dw_w=None, dw_b=None, ln=True, gate=True, ln_eps=1e-6):
    """t = linear(x, w, bias, ln=ln) followed by dwconv(t, dw_w, dw_b, gate=gate): the first half of
    a NAFNet block (conv1 with LayerNorm -> depthwise 3x3 -> SimpleGate,
    python/clarus/models/nafnet/__init__.py:155-156). Backends without a fused kernel run the two
    ops."""
    return self.dwconv(self.linear(x, w, bias, ln=ln, ln_eps=ln_eps), dw_w, dw_b, gate=gate)


_FUSED_DEFAULTS = {"linear_ln_linear": linear_ln_linear_unfused, "linear_gate_linear": linear_gate_linear_unfused,
                   "linear_dwconv": linear_dwconv_unfused}


def give_pair_default(backend_cls) -> None:
    """Attach the unfused defaults (linear_ln_linear_unfused, linear_gate_linear_unfused,
    linear_dwconv_unfused) to a backend base class that lacks those ops, so every backend derived
    from it answers them with their two calls."""
    for name, fn in _FUSED_DEFAULTS.items():
        if not callable(getattr(backend_cls, name, None)):
            setattr(backend_cls, name, fn)


give_pair_default(_Backend)


class _Ops:
    """Ordered backend chain; `ops.<op>(...)` runs the first backend that accepts the call."""

    def __init__(self, backends: list[str], dtype: torch.dtype, device: torch.device,
                 overrides: dict[str, str] | None = None, log=print):
        self.dtype = dtype
        self.device = device
        self.backends: list[_Backend] = []
        self.skipped: dict[str, str] = {}
        for name in backends:
            try:
                self.backends.append(backend_class(name)(dtype, device))
            except _BackendUnavailable as exc:
                self.skipped[name] = str(exc)
                log(f"[dispatch] skipping backend {name!r}: {exc}")
        if not self.backends:
            raise RuntimeError(f"none of the backends {backends} could be constructed ({self.skipped})")
        self.by_name = {b.name: b for b in self.backends}
        self.overrides = dict(overrides or {})
        for op, bname in self.overrides.items():
            if bname not in self.by_name:
                raise ValueError(f"override pins {op!r} to {bname!r}, which is not in this chain")
        self.served: collections.Counter = collections.Counter()

    def _chain(self, op: str):
        chain = [self.by_name[self.overrides[op]]] if op in self.overrides else self.backends
        impls = [(b.name, getattr(b, op)) for b in chain if callable(getattr(b, op, None))]
        if not impls:
            raise AttributeError(f"{op!r}: not an op of any backend in the chain")
        return impls

    def __getattr__(self, op: str):
        if op.startswith("_"):
            raise AttributeError(op)
        impls = self._chain(op)
        served = self.served
        last = len(impls) - 1

        def call(*args, **kwargs):
            for i, (bname, fn) in enumerate(impls):
                try:
                    result = fn(*args, **kwargs)
                except _Unsupported:
                    if i == last:
                        raise
                    continue
                served[(op, bname)] += 1
                return result
        call.__name__ = op
        setattr(self, op, call)  # resolve the chain once per op
        return call

    def report(self) -> dict:
        """{"backends", "skipped", "overrides", "ops": {op: {backend: eager calls}}}."""
        per_op: dict = collections.defaultdict(dict)
        for (op, bname), count in sorted(self.served.items()):
            per_op[op][bname] = count
        return {"backends": [b.name for b in self.backends], "skipped": self.skipped,
                "overrides": self.overrides, "ops": dict(per_op)}


try:  # a clarus installation: use its classes and registry
    import clarus.ops as _host  # type: ignore
except ImportError:
    _host = None

if _host is not None:
    Unsupported = _host.Unsupported
    BackendUnavailable = _host.BackendUnavailable
    Backend = _host.Backend
    Ops = _host.Ops
    register_backend = _host.register_backend
    register_backend("hip", "clarus_amd.hip_ops:HipOps")
    give_pair_default(Backend)  # clarus's Backend has neither fused op of its own
else:
    Unsupported = _Unsupported
    BackendUnavailable = _BackendUnavailable
    Backend = _Backend
    Ops = _Ops
    register_backend = _register_backend
