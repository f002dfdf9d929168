"""GPU: the boundary contracts of the `hip` backend.

1. Adapter validation (the reference's sweep, tools/test_ops_contracts.py:186-266). Each call goes
   through `Ops(["hip", "oracle_cpu"])`, a fresh dispatcher whose second backend is the oracle run
   on the host. Every case states the backend that HipOps' acceptance rules must pick. Either hip
   serves the call within the parity tolerances, or it declines before any launch (Unsupported)
   and the oracle serves it. Both results carry the oracle's dtype and shape. Differences from the
   reference's Triton expectations come from HipOps' own rules, each stated at its case:
   boxmean / dwconv take fp32 x in a bf16 backend and return the compute dtype as the torch
   backend does (torch_ref.py:133-155), and dwconv takes bias=None.
2. `out` aliasing `residual` (tools/test_kernel_contracts.py:160-181): with zero weights, unit
   bias and a zero residual the aliased output reads 1 everywhere; with random operands it equals
   the oracle run on a copy of the residual. conv3x3 through HipOps, and clarus_hip_gemm with
   c == res through the C ABI on each kernel family that takes a residual (ring streaming, DMA
   tiles, the library's own choice, the persistent register-resident kernel and the
   weight-streaming kernel).
"""
from __future__ import annotations

import collections
import ctypes

import pytest
import torch

from _tol import assert_bf16, assert_fp32
from clarus_amd.dispatch import Ops, register_backend
from oracle.torch_ref import TorchRef

pytestmark = pytest.mark.gpu
REF = TorchRef(torch.float32, "cpu")


def _to(obj, device):
    if isinstance(obj, torch.Tensor):
        return obj.to(device)
    if isinstance(obj, (list, tuple)):
        return type(obj)(_to(v, device) for v in obj)
    if isinstance(obj, dict):
        return {k: _to(v, device) for k, v in obj.items()}
    if hasattr(obj, "with_data"):  # a Small map
        return obj.with_data(obj.data.to(device))
    return obj


@register_backend("oracle_cpu")
class _CpuOracle:
    """The oracle as the chain's last backend: copies the arguments to the host, runs there, and
    returns the result on the caller's device (test infrastructure only)."""

    def __init__(self, dtype, device):
        self.dtype, self.device = dtype, device
        self._r = TorchRef(dtype, "cpu")

    def __getattr__(self, op):
        if op.startswith("_"):
            raise AttributeError(op)
        fn = getattr(self._r, op)

        def call(*args, **kwargs):
            return _to(fn(*_to(args, "cpu"), **_to(kwargs, "cpu")), self.device)
        return call


def rnd(g, *shape, scale=1.0, dtype=torch.bfloat16):
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.fixture(scope="module")
def chain(gpu_device):
    ops = Ops(["hip", "oracle_cpu"], torch.bfloat16, gpu_device, log=print)
    assert "hip" in ops.by_name, ops.skipped
    return ops


def _data(t):
    return t.data if hasattr(t, "with_data") else t


def run(ops, what, op, args, kw=None, expect="hip"):
    """Runs ops.<op>(*args, **kw) on the device, asserts the serving backend and holds the result to
    the oracle (its dtype and shape; values: fp32 outputs to 1e-5 relative, bf16 outputs to the
    bf16 rule against the fp32 oracle before its cast)."""
    kw = kw or {}
    dev = ops.device
    before = collections.Counter(ops.served)
    print(f"[contract] {what}: expect {expect}", flush=True)
    got = getattr(ops, op)(*_to(args, dev), **_to(kw, dev))
    torch.cuda.synchronize()
    served = [b for (o, b), v in ops.served.items() if o == op and v > before.get((o, b), 0)]
    assert served == [expect], f"{what}: served by {served}, expected {expect}"
    ref = _data(getattr(TorchRef(ops.dtype, "cpu"), op)(*_to(args, "cpu"), **_to(kw, "cpu")))
    ref32 = _data(getattr(REF, op)(*_to(args, "cpu"), **_to(kw, "cpu"))).float()
    g = _data(got)
    assert g.dtype == ref.dtype and tuple(g.shape) == tuple(ref.shape), \
        f"{what}: {g.dtype} {tuple(g.shape)} vs the oracle's {ref.dtype} {tuple(ref.shape)}"
    if g.dtype == torch.bfloat16:
        d, flips = assert_bf16(g.cpu(), ref32, what=what)
        print(f"[contract] {what}: {expect}, max|d| {d:.2e} (flips {flips})")
    else:
        e = assert_fp32(g.float().cpu(), ref32, what=what)
        print(f"[contract] {what}: {expect}, rel err {e:.2e}")


def test_adapter_validation(chain):
    """tools/test_ops_contracts.py:186-266 with bf16 activations: n, h, w, k, c = 2, 16, 24, 64, 48."""
    g = torch.Generator().manual_seed(7)
    dev = chain.device

    def R(*shape, scale=1.0, dtype=torch.bfloat16):  # views are taken on the device copies
        return rnd(g, *shape, scale=scale, dtype=dtype).to(dev)

    def N(*shape):
        return torch.randn(*shape, generator=g).to(dev)
    n, h, w, k, c = 2, 16, 24, 64, 48
    wide = R(n, h, w, 2 * k)
    x = wide[..., :k].contiguous()
    wt = R(k, c, scale=0.1)
    b = N(c)
    res = R(n, h, w, c)
    run(chain, "linear contiguous", "linear", (x, wt, b), dict(residual=res))
    run(chain, "linear x channel slice -> oracle", "linear", (wide[..., :k], wt, b), expect="oracle_cpu")
    run(chain, "linear x batch slice -> oracle", "linear", (R(2 * n, h, w, k)[::2], wt, b), expect="oracle_cpu")
    run(chain, "linear residual transposed -> oracle", "linear", (x, wt, b),
        dict(residual=R(n, w, h, c).transpose(1, 2)), expect="oracle_cpu")
    run(chain, "linear residual broadcast -> oracle", "linear", (x, wt, b), dict(residual=R(1, 1, 1, c)),
        expect="oracle_cpu")
    run(chain, "linear fp16 x -> oracle (no fp16 kernels)", "linear", (x.half(), wt, b), expect="oracle_cpu")

    w4 = R(c, k, 2, 2, scale=0.1)
    run(chain, "down contiguous", "down", (x, w4, b))
    run(chain, "down x channel slice -> oracle", "down", (wide[..., :k], w4, b), expect="oracle_cpu")
    wu = R(k, 4 * 16, scale=0.1)
    run(chain, "up residual contiguous", "up", (x, wu), dict(residual=R(n, 2 * h, 2 * w, 16)))
    run(chain, "up residual channel slice -> oracle", "up", (x, wu),
        dict(residual=R(n, 2 * h, 2 * w, 32)[..., :16]), expect="oracle_cpu")

    run(chain, "boxmean x channel slice -> oracle", "boxmean", (wide[..., :k], (8, 8)), expect="oracle_cpu")
    # HipOps.boxmean / dwconv write the compute dtype whatever x's dtype (as torch_ref.py:133-155),
    # so fp32 x stays on hip (the reference's Triton kernels write x's dtype and decline it)
    run(chain, "boxmean fp32 x (compute-dtype output)", "boxmean", (x.float(), (8, 8)))
    wd, bd = R(k, 1, 3, 3, scale=0.3), N(k)
    run(chain, "dwconv", "dwconv", (x, wd, bd))
    run(chain, "dwconv bias None (hip runs it without bias)", "dwconv", (x, wd, None))
    run(chain, "dwconv fp32 x (compute-dtype output)", "dwconv", (x.float(), wd, bd))
    run(chain, "dwconv x channel slice -> oracle", "dwconv", (wide[..., :k], wd, bd), expect="oracle_cpu")

    w3 = R(c, k, 3, 3, scale=0.05)
    run(chain, "conv3x3 x channel slice (uniform pixel stride)", "conv3x3", (wide[..., :k], w3, b))
    run(chain, "conv3x3 x H/W transposed -> oracle", "conv3x3", (R(n, w, h, k).transpose(1, 2), w3, b),
        expect="oracle_cpu")
    run(chain, "conv3x3 residual broadcast -> oracle", "conv3x3", (x, w3, b), dict(residual=R(1, 1, 1, c)),
        expect="oracle_cpu")
    we = R(3, k, 3, 3, scale=0.05)
    inp = torch.rand(n, 3, h, w, generator=g).to(dev)
    run(chain, "ending", "ending", (x, we, N(3), inp))
    run(chain, "ending x H/W transposed -> oracle", "ending",
        (R(n, w, h, k).transpose(1, 2), we, N(3), inp), expect="oracle_cpu")

    lw, lb = N(k), N(k)
    xf = (N(n, h, w, k) * 100).bfloat16()
    run(chain, "ln_mul_linear m channel slice", "ln_mul_linear", (xf, lw, lb, wide[..., k:], wt, b))
    run(chain, "ln_mul_linear m batch slice -> oracle", "ln_mul_linear",
        (xf, lw, lb, R(2 * n, h, w, k)[::2], wt, b), expect="oracle_cpu")
    run(chain, "ln_mul_linear m expanded batch -> oracle", "ln_mul_linear",
        (xf, lw, lb, R(1, h, w, k).expand(n, -1, -1, -1), wt, b), expect="oracle_cpu")
    run(chain, "ln_mul_linear residual broadcast -> oracle", "ln_mul_linear", (xf, lw, lb, x, wt, b),
        dict(residual=R(1, 1, 1, c)), expect="oracle_cpu")

    mix = N(n, k, c) * 0.1
    run(chain, "linear_per_image x channel slice", "linear_per_image", (wide[..., k:], mix), dict(residual=res))
    run(chain, "linear_per_image residual transposed -> oracle", "linear_per_image", (x, mix),
        dict(residual=R(n, w, h, c).transpose(1, 2)), expect="oracle_cpu")

    f = N(c, 8, 5)
    run(chain, "linear_patch_filter", "linear_patch_filter", (x, wt, b, f))
    run(chain, "linear_patch_filter fp32 x -> oracle (output dtype)", "linear_patch_filter",
        (x.float(), wt, b, f), expect="oracle_cpu")
    run(chain, "linear_patch_filter residual broadcast -> oracle", "linear_patch_filter", (x, wt, b, f),
        dict(residual=R(1, 1, 1, c)), expect="oracle_cpu")

    qkv = R(n, h, w, 3 * 96)
    t = torch.rand(2, generator=g).to(dev) + 0.5
    run(chain, "channel_attention", "channel_attention", (qkv, 2, t))
    run(chain, "channel_attention qkv channel slice -> oracle", "channel_attention",
        (R(n, h, w, 3 * 96 + 8)[..., :3 * 96], 2, t), expect="oracle_cpu")
    xp = R(n, h, w, c)
    run(chain, "patch_filter", "patch_filter", (xp, f))
    run(chain, "patch_filter residual broadcast -> oracle", "patch_filter", (xp, f),
        dict(residual=R(1, 1, 1, c)), expect="oracle_cpu")
    run(chain, "patch_corr wider x (channels beyond 2c)", "patch_corr", (wide, k // 2))
    run(chain, "patch_corr channel stride 2 -> oracle", "patch_corr", (R(n, h, w, 4 * k)[..., ::2], k // 2),
        expect="oracle_cpu")


# ------------------------------------------------------------------ out aliasing residual
@pytest.fixture(scope="module")
def hip_bf16(gpu_device):
    from clarus_amd.hip_ops import HipOps
    return HipOps(torch.bfloat16, gpu_device)


@pytest.mark.parametrize("rdt", [torch.bfloat16, torch.float32])
def test_conv3x3_out_aliases_residual(rdt, hip_bf16):
    """conv3x3(..., residual=r, out=r): zero weights, unit bias, r = 0 gives 1 (the reference's
    check); random weights give the oracle's result on a copy of r (also on a channel slice of a
    wider buffer, as RRDBNet's dense blocks write)."""
    g = torch.Generator().manual_seed(11)
    x = rnd(g, 1, 16, 24, 48).cuda()
    r = torch.zeros(1, 16, 24, 32, device="cuda", dtype=rdt)
    out = hip_bf16.conv3x3(x, torch.zeros(32, 48, 3, 3, device="cuda", dtype=torch.bfloat16),
                           torch.ones(32, device="cuda"), residual=r, out=r)
    torch.cuda.synchronize()
    assert out.data_ptr() == r.data_ptr() and bool((r == 1).all()), r.max().item()
    buf = rnd(g, 1, 37, 29, 96, dtype=rdt)
    w3 = rnd(g, 32, 48, 3, 3, scale=0.05)
    b = torch.randn(32, generator=g)
    xs = rnd(g, 1, 37, 29, 48)
    r0 = buf[..., 16:48].clone()
    ref = REF.conv3x3(xs, w3, b, act="lrelu", residual=r0, out_scale=0.2)
    bd = buf.cuda()
    rs = bd[..., 16:48]
    hip_bf16.conv3x3(xs.cuda(), w3.cuda(), b.cuda(), act="lrelu", residual=rs, out=rs, out_scale=0.2)
    torch.cuda.synchronize()
    what = f"conv3x3 out=residual slice {rdt}"
    if rdt == torch.bfloat16:
        assert_bf16(rs.cpu(), ref, what=what)
    else:
        assert_fp32(rs.cpu(), ref, what=what)
    assert torch.equal(bd[..., :16].cpu(), buf[..., :16]) and torch.equal(bd[..., 48:].cpu(), buf[..., 48:])


# (kernel family, entry, tile, m, k, n, residual / output dtype)
GEMM_ALIAS = [
    ("ring streaming", "gemm", 16, 3001, 64, 64, torch.bfloat16),
    ("ring streaming", "gemm", 16, 3001, 32, 200, torch.float32),
    ("DMA tile", "gemm", 11, 3001, 256, 256, torch.bfloat16),
    ("DMA 32x32 tile", "gemm", 13, 5000, 512, 512, torch.float32),
    ("library choice (c64 level-0 shape)", "gemm", 0, 20011, 64, 64, torch.bfloat16),
    ("library choice (c256)", "gemm", 0, 9000, 256, 256, torch.bfloat16),
    ("register-resident persistent", "wr", 0, 20011, 256, 256, torch.bfloat16),
    ("register-resident persistent", "wr", 0, 20011, 128, 512, torch.bfloat16),
    ("weight streaming", "wp", 0, 14400, 512, 512, torch.float32),
    ("weight streaming", "wp", 0, 20000, 256, 512, torch.bfloat16),
]


@pytest.mark.parametrize("family,entry,tile,m,k,n,dt", GEMM_ALIAS)
def test_gemm_out_aliases_residual(family, entry, tile, m, k, n, dt, hip_bf16):
    """clarus_hip_gemm / _wr / _wp with args->c == args->res (same pointer and strides)."""
    from clarus_amd import _lib
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator().manual_seed(m + k + n)
    print(f"[contract] gemm out=residual {family} tile {tile} M{m} K{k} N{n} {dt}", flush=True)

    def launch(x, w, b, sc, buf):
        args = _lib.GemmArgs(a=x.data_ptr(), wt=0, c=buf.data_ptr(), bias=_lib.ptr(b), scale=_lib.ptr(sc),
                             res=buf.data_ptr(), m=m, n=n, k=k, batch=1, lda=k, ldc=n, ldr=n,
                             a_dtype=_lib.BF16, w_dtype=_lib.BF16, c_dtype=_lib.dtype_code(dt),
                             r_dtype=_lib.dtype_code(dt), out_scale=1.0, tile=tile)
        if entry == "gemm":
            wt = w.t().contiguous()
            args.wt = wt.data_ptr()
            rc = lib.clarus_hip_gemm(ctypes.byref(args), stream)
        elif entry == "wr":
            rc = lib.clarus_hip_gemm_wr(ctypes.byref(args), hip_bf16._wr_pack(w, False).data_ptr(), stream)
        else:
            rc = lib.clarus_hip_gemm_wp(ctypes.byref(args), hip_bf16._frag_pack(w, False).data_ptr(), stream)
        _lib.check(rc, f"gemm {entry}")
        torch.cuda.synchronize()
        return _lib.last_kernel()

    # the reference's known answer: zero weights, unit bias, residual 0 -> 1
    x = rnd(g, m, k).cuda()
    buf = torch.zeros(m, n, device="cuda", dtype=dt)
    kern = launch(x, torch.zeros(k, n, device="cuda", dtype=torch.bfloat16), torch.ones(n, device="cuda"), None, buf)
    assert bool((buf == 1).all()), f"{family} ({kern}): max {buf.max().item()} min {buf.min().item()}"
    # random operands: the oracle on a copy of the residual
    xc, w = rnd(g, m, k), rnd(g, k, n, scale=k ** -0.5)
    b, sc, r0 = torch.randn(n, generator=g), torch.randn(n, generator=g), rnd(g, m, n, dtype=dt)
    ref = REF.linear(xc, w, b, scale=sc, residual=r0)
    buf = r0.cuda()
    kern = launch(xc.cuda(), w.cuda(), b.cuda(), sc.cuda(), buf)
    what = f"gemm out=residual {family} ({kern}) M{m} K{k} N{n} {dt}"
    if dt == torch.bfloat16:
        d, flips = assert_bf16(buf.cpu(), ref, what=what)
        print(f"[contract] {what}: max|d| {d:.2e} flips {flips}")
    else:
        e = assert_fp32(buf.cpu(), ref, what=what)
        print(f"[contract] {what}: rel err {e:.2e}")
