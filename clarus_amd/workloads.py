"""Benchmark workloads of the GEMM-family hot path.

Each case holds seeded inputs resident on the device, a closure that runs the op once through
the `hip` backend, and its ALGORITHMIC flop and byte counts (the formulas of the measurement
plan; they are fixed by the op and shape, not read from counters):

  config 2 (NAFNet-w64 720p pointwise GEMMs, bf16, M = H * W pixels)
    expand c -> 2c + bias + SimpleGate : F = 4 M c^2, B = 2Mc (A) + 2Mc (out) + 4c^2 + 8c
    c -> c + bias, * beta, + residual  : F = 2 M c^2, B = 2Mc + 2 r M c + 2c^2 + 8c,
                                         r = 2 (bf16 residual / output) for c < 512, 4 (fp32) above
  config 3 (patch DFT, fp32, fused fwd 64->80 / filter / inv 80->64) per patch-channel:
    F = 2*64*80 + 6*40 + 2*80*64, B = 4*64 (in) + 4*64 (out); F priced at the bf16 MFMA peak (the
    kernels issue bf16 MFMAs, three per fp32-accurate product), so the bound is the HBM floor
  config 4 (Restormer MDTA, level l: C = 48 * 2^l, heads 2^l, HW = 921600 / 4^l), e = element size
    Gram + norms : F = heads (2 * 48^2 HW + 4 * 48 HW), B = 2 C HW e + heads * 48^2 * 4
    attn . V     : F = heads * 2 * 48^2 HW,          B = 2 C HW e
  config 5 (RRDBNet 3x3, bf16, M output pixels): F = 2 M 9 Cin Cout,
    B = 2 M_in Cin + 2 M Cout (+ 2 M 64 residual) + 18 Cin Cout
Peaks (MI355X datasheet): bf16 MFMA 2.5 PFLOP/s, fp32 MFMA 157.3 TFLOP/s, HBM 8 TB/s.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable

import torch

PEAK_FLOPS = {"bf16": 2.5e15, "fp32": 157.3e12, "fp64": 78.6e12}
PEAK_HBM = 8.0e12


@dataclass
class OpCase:
    name: str
    config: int
    dtype: str            # arithmetic type of the products: "bf16" or "fp32"
    flops: float
    nbytes: float
    run: Callable[[], object]
    cpu: dict = field(default_factory=dict)  # the op's inputs on the host
    # the same op on a CPU backend with the reference's op signatures (the caller passes the
    # backend, so this package never imports one): cpu_run(backend) runs it once on `cpu`
    cpu_run: Callable[[object], object] | None = None
    # cpu_run covers 1 / cpu_scale of the op's work (a bounded sample where the CPU backend would
    # take minutes); the reported CPU time is the sample's times cpu_scale
    cpu_scale: float = 1.0
    cpu_sample: str = ""
    # the MFMA instructions the kernel issues, whose peak prices the algorithmic flops (default:
    # the arithmetic type). The patch DFT ops compute fp32-accurate products as three bf16 MFMAs,
    # so their flops are priced at the bf16 peak, in config 3 as in the fused FFTformer DFFN op:
    # one rule for both, with the HBM floor as the bound wherever it is the larger
    mfma: str = ""

    def t_bound(self) -> tuple[float, str]:
        tm = self.flops / PEAK_FLOPS[self.mfma or self.dtype]
        tb = self.nbytes / PEAK_HBM
        # fp64 ops (the metrics) run on the vector ALUs; MI355X's fp64 vector and matrix peaks agree
        return (tm, "fp64" if self.dtype == "fp64" else "mfma") if tm >= tb else (tb, "hbm")


def kernel_of(case: OpCase) -> str:
    """Runs the case once and returns the kernel the library chose for its last launch."""
    from . import _lib
    case.run()
    return _lib.last_kernel()


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _kaiming_uniform_kn(g, cin, cout):
    """nn.Conv2d default 1x1 init (kaiming_uniform, a = sqrt(5): bound 1/sqrt(fan_in)) as [K, N]."""
    return ((torch.rand(cout, cin, generator=g) * 2 - 1) / math.sqrt(cin)).t().contiguous()


CONFIG2_LEVELS = [(64, 720, 1280), (128, 360, 640), (256, 180, 320), (512, 90, 160), (1024, 45, 80)]


def config2_names() -> list[str]:
    """Names of the config-2 step ops, in the order config2_cases builds them."""
    return [n for c, _, _ in CONFIG2_LEVELS for n in (f"c{c} expand+gate", f"c{c} c->c+scale+res")]


def config2_cases(hip, device, seed: int = 0, levels=None) -> list[OpCase]:
    """Per level: u = linear(x, We, be, gate=True); y = linear(u, Wc, bc, scale=beta, residual=r).
    levels: the widths c to build (all five by default)."""
    cases = []
    for c, h, w in CONFIG2_LEVELS:
        if levels is not None and c not in levels:
            continue
        g = _gen(seed + c)
        m = h * w
        x = torch.randn(1, h, w, c, generator=g).bfloat16()
        we = _kaiming_uniform_kn(g, c, 2 * c).bfloat16()
        be = torch.rand(2 * c, generator=g) * 0.2 - 0.1
        wc = _kaiming_uniform_kn(g, c, c).bfloat16()
        bc = torch.rand(c, generator=g) * 0.2 - 0.1
        beta = torch.randn(c, generator=g) * 0.1
        rdt = torch.float32 if c >= 512 else torch.bfloat16
        r = torch.randn(1, h, w, c, generator=g).to(rdt)
        cpu = dict(x=x, we=we, be=be, wc=wc, bc=bc, beta=beta, r=r, rdt=rdt)
        d = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in cpu.items()}
        u = hip.linear(d["x"], d["we"], d["be"], gate=True)  # also the c->c input
        cpu["u"] = u  # the c->c op's input as the device holds it

        def expand(d=d):
            return hip.linear(d["x"], d["we"], d["be"], gate=True)

        def cc(d=d, u=u):
            return hip.linear(u, d["wc"], d["bc"], scale=d["beta"], residual=d["r"], out_dtype=d["rdt"])
        rb = 2 if c < 512 else 4
        cpu["u_host"] = u.cpu()
        cases.append(OpCase(f"c{c} expand+gate", 2, "bf16", 4.0 * m * c * c,
                            2.0 * m * c + 2.0 * m * c + 4.0 * c * c + 8.0 * c, expand, cpu,
                            lambda r, d=cpu: r.linear(d["x"], d["we"], d["be"], gate=True)))
        cases.append(OpCase(f"c{c} c->c+scale+res", 2, "bf16", 2.0 * m * c * c,
                            2.0 * m * c + 2.0 * rb * m * c + 2.0 * c * c + 8.0 * c, cc, cpu,
                            lambda r, d=cpu: r.linear(d["u_host"], d["wc"], d["bc"], scale=d["beta"],
                                                      residual=d["r"], out_dtype=d["rdt"])))
    return cases


def config1_cases(hip32, device, seed: int = 0) -> list[OpCase]:
    """fp32 pointwise chain on x [1, 256, 256, 32]: as two ops (gate op, then scale + residual op;
    u makes the round trip through HBM: B counts x, u twice, x again and the output) and as one
    (linear_gate_linear: B = x read once, the output written once)."""
    g = _gen(seed)
    x = torch.randn(1, 256, 256, 32, generator=g)
    w1 = _kaiming_uniform_kn(g, 32, 64)
    b1 = torch.rand(64, generator=g) * 0.2 - 0.1
    w2 = _kaiming_uniform_kn(g, 32, 32)
    b2 = torch.rand(32, generator=g) * 0.2 - 0.1
    beta = torch.randn(32, generator=g) * 0.1
    host = (x, w1, b1, w2, b2, beta)
    d = [t.to(device) for t in host]
    m = 256 * 256

    def chain(d=d, r=None):
        r = r or hip32
        uu = r.linear(d[0], d[1], d[2], gate=True)
        return r.linear(uu, d[3], d[4], scale=d[5], residual=d[0])
    def fused(d=d, r=None):
        from .dispatch import linear_gate_linear_unfused
        r = r or hip32
        fn = getattr(r, "linear_gate_linear", None)
        args = (d[0], d[1], d[2], d[3], d[4])
        return fn(*args, scale=d[5]) if fn is not None else linear_gate_linear_unfused(r, *args, scale=d[5])
    flops = 2.0 * m * 32 * 64 + 2.0 * m * 32 * 32
    wbytes = 4.0 * (32 * 64 + 32 * 32) + 4.0 * (64 + 64)
    return [OpCase("config1 fp32 chain (gate, scale+res)", 1, "fp32", flops,
                   4.0 * m * 32 * 2 + 4.0 * m * 32 * 2 + wbytes, chain, {"inputs": host}, lambda r: chain(host, r)),
            OpCase("config1 fp32 chain, one op (linear_gate_linear)", 1, "fp32", flops, 4.0 * m * 32 * 2 + wbytes,
                   fused, {"inputs": host}, lambda r: fused(host, r))]


def config3_cases(hip32, device, seed: int = 0) -> list[OpCase]:
    cases = []
    for c, h, w in [(48, 720, 1280), (96, 360, 640), (192, 180, 320)]:
        g = _gen(seed + c)
        xh = torch.randn(1, h, w, c, generator=g)
        fh = torch.randn(c, 8, 5, generator=g)
        x, f = xh.to(device), fh.to(device)
        units = (h // 8) * (w // 8) * c
        cases.append(OpCase(f"patch_filter fused C{c} {h}x{w}", 3, "fp32",
                            units * (2.0 * 64 * 80 + 6 * 40 + 2.0 * 80 * 64), units * 4.0 * 128,
                            lambda x=x, f=f: hip32.patch_filter(x, f), {"x": xh, "f": fh},
                            lambda r, x=xh, f=fh: r.patch_filter(x, f), mfma="bf16"))
    return cases


def config4_cases(hip_bf16, hip32, device, seed: int = 0) -> list[OpCase]:
    cases = []
    for dt, hip in ((torch.float32, hip32), (torch.bfloat16, hip_bf16)):
        e = 4 if dt == torch.float32 else 2
        tag = "fp32" if dt == torch.float32 else "bf16"
        for lvl, h, w in [(0, 720, 1280), (1, 360, 640), (2, 180, 320), (3, 90, 160)]:
            g = _gen(seed + lvl)
            c, heads = 48 * 2 ** lvl, 2 ** lvl
            hw = h * w
            qkvh = torch.randn(1, h, w, 3 * c, generator=g).to(dt)
            th = torch.rand(heads, generator=g) * 1.5 + 0.5
            qkv, t = qkvh.to(device), th.to(device)
            cases.append(OpCase(f"mdta gram+norms+softmax l{lvl} {tag}", 4, tag,
                                heads * (2.0 * 48 * 48 * hw + 4.0 * 48 * hw), 2.0 * c * hw * e + heads * 48 * 48 * 4,
                                lambda hip=hip, qkv=qkv, t=t, heads=heads: hip.channel_attention(qkv, heads, t),
                                {"qkv": qkvh, "t": th},
                                lambda r, q=qkvh, t=th, heads=heads: r.channel_attention(q, heads, t)))
            a = hip.channel_attention(qkv, heads, t)
            wa = a.to(dt)  # the maps A [1, heads, 48, 48] in the activation dtype
            # the reference applies the maps as one per-image matrix blockdiag(A^T) through
            # linear_per_image (python/clarus/models/restormer/__init__.py:203-210)
            bd = torch.block_diag(*wa[0].transpose(1, 2).float().cpu()).unsqueeze(0)
            cases.append(OpCase(f"mdta attn.V l{lvl} {tag}", 4, tag, heads * 2.0 * 48 * 48 * hw, 2.0 * c * hw * e,
                                lambda hip=hip, qkv=qkv, wa=wa: hip.attention_apply(qkv, wa),
                                {"qkv": qkvh, "blockdiag": bd},
                                lambda r, q=qkvh, bd=bd, c=c: r.linear_per_image(q[..., 2 * c:], bd)))
    return cases


def config5_cases(hip, device, seed: int = 0) -> list[OpCase]:
    g = _gen(seed)
    h, w = 256, 384
    m = h * w
    bufh = torch.randn(1, h, w, 192, generator=g).bfloat16()
    buf = bufh.to(device)
    out = torch.empty(1, h, w, 192, dtype=torch.bfloat16, device=device)
    outh = torch.empty(1, h, w, 192, dtype=torch.bfloat16)
    cases = []

    def kn(cout, cin):
        return ((torch.randn(cout, cin, 3, 3, generator=g) * math.sqrt(2.0 / (cin * 9))) * 0.1).bfloat16()
    for cin in (64, 96, 128, 160):
        wh, bh = kn(32, cin), torch.zeros(32)
        wt, b = wh.to(device), bh.to(device)
        cases.append(OpCase(f"conv3x3 {cin}->32 +lrelu (slice)", 5, "bf16", 2.0 * m * 9 * cin * 32,
                            2.0 * m * (cin + 32) + 18.0 * cin * 32,
                            lambda cin=cin, wt=wt, b=b: hip.conv3x3(buf[..., :cin], wt, b, act="lrelu",
                                                                    out=buf[..., cin:cin + 32]),
                            {"buf": bufh, "w": wh},
                            lambda r, cin=cin, wt=wh, b=bh: r.conv3x3(bufh[..., :cin], wt, b, act="lrelu",
                                                                      out=bufh[..., cin:cin + 32])))
    w5h, b5h = kn(64, 192), torch.zeros(64)
    w5, b5 = w5h.to(device), b5h.to(device)
    cases.append(OpCase("conv3x3 192->64 *0.2 +res", 5, "bf16", 2.0 * m * 9 * 192 * 64,
                        2.0 * m * (192 + 64) + 2.0 * m * 64 + 18.0 * 192 * 64,
                        lambda: hip.conv3x3(buf, w5, b5, out_scale=0.2, residual=buf[..., :64], out=out[..., :64]),
                        {"buf": bufh, "w": w5h},
                        lambda r: r.conv3x3(bufh, w5h, b5h, out_scale=0.2, residual=bufh[..., :64],
                                            out=outh[..., :64])))
    for hh, ww in [(256, 384), (512, 768)]:
        xh = torch.randn(1, hh, ww, 64, generator=g).bfloat16()
        wh, bh = kn(64, 64), torch.zeros(64)
        x, wt, b = xh.to(device), wh.to(device), bh.to(device)
        mo = 4 * hh * ww
        cases.append(OpCase(f"up2 + conv3x3 64->64 +lrelu out {2 * hh}x{2 * ww}", 5, "bf16", 2.0 * mo * 9 * 64 * 64,
                            2.0 * hh * ww * 64 + 2.0 * mo * 64 + 18.0 * 64 * 64,
                            lambda x=x, wt=wt, b=b: hip.conv3x3(x, wt, b, act="lrelu", up2=True),
                            {"x": xh, "w": wh},
                            lambda r, x=xh, wt=wh, b=bh: r.conv3x3(x, wt, b, act="lrelu", up2=True)))
    return cases


def nafnet_pair_case(hip, device, seed: int = 0) -> OpCase:
    """The NAFNet-w64 720p level-3 residual GEMM and the LayerNorm GEMM on its output as one op
    (linear_ln_linear: conv3 (+ beta * . + fp32 residual) -> LN -> conv4 + SimpleGate), the
    forward's most frequent fused kernel (29 of these and 27 conv5 -> conv1 pairs per forward).
    M = 14400: F = 2 M 512 (512 + 1024); B = 2 M 512 (A) + 4 M 512 (residual) + 4 M 512 (y, fp32)
    + 2 M 512 (u, bf16) + 2 (512^2 + 512 * 1024) (weights) + 4 (512 + 1024 + 512) (vectors)."""
    g = _gen(seed + 3)
    m, k = 90 * 160, 512
    x = torch.randn(1, 90, 160, k, generator=g).bfloat16()
    w3 = _kaiming_uniform_kn(g, k, k).bfloat16()
    b3 = torch.rand(k, generator=g) * 0.2 - 0.1
    beta = torch.randn(k, generator=g) * 0.1
    r = torch.randn(1, 90, 160, k, generator=g)
    w4 = _kaiming_uniform_kn(g, k, 2 * k).bfloat16()
    b4 = torch.rand(2 * k, generator=g) * 0.2 - 0.1
    host = dict(x=x, w3=w3, b3=b3, beta=beta, r=r, w4=w4, b4=b4)
    d = {n: t.to(device) for n, t in host.items()}

    def pair(r_=None, d=d):
        from .dispatch import linear_ln_linear_unfused
        be = r_ or hip
        fn = getattr(be, "linear_ln_linear", None)
        args = (d["x"], d["w3"], d["b3"])
        kw = dict(scale=d["beta"], residual=d["r"], out_dtype=torch.float32, w2=d["w4"], bias2=d["b4"], gate2=True,
                  ln=True)
        return fn(*args, **kw) if fn is not None else linear_ln_linear_unfused(be, *args, **kw)
    flops = 2.0 * m * k * (k + 2 * k)
    nbytes = m * k * (2.0 + 4.0 + 4.0 + 2.0) + 2.0 * (k * k + k * 2 * k) + 4.0 * (k + 2 * k + k)
    return OpCase("nafnet L3 conv3 -> LN -> conv4 (fused pair)", 0, "bf16", flops, nbytes, pair, host,
                  lambda r_: pair(r_, host))


def nafnet_ffn_case(hip, device, seed: int = 0) -> OpCase:
    """The NAFNet-w64 720p level-0 feed-forward half-block as one op (linear_gate_linear: LN ->
    conv4 64 -> 128 + SimpleGate -> conv5 64 -> 64, * gamma + the block's running sum, bf16),
    two per forward (encoder and decoder block). M = 921600: F = 2 M 64 (128 + 64);
    B = 2 M 64 (x) + 2 M 64 (out) + 2 (64 * 128 + 64 * 64) (weights) + 4 (128 + 64 + 64) (vectors)."""
    g = _gen(seed + 5)
    m, c = 720 * 1280, 64
    x = torch.randn(1, 720, 1280, c, generator=g).bfloat16()
    w4 = _kaiming_uniform_kn(g, c, 2 * c).bfloat16()
    b4 = torch.rand(2 * c, generator=g) * 0.2 - 0.1
    w5 = _kaiming_uniform_kn(g, c, c).bfloat16()
    b5 = torch.rand(c, generator=g) * 0.2 - 0.1
    gamma = torch.randn(c, generator=g) * 0.1
    host = dict(x=x, w4=w4, b4=b4, w5=w5, b5=b5, gamma=gamma)
    d = {n: t.to(device) for n, t in host.items()}

    def run(r_=None, d=d):
        from .dispatch import linear_gate_linear_unfused
        be = r_ or hip
        fn = getattr(be, "linear_gate_linear", None)
        args = (d["x"], d["w4"], d["b4"], d["w5"], d["b5"])
        kw = dict(scale=d["gamma"], ln=True)
        return fn(*args, **kw) if fn is not None else linear_gate_linear_unfused(be, *args, **kw)
    flops = 2.0 * m * c * (2 * c + c)
    nbytes = 2.0 * m * c * 2 + 2.0 * (c * 2 * c + c * c) + 4.0 * (2 * c + 2 * c)
    return OpCase("nafnet L0 LN -> conv4 + gate -> conv5 + res (fused FFN)", 0, "bf16", flops, nbytes, run, host,
                  lambda r_: run(r_, host))


def nafnet_lndw_case(hip, device, seed: int = 0) -> OpCase:
    """The NAFNet-w64 720p level-0 first half-block as one op (linear_dwconv: LN -> conv1 64 -> 128
    -> depthwise 3x3 -> SimpleGate, bf16), two per forward. M = 921600: F = 2 M 64 128 (conv1) +
    2 M 128 9 (depthwise) + M 64 (gate); B = 2 M 64 (x) + 2 M 64 (out) + 2 * 64 * 128 (weight) +
    4 (128 + 9 * 128 + 128) (vectors, taps)."""
    g = _gen(seed + 7)
    m, c = 720 * 1280, 64
    x = torch.randn(1, 720, 1280, c, generator=g).bfloat16()
    w1 = _kaiming_uniform_kn(g, c, 2 * c).bfloat16()
    b1 = torch.rand(2 * c, generator=g) * 0.2 - 0.1
    dw = (torch.rand(2 * c, 1, 3, 3, generator=g) * 2 - 1) / 3.0
    dwb = torch.rand(2 * c, generator=g) * 0.2 - 0.1
    host = dict(x=x, w1=w1, b1=b1, dw=dw, dwb=dwb)
    d = {n: t.to(device) for n, t in host.items()}

    def run(r_=None, d=d):
        from .dispatch import linear_dwconv_unfused
        be = r_ or hip
        fn = getattr(be, "linear_dwconv", None)
        args = (d["x"], d["w1"], d["b1"], d["dw"], d["dwb"])
        return fn(*args) if fn is not None else linear_dwconv_unfused(be, *args)
    flops = 2.0 * m * c * 2 * c + 2.0 * m * 2 * c * 9 + m * c
    nbytes = 2.0 * m * c * 2 + 2.0 * c * 2 * c + 4.0 * (2 * c + 9 * 2 * c + 2 * c)
    return OpCase("nafnet L0 LN -> conv1 -> dwconv + gate (fused first half)", 0, "bf16", flops, nbytes, run, host,
                  lambda r_: run(r_, host))


def nafnet_dw_case(hip, device, level: int, seed: int = 0) -> OpCase:
    """The NAFNet-w64 720p depthwise 3x3 + SimpleGate of one block (dwconv on conv1's 2c channels
    -> c, bf16, bias; the reference block's and the fused ops' call alike): level 3 (90 x 160,
    c = 512, 31 calls per forward) or level 0 (720 x 1280, c = 64, 2 calls without the fused first
    half). M pixels: F = 2 M 2c 9 (taps) + M c (gate); B = 2 M 2c (in) + 2 M c (out) + 4 (9 + 1) 2c
    (taps, bias)."""
    g = _gen(seed + 13 + level)
    h, w, c = {3: (90, 160, 512), 0: (720, 1280, 64)}[level]
    m = h * w
    x = torch.randn(1, h, w, 2 * c, generator=g).bfloat16()
    dw = (torch.rand(2 * c, 1, 3, 3, generator=g) * 2 - 1) / 3.0
    dwb = torch.rand(2 * c, generator=g) * 0.2 - 0.1
    host = dict(x=x, dw=dw, dwb=dwb)
    d = {n: t.to(device) for n, t in host.items()}

    def run(r_=None, d=d):
        return (r_ or hip).dwconv(d["x"], d["dw"], d["dwb"], gate=True)
    flops = 2.0 * m * 2 * c * 9 + m * c
    nbytes = 2.0 * m * 2 * c + 2.0 * m * c + 4.0 * 10 * 2 * c
    return OpCase(f"nafnet L{level} dwconv 3x3 + SimpleGate {h}x{w} c{2 * c}->{c}", 0, "bf16", flops, nbytes, run,
                  host, lambda r_: run(r_, host))


def fftformer_dffn_case(hip, device, seed: int = 0) -> OpCase:
    """FFTformer level-0 DFFN project_in + frequency filter at 720p as one op (linear_patch_filter:
    LayerNorm eps 1e-5 -> 1x1 conv 48 -> 288 + bias -> per-patch rfft2 * filter -> irfft2, bf16),
    python/clarus/models/fftformer/__init__.py:160-161. F = 2 M K N (GEMM) + (M / 64) N 20720
    (the dense DFT-GEMM flops of config 3 per patch-channel); B = 2 M K (in) + 2 M N (out) +
    2 K N (weights) + 4 N (bias) + 4 * 80 N (filter gains)."""
    g = _gen(seed + 11)
    h, w, k, n = 720, 1280, 48, 288
    m = h * w
    x = torch.randn(1, h, w, k, generator=g).bfloat16()
    wk = _kaiming_uniform_kn(g, k, n).bfloat16()
    b = torch.rand(n, generator=g) * 0.2 - 0.1
    f = torch.randn(n, 8, 5, generator=g)
    host = dict(x=x, w=wk, b=b, f=f)
    d = {nm: t.to(device) for nm, t in host.items()}

    def run(r=None, d=d):
        return (r or hip).linear_patch_filter(d["x"], d["w"], d["b"], d["f"], ln=True, ln_eps=1e-5)
    flops = 2.0 * m * k * n + (m / 64.0) * n * 20720.0
    nbytes = 2.0 * m * k + 2.0 * m * n + 2.0 * k * n + 4.0 * n + 4.0 * 80 * n
    return OpCase("fftformer L0 DFFN LN -> 48->288 -> patch filter (fused)", 3, "bf16", flops, nbytes, run, host,
                  lambda r: run(r, host))


def evssm_scan_case(hip, device, seed: int = 0) -> OpCase:
    """EVSSM level-0 selective scan at 720p: 8 crops of 384 x 384 (L = 147456), 96 channels,
    r = 3, d_state 8, bf16 u (python/clarus/models/evssm/__init__.py:152). Per (step, channel):
    F = 2 r (dt projection) + 4 (softplus) + 8 * 6 (state update) + 2 * 8 + 2 (output) flops,
    plus 8 exp2; B = 2 (u) + 4 (y) bytes per (step, channel) + 4 (r + 16) per step (dbl). The
    CPU sample is one of the 8 crops."""
    g = _gen(seed + 13)
    t, h, w, d, r = 8, 384, 384, 96, 3
    L = h * w
    u = torch.randn(t, h, w, d, generator=g).bfloat16()
    dbl = torch.randn(t, h, w, r + 16, generator=g)
    dtw = torch.randn(d, r, generator=g) * 0.5
    dtb = torch.randn(d, generator=g) - 2
    dsk = torch.randn(d, generator=g)
    A = -torch.rand(d, 8, generator=g) * 4 - 0.5
    host = dict(u=u, dbl=dbl, dtw=dtw, dtb=dtb, A=A, dsk=dsk)
    dv = {n: v.to(device) for n, v in host.items()}
    sample = {n: (v[:1] if n in ("u", "dbl") else v) for n, v in host.items()}

    def run(be=None, a=dv):
        return (be or hip).selective_scan(a["u"], a["dbl"], a["dtw"], a["dtb"], a["A"], a["dsk"])
    flops = t * L * d * (2.0 * r + 4 + 8 * 6 + 2 * 8 + 2)
    nbytes = t * L * d * (2.0 + 4.0) + t * L * (r + 16) * 4.0
    return OpCase("evssm L0 selective scan 8 x 384x384 d96", 0, "fp32", flops, nbytes, run, host,
                  lambda be: run(be, sample), cpu_scale=float(t), cpu_sample="one of the 8 crops, times 8")


def metrics_case(device, seed: int = 0) -> OpCase:
    """PSNR + SSIM of a 720p uint8 pair (the evaluation loop's per-image metrics). F: per
    pixel-channel ~11 * 30 (channel mix + horizontal taps of 5 moments) + 11 * 10 (vertical) + 20
    (SSIM map) fp64 flops and 3 (squared difference); B = 2 * 3 bytes per pixel."""
    from .metrics import make_metrics
    g = _gen(seed + 17)
    h, w = 720, 1280
    gt = torch.randint(0, 256, (h, w, 3), generator=g, dtype=torch.uint8)
    pred = (gt.float() * 0.9 + 12 + 6 * torch.randn(h, w, 3, generator=g)).round().clamp(0, 255).to(torch.uint8)
    m = make_metrics(device, "hip")
    a, b = pred.to(device), gt.to(device)
    res = torch.zeros(2, dtype=torch.float64, device=device)
    sc = m.scratch(h, w)

    def run():
        m.compute(a, b, res, sc)
        return res
    n = h * w * 3
    return OpCase("psnr + ssim 720p (uint8, fp64 moments)", 0, "fp64", n * (11 * 30 + 11 * 10 + 20 + 3), 2.0 * n, run,
                  {"pred": pred, "gt": gt}, lambda be: be.metrics(pred.numpy(), gt.numpy()))


def all_cases(hip_bf16, hip32, device, seed: int = 0) -> list[OpCase]:
    """Every benchmark op, in the order of bench.py's rows: the config-2 step, configs 1, 3, 4, 5,
    the fused FFTformer DFFN op, the fused NAFNet pair, feed-forward half and first half, the NAFNet
    depthwise conv at levels 3 and 0, EVSSM's scan and the metrics."""
    return (config2_cases(hip_bf16, device, seed) + config1_cases(hip32, device, seed)
            + config3_cases(hip32, device, seed) + config4_cases(hip_bf16, hip32, device, seed)
            + config5_cases(hip_bf16, device, seed) + [fftformer_dffn_case(hip_bf16, device, seed),
                                                        nafnet_pair_case(hip_bf16, device, seed),
                                                        nafnet_ffn_case(hip_bf16, device, seed),
                                                        nafnet_lndw_case(hip_bf16, device, seed),
                                                        nafnet_dw_case(hip_bf16, device, 3, seed),
                                                        nafnet_dw_case(hip_bf16, device, 0, seed),
                                                        evssm_scan_case(hip_bf16, device, seed), metrics_case(device, seed)])
