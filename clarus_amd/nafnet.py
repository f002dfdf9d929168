"""NAFNet / NAFNetLocal forward over the op dispatch: the harness of the end-to-end NAFNet
benchmark and parity test.

Restates the caller side of the hot path from the reference model adapter
(python/clarus/models/nafnet/__init__.py:98-185) and its weight folding
(python/clarus/models/_fold.py:127-136): LayerNorm affine folded into conv1 / conv4, 1x1
weights as [K, N], the up conv's N reordered to (dy, dx, c'), beta / gamma kept as fp32
epilogue scales, TLC local-mean windows per level. Weights are seeded random values in the
upstream state-dict layout (no checkpoints are available offline); beta / gamma are random too,
since upstream zero-init would hide epilogue bugs.

    model = NAFNet(ops, width=64, enc=[1, 1, 1, 28], mid=1, dec=[1, 1, 1, 1])   # GoPro-w64
    y = model.forward(x)          # x [N, 3, H, W] fp32 in [0, 1] -> [N, 3, H, W] fp32
"""
from __future__ import annotations

import statistics
import time

import torch
import torch.nn.functional as F


def state_dict_shapes(width, enc, mid, dec, img_channel=3) -> dict:
    """{key: shape} of the upstream NAFNet(img_channel, width, mid, enc, dec) state dict."""
    def block(p, c):
        return {f"{p}.conv1.weight": (2 * c, c, 1, 1), f"{p}.conv1.bias": (2 * c,),
                f"{p}.conv2.weight": (2 * c, 1, 3, 3), f"{p}.conv2.bias": (2 * c,),
                f"{p}.conv3.weight": (c, c, 1, 1), f"{p}.conv3.bias": (c,),
                f"{p}.sca.1.weight": (c, c, 1, 1), f"{p}.sca.1.bias": (c,),
                f"{p}.conv4.weight": (2 * c, c, 1, 1), f"{p}.conv4.bias": (2 * c,),
                f"{p}.conv5.weight": (c, c, 1, 1), f"{p}.conv5.bias": (c,),
                f"{p}.norm1.weight": (c,), f"{p}.norm1.bias": (c,), f"{p}.norm2.weight": (c,),
                f"{p}.norm2.bias": (c,), f"{p}.beta": (1, c, 1, 1), f"{p}.gamma": (1, c, 1, 1)}
    s = {"intro.weight": (width, img_channel, 3, 3), "intro.bias": (width,),
         "ending.weight": (img_channel, width, 3, 3), "ending.bias": (img_channel,)}
    c = width
    for i, n in enumerate(enc):
        for j in range(n):
            s.update(block(f"encoders.{i}.{j}", c))
        s[f"downs.{i}.weight"], s[f"downs.{i}.bias"] = (2 * c, c, 2, 2), (2 * c,)
        c *= 2
    for j in range(mid):
        s.update(block(f"middle_blks.{j}", c))
    for i, n in enumerate(dec):
        s[f"ups.{i}.0.weight"] = (2 * c, c, 1, 1)
        c //= 2
        for j in range(n):
            s.update(block(f"decoders.{i}.{j}", c))
    return s


def random_state_dict(width, enc, mid, dec, seed=0) -> dict:
    """Seeded random weights: conv weights U(-1/sqrt(fan_in), 1/sqrt(fan_in)) (nn.Conv2d's
    default bound), biases likewise, LayerNorm weight 1 + 0.1 N(0, 1) and bias 0.1 N(0, 1),
    beta / gamma 0.2 N(0, 1); the final conv is scaled by 0.1 so that the restored image stays
    near the input (unsaturated outputs)."""
    g = torch.Generator().manual_seed(seed)
    sd = {}
    for k, shape in state_dict_shapes(width, enc, mid, dec).items():
        if k.endswith(("beta", "gamma")):
            v = 0.2 * torch.randn(shape, generator=g)
        elif ".norm" in k:
            v = (1.0 if k.endswith("weight") else 0.0) + 0.1 * torch.randn(shape, generator=g)
        else:
            w_shape = shape if len(shape) == 4 else None
            fan_in = (w_shape[1] * w_shape[2] * w_shape[3]) if w_shape else None
            if fan_in is None:  # bias: use the matching weight's fan-in
                ws = state_dict_shapes(width, enc, mid, dec)[k[:-len("bias")] + "weight"]
                fan_in = ws[1] * ws[2] * ws[3]
            v = (torch.rand(shape, generator=g) * 2 - 1) / fan_in ** 0.5
            if k.startswith("ending."):
                v = v * 0.1
        sd[k] = v.float()
    return sd


def _ln_fold(w, b, ln_w, ln_b):
    """1x1 conv [N, K, 1, 1] after a LayerNorm affine -> ([K, N], bias [N])."""
    w = w.flatten(1)
    return (w * ln_w[None, :]).t().contiguous(), w @ ln_b + b


def _kn(w):
    return w.reshape(w.shape[0], -1).t().contiguous()


class NAFNet:
    """NAFNetLocal (TLC, train_size 256) or plain NAFNet over an `Ops` dispatcher."""

    def __init__(self, ops, width=64, enc=(1, 1, 1, 28), mid=1, dec=(1, 1, 1, 1), tlc=(256, 256),
                 res_fp32_level=3, seed=0, state_dict=None, fused_pairs=True):
        self.ops = ops
        # True: blocks of width pair_width send each residual GEMM and the LayerNorm GEMM on its
        # output to ops.linear_ln_linear (conv3 -> conv4, and conv5 -> the next block's conv1
        # within a stage), blocks of other widths their feed-forward half (conv4 -> SimpleGate ->
        # conv5) to ops.linear_gate_linear, and a conv1 not computed by such a pair goes with the
        # depthwise conv after it to ops.linear_dwconv; a backend may run each as one kernel.
        # False: the reference block's five linear calls (models/nafnet/__init__.py:152-161)
        self.fused_pairs = fused_pairs
        self.pair_width = 512
        self.dtype = ops.dtype
        self.device = ops.device
        self.width, self.enc, self.mid, self.dec = width, list(enc), mid, list(dec)
        self.padder = 2 ** len(self.enc)
        self.tlc = tlc
        self.res_fp32_level = res_fp32_level
        sd = state_dict if state_dict is not None else random_state_dict(width, self.enc, mid, self.dec, seed)
        self.w = self._fold(sd)

    # ------------------------------------------------------------------ weights
    def _put(self, out, name, v, fp32=False):
        out[name] = v.to(device=self.device, dtype=torch.float32 if fp32 else self.dtype).contiguous()

    def _fold_block(self, out, sd, src, dst):
        w, b = _ln_fold(sd[f"{src}.conv1.weight"], sd[f"{src}.conv1.bias"], sd[f"{src}.norm1.weight"],
                        sd[f"{src}.norm1.bias"])
        self._put(out, f"{dst}.conv1.w", w)
        self._put(out, f"{dst}.conv1.bias", b, True)
        self._put(out, f"{dst}.dw.w", sd[f"{src}.conv2.weight"])
        self._put(out, f"{dst}.dw.bias", sd[f"{src}.conv2.bias"], True)
        self._put(out, f"{dst}.sca.w", _kn(sd[f"{src}.sca.1.weight"]))
        self._put(out, f"{dst}.sca.bias", sd[f"{src}.sca.1.bias"], True)
        self._put(out, f"{dst}.conv3.w", _kn(sd[f"{src}.conv3.weight"]))
        self._put(out, f"{dst}.conv3.bias", sd[f"{src}.conv3.bias"], True)
        self._put(out, f"{dst}.conv3.scale", sd[f"{src}.beta"].flatten(), True)
        w, b = _ln_fold(sd[f"{src}.conv4.weight"], sd[f"{src}.conv4.bias"], sd[f"{src}.norm2.weight"],
                        sd[f"{src}.norm2.bias"])
        self._put(out, f"{dst}.conv4.w", w)
        self._put(out, f"{dst}.conv4.bias", b, True)
        self._put(out, f"{dst}.conv5.w", _kn(sd[f"{src}.conv5.weight"]))
        self._put(out, f"{dst}.conv5.bias", sd[f"{src}.conv5.bias"], True)
        self._put(out, f"{dst}.conv5.scale", sd[f"{src}.gamma"].flatten(), True)

    def _fold(self, sd):
        out: dict = {}
        self._put(out, "intro.w", sd["intro.weight"], True)
        self._put(out, "intro.bias", sd["intro.bias"], True)
        self._put(out, "ending.w", sd["ending.weight"])
        self._put(out, "ending.bias", sd["ending.bias"], True)
        for i, n in enumerate(self.enc):
            for j in range(n):
                self._fold_block(out, sd, f"encoders.{i}.{j}", f"enc{i}.{j}")
            self._put(out, f"down{i}.w", sd[f"downs.{i}.weight"])
            self._put(out, f"down{i}.bias", sd[f"downs.{i}.bias"], True)
        for j in range(self.mid):
            self._fold_block(out, sd, f"middle_blks.{j}", f"mid.{j}")
        for i, n in enumerate(self.dec):
            w = sd[f"ups.{i}.0.weight"].flatten(1)  # [4C', C]; rows run over (c', dy, dx), dx fastest
            cq = w.shape[0] // 4
            self._put(out, f"up{i}.w", w.view(cq, 2, 2, -1).permute(1, 2, 0, 3).reshape(4 * cq, -1).t())
            for j in range(n):
                self._fold_block(out, sd, f"decoders.{i}.{j}", f"dec{i}.{j}")
        return out

    # ------------------------------------------------------------------ forward
    def _rdt(self, level):
        return torch.float32 if level >= self.res_fp32_level else self.dtype

    def tlc_kernel(self, level):
        """(kh, kw) of the local mean replacing the global average pool at this level: feature
        size of the train image zero-padded to the multiple `padder`, times
        int(1.5 * train) // train (models/nafnet/__init__.py:142-150)."""
        if self.tlc is None:
            return (1 << 30, 1 << 30)
        return tuple(((t + self.padder - 1) // self.padder * self.padder >> level) * int(t * 1.5) // t
                     for t in self.tlc)

    def _block_reference(self, x, p, level):
        """One NAFBlock as the reference model calls it: five linear ops, a depthwise conv and the
        box mean (models/nafnet/__init__.py:152-161)."""
        o, w = self.ops, self.w
        t = o.linear(x, w[f"{p}.conv1.w"], w[f"{p}.conv1.bias"], ln=True)
        t = o.dwconv(t, w[f"{p}.dw.w"], w[f"{p}.dw.bias"], gate=True)
        sca = o.linear(o.boxmean(t, self.tlc_kernel(level)), w[f"{p}.sca.w"], w[f"{p}.sca.bias"])
        y = o.linear(t, w[f"{p}.conv3.w"], w[f"{p}.conv3.bias"], scale=w[f"{p}.conv3.scale"], residual=x,
                     mul=sca, out_dtype=self._rdt(level))
        u = o.linear(y, w[f"{p}.conv4.w"], w[f"{p}.conv4.bias"], ln=True, gate=True)
        return o.linear(u, w[f"{p}.conv5.w"], w[f"{p}.conv5.bias"], scale=w[f"{p}.conv5.scale"], residual=y,
                        out_dtype=self._rdt(level))

    def _pair(self, x, w, bias=None, scale=None, residual=None, mul=None, out_dtype=None, w2=None, bias2=None,
              gate2=False, ln=True):
        """ops.linear_ln_linear, or its two linear calls when no backend in the chain has the op."""
        o = self.ops
        try:
            fn = o.linear_ln_linear
        except AttributeError:
            fn = None
        if fn is None:
            y = o.linear(x, w, bias, scale=scale, residual=residual, mul=mul, out_dtype=out_dtype)
            return y, o.linear(y, w2, bias2, ln=ln, gate=gate2)
        return fn(x, w, bias, scale=scale, residual=residual, mul=mul, out_dtype=out_dtype, w2=w2, bias2=bias2,
                  gate2=gate2, ln=ln)

    def _ffn(self, y, p, level):
        """ops.linear_gate_linear on the block's running sum y (conv4 with LayerNorm and SimpleGate,
        then conv5 scaled by gamma on y), or its two linear calls when no backend has the op."""
        o, w = self.ops, self.w
        w4, b4, w5, b5 = w[f"{p}.conv4.w"], w[f"{p}.conv4.bias"], w[f"{p}.conv5.w"], w[f"{p}.conv5.bias"]
        try:
            fn = o.linear_gate_linear
        except AttributeError:
            fn = None
        if fn is None:
            u = o.linear(y, w4, b4, ln=True, gate=True)
            return o.linear(u, w5, b5, scale=w[f"{p}.conv5.scale"], residual=y, out_dtype=self._rdt(level))
        return fn(y, w4, b4, w5, b5, scale=w[f"{p}.conv5.scale"], ln=True, out_dtype=self._rdt(level))

    def _conv1_dw(self, x, p):
        """ops.linear_dwconv on the block input (conv1 with LayerNorm, then the depthwise conv with
        SimpleGate), or its two calls when no backend has the op."""
        o, w = self.ops, self.w
        args = (w[f"{p}.conv1.w"], w[f"{p}.conv1.bias"], w[f"{p}.dw.w"], w[f"{p}.dw.bias"])
        try:
            fn = o.linear_dwconv
        except AttributeError:
            fn = None
        if fn is None:
            return o.dwconv(o.linear(x, args[0], args[1], ln=True), args[2], args[3], gate=True)
        return fn(x, *args, ln=True, gate=True)

    def _block(self, x, p, level, t=None, nxt=None):
        """One NAFBlock on x. t: its conv1 output when the previous block's fused op already
        computed it. nxt: the next block's key at the same width, whose conv1 (LayerNorm of this
        block's output) is then computed with this block's conv5 as one op. Returns (z, the next
        block's conv1 output or None)."""
        o, w = self.ops, self.w
        if t is None:
            t = self._conv1_dw(x, p)
        else:
            t = o.dwconv(t, w[f"{p}.dw.w"], w[f"{p}.dw.bias"], gate=True)
        sca = o.linear(o.boxmean(t, self.tlc_kernel(level)), w[f"{p}.sca.w"], w[f"{p}.sca.bias"])
        if x.shape[-1] != self.pair_width:
            y = o.linear(t, w[f"{p}.conv3.w"], w[f"{p}.conv3.bias"], scale=w[f"{p}.conv3.scale"], residual=x,
                         mul=sca, out_dtype=self._rdt(level))
            return self._ffn(y, p, level), None
        # conv3 (+ residual) and conv4 (LayerNorm of its output, SimpleGate) as one op, which a
        # backend may run as one kernel
        y, u = self._pair(t, w[f"{p}.conv3.w"], w[f"{p}.conv3.bias"], scale=w[f"{p}.conv3.scale"], residual=x,
                          mul=sca, out_dtype=self._rdt(level), w2=w[f"{p}.conv4.w"], bias2=w[f"{p}.conv4.bias"],
                          gate2=True, ln=True)
        if nxt is None:
            return o.linear(u, w[f"{p}.conv5.w"], w[f"{p}.conv5.bias"], scale=w[f"{p}.conv5.scale"], residual=y,
                            out_dtype=self._rdt(level)), None
        return self._pair(u, w[f"{p}.conv5.w"], w[f"{p}.conv5.bias"], scale=w[f"{p}.conv5.scale"], residual=y,
                          out_dtype=self._rdt(level), w2=w[f"{nxt}.conv1.w"], bias2=w[f"{nxt}.conv1.bias"],
                          gate2=False, ln=True)

    def _stage(self, x, prefix, nb, level):
        """nb consecutive blocks {prefix}.0 .. {prefix}.{nb - 1} at one width."""
        if not self.fused_pairs:
            for j in range(nb):
                x = self._block_reference(x, f"{prefix}.{j}", level)
            return x
        t = None
        for j in range(nb):
            x, t = self._block(x, f"{prefix}.{j}", level, t, f"{prefix}.{j + 1}" if j + 1 < nb else None)
        return x

    @torch.no_grad()
    def forward(self, inp):
        o, w = self.ops, self.w
        n, _, h, wd = inp.shape
        ph, pw = (-h) % self.padder, (-wd) % self.padder
        if ph or pw:
            inp = F.pad(inp, (0, pw, 0, ph))
        x = o.intro(inp, w["intro.w"], w["intro.bias"], out_dtype=self._rdt(0))
        skips = []
        for i, nb in enumerate(self.enc):
            x = self._stage(x, f"enc{i}", nb, i)
            skips.append(x)
            x = o.down(x, w[f"down{i}.w"], w[f"down{i}.bias"], out_dtype=self._rdt(i + 1))
        x = self._stage(x, "mid", self.mid, len(self.enc))
        for i, nb in enumerate(self.dec):
            level = len(self.enc) - 1 - i
            x = o.up(x, w[f"up{i}.w"], residual=skips[level], out_dtype=self._rdt(level))
            x = self._stage(x, f"dec{i}", nb, level)
        out = o.ending(x, w["ending.w"], w["ending.bias"], inp)
        return out[:, :, :h, :wd]


def psnr(pred: torch.Tensor, gt: torch.Tensor, peak: float = 1.0) -> float:
    """PSNR in dB with float64 MSE (basicsr's rule, python/clarus/metrics.py:46-56)."""
    mse = torch.mean((pred.double() - gt.double()) ** 2).item()
    return float("inf") if mse == 0 else 10.0 * torch.log10(torch.tensor(peak * peak / mse)).item()


def bench_forward(dev, reps: int = 20, fused_pairs: bool = True, log=print) -> dict:
    """NAFNet-GoPro-w64 (NAFNetLocal, enc [1, 1, 1, 28], mid 1, dec [1, 1, 1, 1]) 720p bf16
    forward: GEMM-family ops, depthwise conv and TLC box mean on `hip`, pixel (un)shuffle and
    elementwise adds on torch; captured in a HIP graph after an eager warm-up, median of `reps`
    event-timed replays. fused_pairs: the harness's fused ops (residual GEMM -> LayerNorm GEMM
    pairs, the feed-forward half; each one kernel on `hip`), or the reference block's five linear
    calls."""
    from . import spatial_torch  # noqa: F401  (registers "torch" for the non-GEMM ops)
    from .dispatch import Ops
    ops = Ops(["hip", "torch"], torch.bfloat16, dev, log=lambda *a: None)
    if "hip" not in ops.by_name:
        raise RuntimeError(f"hip backend unavailable: {ops.skipped}")
    model = NAFNet(ops, fused_pairs=fused_pairs)
    g = torch.Generator().manual_seed(1)
    x = torch.rand(1, 3, 720, 1280, generator=g).to(dev)
    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        for _ in range(2):
            model.forward(x)
    torch.cuda.synchronize()
    eager = []
    for _ in range(3):
        t0 = time.perf_counter()
        model.forward(x)
        torch.cuda.synchronize()
        eager.append((time.perf_counter() - t0) * 1e3)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y = model.forward(x)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    report = ops.report()
    served = {op: list(v) for op, v in report["ops"].items()}
    res = {"ms": round(statistics.median(times), 3), "eager_ms": round(statistics.median(eager), 3),
           "reps": reps, "input": "1x3x720x1280 fp32 U(0,1), seeded", "dtype": "bf16",
           "model": "NAFNetLocal w64 enc[1,1,1,28] mid1 dec[1,1,1,1], random init",
           "block": ("fused ops: linear_ln_linear pairs (width 512), linear_gate_linear (other widths), "
                     "linear_dwconv (width 64)" if fused_pairs else "reference block: five linear calls"),
           "served": served, "finite": bool(torch.isfinite(y).all().item())}
    log(f"[bench] NAFNet-w64 720p bf16 forward ({res['block']}): graph {res['ms']} ms, eager {res['eager_ms']} ms")
    return res
