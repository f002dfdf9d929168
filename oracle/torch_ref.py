"""TEST ORACLE: the reference PyTorch backend's semantics for the GEMM-family ops, in fp32.

Restated from python/clarus/ops/torch_ref.py (cited per method). Math runs in fp32 on the
device of the inputs (the CPU in tests and in bench.py's cpu_baseline) and is cast to the
output dtype at the end of each op, exactly where the reference casts. Only tests/, smoke()
and bench.py's cpu_baseline may use this module.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class Small:
    """TLC local-mean map (torch_ref.py:18-33): data [N, oh, ow, C]; full-resolution value at
    (y, x) = data[clamp(y - pt, 0, oh - 1), clamp(x - pl, 0, ow - 1)]."""

    data: torch.Tensor
    pt: int
    pl: int
    H: int
    W: int

    def with_data(self, data):
        return Small(data, self.pt, self.pl, self.H, self.W)


def box_geometry(h: int, w: int, k):
    """torch_ref.py:36-41: (k1, k2, oh, ow, pt, pl) of a (kh, kw) valid local mean."""
    kh, kw = (k, k) if isinstance(k, int) else k
    k1, k2 = min(h, kh), min(w, kw)
    oh, ow = h - k1 + 1, w - k2 + 1
    return k1, k2, oh, ow, (h - oh) // 2, (w - ow) // 2


def _is_small(x) -> bool:
    return not torch.is_tensor(x) and hasattr(x, "data") and hasattr(x, "pt")


def _to_nchw(x):
    return x.permute(0, 3, 1, 2)


def _to_nhwc(x):
    return x.permute(0, 2, 3, 1).contiguous()


class TorchRef:
    """The reference backend's op semantics; `dtype` is the activation dtype."""

    name = "oracle"

    def __init__(self, dtype: torch.dtype = torch.float32, device="cpu"):
        self.dtype = dtype
        self.device = torch.device(device)

    # ---------------------------------------------------------------- helpers
    @staticmethod
    def expand(s) -> torch.Tensor:
        """torch_ref.py:85-91: replicate-pad the local-mean map to full resolution."""
        oh, ow = s.data.shape[1], s.data.shape[2]
        rows = torch.clamp(torch.arange(s.H, device=s.data.device) - s.pt, 0, oh - 1)
        cols = torch.clamp(torch.arange(s.W, device=s.data.device) - s.pl, 0, ow - 1)
        return s.data[:, rows][:, :, cols]

    @staticmethod
    def ln(x, eps=1e-6, rms=False):
        """torch_ref.py:93-100: two-pass LayerNorm (no affine) or RMS norm over the last dim."""
        x = x.float()
        if rms:
            return x * torch.rsqrt(x.square().mean(-1, keepdim=True) + eps)
        centred = x - x.mean(-1, keepdim=True)
        return centred * torch.rsqrt(centred.square().mean(-1, keepdim=True) + eps)

    def _odt(self, out_dtype):
        return out_dtype or self.dtype

    # ---------------------------------------------------------------- GEMM family
    def linear(self, x, w, bias=None, ln=False, act=None, gate=False, scale=None,
               residual=None, mul=None, out_dtype=None, ln_eps=1e-6):
        """torch_ref.py:103-131. Order: (* expand(mul)) -> LN -> @ w -> + bias -> gate -> GELU
        -> * scale -> + residual -> cast."""
        if _is_small(x):
            return x.with_data(self.linear(x.data, w, bias, ln, act, gate, scale, residual, mul, out_dtype, ln_eps))
        a = x.float()
        if mul is not None:
            a = a * self.expand(mul).float()
        if ln:
            a = self.ln(a, ln_eps, rms=(ln == "rms"))
        y = a @ w.float()
        if bias is not None:
            y = y + bias
        if gate:
            half = y.shape[-1] // 2
            y = y[..., :half] * y[..., half:]
        if act == "gelu":
            y = F.gelu(y)
        if scale is not None:
            y = y * scale
        if residual is not None:
            y = residual.float() + y
        return y.to(self._odt(out_dtype))

    def intro(self, inp, w, b, out_dtype=None):
        """torch_ref.py:157-158: 3x3 conv (pad 1) of the NCHW image -> NHWC."""
        return _to_nhwc(F.conv2d(inp.float(), w.float(), b, padding=1)).to(self._odt(out_dtype))

    def down(self, x, w4d, b, out_dtype=None):
        """torch_ref.py:160-161: 2x2 stride-2 conv."""
        return _to_nhwc(F.conv2d(_to_nchw(x).float(), w4d.float(), b, stride=2)).to(self._odt(out_dtype))

    def up(self, x, w, residual=None, out_dtype=None):
        """torch_ref.py:163-171: 1x1 conv to 4C' (N ordered (dy, dx, c')) + PixelShuffle(2)."""
        n, h, wd, _ = x.shape
        y = x.float() @ w.float()
        cq = y.shape[-1] // 4
        y = y.reshape(n, h, wd, 2, 2, cq).permute(0, 1, 3, 2, 4, 5).reshape(n, 2 * h, 2 * wd, cq)
        if residual is not None:
            y = y + residual.float()
        return y.to(self._odt(out_dtype))

    def ending(self, x, w, b, inp):
        """torch_ref.py:173-175: final 3x3 conv + global residual -> fp32 NCHW."""
        return F.conv2d(_to_nchw(x).float(), w.float(), b, padding=1) + inp

    def conv3x3(self, x, w, b=None, out_dtype=None, act=None, residual=None, out_scale=1.0, up2=False,
                out=None, slope=0.2):
        """torch_ref.py:178-199: y = act(conv3x3(up2?(x)) + b) * out_scale (+ residual)."""
        xi = _to_nchw(x).float()
        if up2:
            xi = F.interpolate(xi, scale_factor=2, mode="nearest")
        y = F.conv2d(xi, w.float(), b, padding=1).permute(0, 2, 3, 1)
        if act == "lrelu":
            y = F.leaky_relu(y, slope)
        if out_scale != 1.0:
            y = y * out_scale
        if residual is not None:
            y = y + residual.float()
        if out is not None:
            out.copy_(y)
            return out
        return y.contiguous().to(self._odt(out_dtype))

    def channel_attention(self, qkv, heads, temperature):
        """torch_ref.py:220-235: softmax((q/|q|)(k/|k|)^T * t) per image and head, fp32."""
        n, h, w, c3 = qkv.shape
        c = c3 // 3
        ch = c // heads
        q = qkv[..., :c].reshape(n, h * w, heads, ch).float().permute(0, 2, 3, 1)      # [n, hd, ch, P]
        k = qkv[..., c:2 * c].reshape(n, h * w, heads, ch).float().permute(0, 2, 1, 3)  # [n, hd, P, ch]
        g = torch.matmul(q, k)
        nq = q.square().sum(-1).clamp_min(1e-24).rsqrt()
        nk = k.square().sum(-2).clamp_min(1e-24).rsqrt()
        g = g * nq[..., :, None] * nk[..., None, :] * temperature.reshape(1, heads, 1, 1).float()
        return torch.softmax(g, dim=-1)

    def linear_per_image(self, x, w, residual=None, out_dtype=None, bias=None):
        """torch_ref.py:237-245: per image x[i] @ w[i] (+ bias, + residual)."""
        n, h, wd, k = x.shape
        y = torch.bmm(x.reshape(n, h * wd, k).float(), w.float()).reshape(n, h, wd, -1)
        if bias is not None:
            y = y + bias
        if residual is not None:
            y = y + residual.float()
        return y.to(self._odt(out_dtype))

    def patch_filter(self, x, f, residual=None, out_dtype=None):
        """torch_ref.py:253-270: per p x p patch and channel irfft2(rfft2(patch) * f[c]),
        reflect-padding sizes that are not multiples of p (result cropped)."""
        n, h, w, c = x.shape
        p = f.shape[1]
        xi = _to_nchw(x).float()
        ph, pw = (-h) % p, (-w) % p
        if ph or pw:
            xi = F.pad(xi, (0, pw, 0, ph), mode="reflect")
        hh, ww = h + ph, w + pw
        patches = xi.reshape(n, c, hh // p, p, ww // p, p).permute(0, 1, 2, 4, 3, 5)
        spec = torch.fft.rfft2(patches) * f.float().reshape(1, c, 1, 1, p, p // 2 + 1)
        y = torch.fft.irfft2(spec, s=(p, p))
        y = y.permute(0, 2, 4, 3, 5, 1).reshape(n, hh, ww, c)[:, :h, :w]
        if residual is not None:
            y = y + residual.float()
        return y.contiguous().to(self._odt(out_dtype))

    def linear_patch_filter(self, x, w, bias, f, ln=False, ln_eps=1e-6, residual=None):
        """torch_ref.py:272-276: patch_filter(linear(x, w, bias, ln) kept fp32, f, residual)."""
        y = self.linear(x, w, bias, ln=ln, ln_eps=ln_eps, out_dtype=torch.float32)
        return self.patch_filter(y, f, residual=residual)

    def patch_corr(self, x, c, p=8):
        """torch_ref.py:278-288: per patch irfft2(rfft2(q) * rfft2(k)) -> fp32 [N, H, W, c]."""
        n, h, w, _ = x.shape

        def patches(t):
            return _to_nchw(t).float().reshape(n, c, h // p, p, w // p, p).permute(0, 1, 2, 4, 3, 5)
        spec = torch.fft.rfft2(patches(x[..., :c])) * torch.fft.rfft2(patches(x[..., c:2 * c]))
        y = torch.fft.irfft2(spec, s=(p, p))
        return y.permute(0, 2, 4, 3, 5, 1).reshape(n, h, w, c).contiguous()

    def ln_mul_linear(self, x, ln_w, ln_b, m, w, bias=None, m_act=None, residual=None, ln_eps=1e-5,
                      out_dtype=None):
        """torch_ref.py:290-302: ((LN(x) * ln_w + ln_b) * act(m)) @ w (+ bias, + residual)."""
        a = self.ln(x, ln_eps) * ln_w + ln_b
        mm = m.float()
        a = a * (F.gelu(mm) if m_act == "gelu" else mm)
        y = a @ w.float()
        if bias is not None:
            y = y + bias
        if residual is not None:
            y = y + residual.float()
        return y.to(self._odt(out_dtype))

    # ---------------------------------------------------------------- non-GEMM ops of the harnesses
    def boxmean(self, x, k):
        """torch_ref.py:133-141: valid local mean via a 2-D prefix sum (TLC)."""
        n, h, w, c = x.shape
        k1, k2, oh, ow, pt, pl = box_geometry(h, w, k)
        s = F.pad(x.float().cumsum(dim=2).cumsum(dim=1), (0, 0, 1, 0, 1, 0))
        win = s[:, k1:, k2:] + s[:, :-k1, :-k2] - s[:, :-k1, k2:] - s[:, k1:, :-k2]
        return Small((win / (k1 * k2)).to(self.dtype), pt, pl, h, w)

    def dwconv(self, x, w, b, dil=1, gate=False, act=None):
        """torch_ref.py:143-155: depthwise conv ('same'), optional gate / GELU."""
        kh, kw = w.shape[-2:]
        y = F.conv2d(_to_nchw(x).float(), w.float(), b, padding=(dil * (kh // 2), dil * (kw // 2)),
                     dilation=dil, groups=x.shape[-1]).permute(0, 2, 3, 1)
        if gate:
            half = y.shape[-1] // 2
            first = F.gelu(y[..., :half]) if gate == "gelu" else y[..., :half]
            y = first * y[..., half:]
        if act == "gelu":
            y = F.gelu(y)
        return y.contiguous().to(self.dtype)

    def selective_scan(self, u, dbl, dt_w, dt_bias, A, D, chunk=32):
        """torch_ref.py:312-341: Mamba selective scan along each crop's raster sequence, computed
        chunk by chunk in closed form: within a chunk, h_l = exp(S_l) h_in + sum_{s <= l}
        exp(S_l - S_s) delta_s B_s u_s with S the running sum of delta A; y_l = C_l . h_l + D u_l.
        delta = softplus(dt_raw @ dt_w^T + dt_bias); dbl = (dt_raw | B | C). Returns fp32."""
        t, hh, ww, d = u.shape
        L, r, ns = hh * ww, dt_w.shape[1], A.shape[1]
        u = u.reshape(t, L, d).float()
        dbl = dbl.reshape(t, L, -1).float()
        delta = F.softplus(dbl[..., :r] @ dt_w.float().t() + dt_bias.float())
        bm, cm = dbl[..., r:r + ns], dbl[..., r + ns:r + 2 * ns]
        a = A.float()
        state = torch.zeros(t, d, ns, device=u.device)
        out = []
        for s0 in range(0, L, chunk):
            dl, uc = delta[:, s0:s0 + chunk], u[:, s0:s0 + chunk]
            c = dl.shape[1]
            run = (dl[..., None] * a).cumsum(1)                                 # [t, c, d, n]
            inj = (dl * uc)[..., None] * bm[:, s0:s0 + c, None, :]            # [t, c, d, n]
            gap = run[:, :, None] - run[:, None, :]                            # [t, l, s, d, n]
            low = torch.ones(c, c, dtype=torch.bool, device=u.device).tril()
            decay = torch.where(low[None, :, :, None, None], gap, float("-inf")).exp()
            hs = run.exp() * state[:, None] + torch.einsum("tlsdn,tsdn->tldn", decay, inj)
            out.append(torch.einsum("tldn,tln->tld", hs, cm[:, s0:s0 + c]))
            state = hs[:, -1]
        y = torch.cat(out, 1) + u * D.float()
        return y.view(t, hh, ww, d)
