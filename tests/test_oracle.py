"""CPU: pin the oracle (oracle/torch_ref.py) before trusting it as the parity reference.

Each oracle op is checked against an independent float64 computation written differently
(explicit loops / numpy / index maps), against the reference's own known-answer tests
(tools/test_ops_contracts.py:108-111, tools/test_kernel_contracts.py:65-96,
tools/test_model_contracts.py:149-163), against numpy.fft for the patch DFT ops, and against
closed forms (softmax rows sum to 1, the Gram of q with itself, Parseval). A deliberately
planted mistake in the oracle (a dropped term, a swapped index) fails at least one of these.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.torch_ref import Small, TorchRef, box_geometry

REF = TorchRef(torch.float32, "cpu")


def gen(seed):
    return torch.Generator().manual_seed(seed)


def rnd(g, *shape, scale=1.0):
    return torch.randn(*shape, generator=g) * scale


def close(a, b, tol=2e-6):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    err = np.abs(a - b).max() / max(np.abs(b).max(), 1e-300)
    assert err < tol, err


def gelu64(x):
    return 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))


# ------------------------------------------------------------------ linear
def linear64(x, w, bias=None, ln=False, gate=False, act=None, scale=None, residual=None, mul=None, eps=1e-6):
    a = x.double().numpy().copy()
    if mul is not None:
        s = mul.data.double().numpy()
        n, h, wd, k = a.shape
        for y in range(h):
            for xx in range(wd):
                sy = min(max(y - mul.pt, 0), s.shape[1] - 1)
                sx = min(max(xx - mul.pl, 0), s.shape[2] - 1)
                a[:, y, xx] *= s[:, sy, sx]
    if ln:
        mu = a.mean(-1, keepdims=True) if ln is True else 0.0
        d = a - mu
        a = d / np.sqrt((d * d).mean(-1, keepdims=True) + eps)
    out = np.einsum("nhwk,kj->nhwj", a, w.double().numpy())
    if bias is not None:
        out = out + bias.double().numpy()
    if gate:
        half = out.shape[-1] // 2
        out = out[..., :half] * out[..., half:]
    if act == "gelu":
        out = gelu64(out)
    if scale is not None:
        out = out * scale.double().numpy()
    if residual is not None:
        out = out + residual.double().numpy()
    return out


@pytest.mark.parametrize("ln", [False, True, "rms"])
@pytest.mark.parametrize("gate", [False, True])
def test_linear_vs_float64(ln, gate):
    g = gen(1)
    x, w = rnd(g, 2, 5, 7, 24), rnd(g, 24, 20, scale=0.2)
    b, sc, res = rnd(g, 20), rnd(g, 10 if gate else 20), rnd(g, 2, 5, 7, 10 if gate else 20)
    for act in (None, "gelu"):
        got = REF.linear(x, w, b, ln=ln, gate=gate, act=act, scale=sc, residual=res)
        close(got, linear64(x, w, b, ln=ln, gate=gate, act=act, scale=sc, residual=res))


def test_linear_mul_vs_float64():
    g = gen(2)
    n, h, w = 2, 9, 13
    k1, k2, oh, ow, pt, pl = box_geometry(h, w, (4, 5))
    s = Small(rnd(g, n, oh, ow, 16), pt, pl, h, w)
    x, wt = rnd(g, n, h, w, 16), rnd(g, 16, 12)
    close(REF.linear(x, wt, mul=s), linear64(x, wt, mul=s))
    # a Small input maps linear over the map itself
    got = REF.linear(s, wt)
    assert isinstance(got, Small) and (got.pt, got.pl) == (pt, pl)
    close(got.data, np.einsum("nhwk,kj->nhwj", s.data.double().numpy(), wt.double().numpy()))


def test_linear_known_answers():
    # tools/test_ops_contracts.py:108-111 (the reference's CPU known answer, fp16 inputs)
    y = TorchRef(torch.float16).linear(torch.full((1, 1, 1, 64), 400.0).half(), torch.full((64, 4), 200.0).half(),
                                       scale=torch.full((4,), 1e-4), out_dtype=torch.float32)
    assert torch.all(y == 512.0)
    # tools/test_kernel_contracts.py:66-70, 76-78, 92-96
    w = torch.full((16, 32), 1 / 16)
    assert torch.all(REF.linear(torch.full((1, 1, 1, 16), 256.0), w, gate=True) == 65536)
    assert torch.all(REF.linear(torch.full((1, 1, 1, 16), 2.0), w, gate=True) == 4)
    assert torch.all(REF.linear(torch.full((1, 1, 1, 16), 2.0 ** -18), torch.full((16, 16), 256.0)) == 2.0 ** -6)


def test_linear_cast_at_the_end():
    """The epilogue runs in fp32 and the cast to the activation dtype happens once, last."""
    x = torch.full((1, 1, 1, 8), 1.0)
    w = torch.full((8, 2), 1.0 / 3.0)
    y16 = TorchRef(torch.bfloat16).linear(x, w, scale=torch.full((2,), 3.0))
    y32 = REF.linear(x, w, scale=torch.full((2,), 3.0))
    assert y16.dtype == torch.bfloat16 and torch.equal(y16, y32.bfloat16())


# ------------------------------------------------------------------ down / up / convs
def test_down_vs_loops():
    g = gen(3)
    x, w4, b = rnd(g, 2, 7, 9, 6), rnd(g, 5, 6, 2, 2), rnd(g, 5)
    got = REF.down(x, w4, b)
    xs, ws, bs = x.double().numpy(), w4.double().numpy(), b.double().numpy()
    ref = np.zeros((2, 3, 4, 5))
    for yo in range(3):
        for xo in range(4):
            for dy in range(2):
                for dx in range(2):
                    ref[:, yo, xo] += xs[:, 2 * yo + dy, 2 * xo + dx] @ ws[:, :, dy, dx].T
    close(got, ref + bs)


def test_up_vs_pixel_shuffle_map():
    """N ordered (dy, dx, c'): output (2y + dy, 2x + dx, c') = x[y, x] . w[:, (dy * 2 + dx) * C' + c']."""
    g = gen(4)
    x, w, res = rnd(g, 2, 3, 4, 6), rnd(g, 6, 4 * 5), rnd(g, 2, 6, 8, 5)
    got = REF.up(x, w, residual=res)
    xs, ws = x.double().numpy(), w.double().numpy()
    ref = res.double().numpy().copy()
    for y in range(3):
        for xx in range(4):
            for dy in range(2):
                for dx in range(2):
                    q = dy * 2 + dx
                    ref[:, 2 * y + dy, 2 * xx + dx] += xs[:, y, xx] @ ws[:, q * 5:(q + 1) * 5]
    close(got, ref)


def conv3x3_64(x, w, b, up2=False):
    xs = x.double().numpy()
    if up2:
        xs = xs.repeat(2, axis=1).repeat(2, axis=2)
    n, h, wd, cin = xs.shape
    pad = np.zeros((n, h + 2, wd + 2, cin))
    pad[:, 1:-1, 1:-1] = xs
    ws = w.double().numpy()
    out = np.zeros((n, h, wd, w.shape[0]))
    for ky in range(3):
        for kx in range(3):
            out += pad[:, ky:ky + h, kx:kx + wd] @ ws[:, :, ky, kx].T
    return out + (0 if b is None else b.double().numpy())


@pytest.mark.parametrize("up2", [False, True])
def test_conv3x3_vs_float64(up2):
    g = gen(5)
    x, w, b = rnd(g, 2, 5, 6, 8), rnd(g, 7, 8, 3, 3, scale=0.3), rnd(g, 7)
    res = rnd(g, 2, 10 if up2 else 5, 12 if up2 else 6, 7)
    got = REF.conv3x3(x, w, b, act="lrelu", out_scale=0.2, residual=res, up2=up2)
    ref = conv3x3_64(x, w, b, up2)
    ref = np.where(ref >= 0, ref, 0.2 * ref) * 0.2 + res.double().numpy()
    close(got, ref)
    buf = torch.zeros(2, 5, 6, 16)
    buf[..., :8] = x
    REF.conv3x3(buf[..., :8], w, b, out=buf[..., 8:15])
    close(buf[..., 8:15], conv3x3_64(x, w, b))


def test_intro_and_ending_vs_float64():
    g = gen(6)
    img = torch.rand(2, 3, 6, 7, generator=g)
    wi, bi = rnd(g, 8, 3, 3, 3), rnd(g, 8)
    close(REF.intro(img, wi, bi), conv3x3_64(img.permute(0, 2, 3, 1), wi, bi))
    x, we, be = rnd(g, 2, 6, 7, 8), rnd(g, 3, 8, 3, 3), rnd(g, 3)
    ref = conv3x3_64(x, we, be).transpose(0, 3, 1, 2) + img.double().numpy()
    close(REF.ending(x, we, be, img), ref)


# ------------------------------------------------------------------ attention
def test_channel_attention_vs_float64():
    g = gen(7)
    n, h, w, heads, ch = 2, 5, 6, 3, 8
    qkv, t = rnd(g, n, h, w, 3 * heads * ch), torch.rand(heads, generator=g) + 0.5
    got = REF.channel_attention(qkv, heads, t).double().numpy()
    a = qkv.double().numpy().reshape(n, h * w, 3, heads, ch)
    for i in range(n):
        for hd in range(heads):
            q, k = a[i, :, 0, hd], a[i, :, 1, hd]
            qn = q / np.linalg.norm(q, axis=0)
            kn = k / np.linalg.norm(k, axis=0)
            logits = qn.T @ kn * t[hd].item()
            e = np.exp(logits - logits.max(1, keepdims=True))
            close(got[i, hd], e / e.sum(1, keepdims=True))
    assert np.allclose(got.sum(-1), 1.0, atol=1e-6)


def test_channel_attention_self_gram_closed_form():
    """q == k: the normalised Gram has a unit diagonal, so with a huge temperature the softmax
    concentrates on the diagonal for orthogonal channels."""
    ch = 4
    q = torch.zeros(1, 4, 4, ch)
    for c in range(ch):
        q[0, c, :, c] = 1.0  # orthogonal channels
    qkv = torch.cat([q, q, q], dim=-1)
    a = REF.channel_attention(qkv, 1, torch.tensor([50.0]))
    assert torch.allclose(a[0, 0], torch.eye(ch), atol=1e-6)


def test_linear_per_image_vs_float64():
    g = gen(8)
    x, w, b, res = rnd(g, 2, 3, 4, 6), rnd(g, 2, 6, 5), rnd(g, 5), rnd(g, 2, 3, 4, 5)
    ref = np.einsum("nhwk,nkj->nhwj", x.double().numpy(), w.double().numpy()) + b.double().numpy() + \
        res.double().numpy()
    close(REF.linear_per_image(x, w, residual=res, bias=b), ref)


# ------------------------------------------------------------------ patch DFT ops
def patch_filter64(x, f, residual=None):
    xs = x.double().numpy()
    n, h, w, c = xs.shape
    ph, pw = (-h) % 8, (-w) % 8
    xp = np.pad(xs, ((0, 0), (0, ph), (0, pw), (0, 0)), mode="reflect")
    out = np.zeros_like(xp)
    fs = f.double().numpy()
    for py in range(xp.shape[1] // 8):
        for px in range(xp.shape[2] // 8):
            patch = xp[:, py * 8:(py + 1) * 8, px * 8:(px + 1) * 8, :].transpose(0, 3, 1, 2)  # n c 8 8
            spec = np.fft.rfft2(patch) * fs[None]
            out[:, py * 8:(py + 1) * 8, px * 8:(px + 1) * 8, :] = np.fft.irfft2(spec, s=(8, 8)).transpose(0, 2, 3, 1)
    out = out[:, :h, :w]
    return out if residual is None else out + residual.double().numpy()


@pytest.mark.parametrize("h,w", [(16, 24), (13, 19)])
def test_patch_filter_vs_numpy_fft(h, w):
    g = gen(9)
    x, f, res = rnd(g, 2, h, w, 5), rnd(g, 5, 8, 5), rnd(g, 2, h, w, 5)
    close(REF.patch_filter(x, f, residual=res), patch_filter64(x, f, res), tol=5e-6)


def test_patch_filter_identity_and_parseval():
    """f == 1 is the identity (irfft2 o rfft2), whatever the input."""
    g = gen(10)
    x = rnd(g, 1, 16, 16, 3)
    close(REF.patch_filter(x, torch.ones(3, 8, 5)), x, tol=5e-6)


def test_patch_corr_vs_numpy_fft():
    g = gen(11)
    n, h, w, c = 2, 16, 8, 3
    x = rnd(g, n, h, w, 2 * c + 2)
    got = REF.patch_corr(x, c)
    xs = x.double().numpy()
    ref = np.zeros((n, h, w, c))
    for py in range(h // 8):
        for px in range(w // 8):
            q = xs[:, py * 8:(py + 1) * 8, px * 8:(px + 1) * 8, :c].transpose(0, 3, 1, 2)
            k = xs[:, py * 8:(py + 1) * 8, px * 8:(px + 1) * 8, c:2 * c].transpose(0, 3, 1, 2)
            y = np.fft.irfft2(np.fft.rfft2(q) * np.fft.rfft2(k), s=(8, 8))
            ref[:, py * 8:(py + 1) * 8, px * 8:(px + 1) * 8] = y.transpose(0, 2, 3, 1)
    close(got, ref, tol=5e-6)
    # circular convolution of each patch with itself: for a delta patch it is the delta at 2 * index
    d = torch.zeros(1, 8, 8, 2)
    d[0, 1, 2, :] = 1.0
    y = REF.patch_corr(d, 1)
    assert abs(y[0, 2, 4, 0].item() - 1.0) < 1e-6 and abs(y.abs().sum().item() - 1.0) < 1e-5


def test_ln_mul_linear_vs_float64():
    g = gen(12)
    x, m = rnd(g, 2, 3, 5, 16, scale=5.0) + 3, rnd(g, 2, 3, 5, 16)
    lw, lb, w, b, res = rnd(g, 16), rnd(g, 16), rnd(g, 16, 6), rnd(g, 6), rnd(g, 2, 3, 5, 6)
    xs = x.double().numpy()
    mu = xs.mean(-1, keepdims=True)
    a = (xs - mu) / np.sqrt(((xs - mu) ** 2).mean(-1, keepdims=True) + 1e-5) * lw.double().numpy() + lb.double().numpy()
    for act in (None, "gelu"):
        mm = m.double().numpy()
        a2 = a * (gelu64(mm) if act == "gelu" else mm)
        ref = a2 @ w.double().numpy() + b.double().numpy() + res.double().numpy()
        close(REF.ln_mul_linear(x, lw, lb, m, w, b, m_act=act, residual=res), ref)


# ------------------------------------------------------------------ non-GEMM helpers of the harness
def test_boxmean_vs_loops():
    g = gen(13)
    x = rnd(g, 1, 7, 9, 2)
    s = REF.boxmean(x, (3, 4))
    k1, k2, oh, ow, pt, pl = box_geometry(7, 9, (3, 4))
    xs = x.double().numpy()
    ref = np.array([[xs[0, i:i + k1, j:j + k2].mean((0, 1)) for j in range(ow)] for i in range(oh)])
    close(s.data[0], ref, tol=1e-6)
    assert (s.pt, s.pl, s.H, s.W) == (pt, pl, 7, 9)


def test_dwconv_vs_loops():
    g = gen(14)
    x, w, b = rnd(g, 1, 5, 6, 4), rnd(g, 4, 1, 3, 3), rnd(g, 4)
    got = REF.dwconv(x, w, b, gate=True)
    xs = np.pad(x.double().numpy(), ((0, 0), (1, 1), (1, 1), (0, 0)))
    ref = np.zeros((1, 5, 6, 4))
    for ky in range(3):
        for kx in range(3):
            ref += xs[:, ky:ky + 5, kx:kx + 6] * w.double().numpy()[:, 0, ky, kx]
    ref += b.double().numpy()
    close(got, ref[..., :2] * ref[..., 2:])
