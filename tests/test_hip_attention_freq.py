"""GPU parity: Restormer channel attention (split-K Gram + norms + softmax) and the FFTformer
patch-DFT ops (patch_filter, linear_patch_filter, patch_corr) vs the oracle.

Cases follow tools/test_kernels.py:200-208,237-247, tools/test_ops_contracts.py:128-141 and
BASELINE configs 3 (patch DFT at C = 48 / 96 / 192, 720p / 360p / 180p) and 4 (MDTA levels).
"""
from __future__ import annotations

import pytest
import torch

from _tol import assert_abs, assert_bf16, assert_fp32
from oracle.torch_ref import TorchRef

pytestmark = pytest.mark.gpu
REF = TorchRef(torch.float32, "cpu")


@pytest.fixture(scope="module")
def hip_bf16(gpu_device):
    from clarus_amd.hip_ops import HipOps
    return HipOps(torch.bfloat16, gpu_device)


@pytest.fixture(scope="module")
def hip_f32(gpu_device):
    from clarus_amd.hip_ops import HipOps
    return HipOps(torch.float32, gpu_device)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def rnd(g, *shape, scale=1.0, dtype=torch.float32):
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


# ------------------------------------------------------------------ channel attention
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_channel_attention_small(dt, hip_bf16, hip_f32):
    """tools/test_kernels.py:200-208 shape: n=2, 21x34, 4 heads of 48 channels."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(1)
    heads, ch = 4, 48
    qkv = rnd(g, 2, 21, 34, 3 * heads * ch, dtype=dt)
    t = torch.rand(heads, generator=g) * 1.5 + 0.5
    got = hip.channel_attention(qkv.cuda(), heads, t.cuda())
    ref = REF.channel_attention(qkv, heads, t)
    assert_fp32(got.cpu(), ref, rel=1e-5, what=f"channel_attention {dt}")
    assert torch.allclose(got.sum(-1).cpu(), torch.ones(2, heads, ch), atol=1e-5)


@pytest.mark.parametrize("ch", [8, 24, 64])
def test_channel_attention_head_widths(ch, hip_f32):
    g = gen(2)
    heads = 2
    qkv = rnd(g, 1, 17, 23, 3 * heads * ch)
    t = torch.rand(heads, generator=g) + 0.5
    assert_fp32(hip_f32.channel_attention(qkv.cuda(), heads, t.cuda()).cpu(), REF.channel_attention(qkv, heads, t),
                rel=1e-5, what=f"channel_attention ch{ch}")


def test_channel_attention_launch_slices_and_reuse(hip_f32):
    """More (image, head) pairs than one launch takes (70 images x 8 heads = 560 > 496: two
    launches on the same arrival counters), against the oracle; the same call repeated, and again
    after a larger call on the same cached workspace, bit-identical (every call leaves the counters
    zero and sums in a fixed order)."""
    g = gen(3)
    heads, ch = 8, 8
    qkv = rnd(g, 70, 6, 10, 3 * heads * ch)
    t = torch.rand(heads, generator=g) + 0.5
    print("[attention] 70 images x 8 heads, then 4 heads at 180x320", flush=True)
    a1 = hip_f32.channel_attention(qkv.cuda(), heads, t.cuda())
    assert_fp32(a1.cpu(), REF.channel_attention(qkv, heads, t), rel=1e-5, what="channel_attention 70 images")
    a2 = hip_f32.channel_attention(qkv.cuda(), heads, t.cuda())
    big = rnd(g, 1, 180, 320, 3 * 192)
    tb = torch.rand(4, generator=g) + 0.5
    b1 = hip_f32.channel_attention(big.cuda(), 4, tb.cuda())
    a3 = hip_f32.channel_attention(qkv.cuda(), heads, t.cuda())
    b2 = hip_f32.channel_attention(big.cuda(), 4, tb.cuda())
    torch.cuda.synchronize()
    assert torch.equal(a1, a2) and torch.equal(a1, a3) and torch.equal(b1, b2)
    assert_fp32(b1.cpu(), REF.channel_attention(big, 4, tb), rel=1e-5, what="channel_attention 180x320")


CONFIG4 = [(0, 720, 1280), (1, 360, 640), (2, 180, 320), (3, 90, 160)]


@pytest.mark.parametrize("lvl,h,w", CONFIG4)
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_config4_mdta(lvl, h, w, dt, hip_bf16, hip_f32):
    """BASELINE config 4 at level l: C = 48 * 2^l, heads 2^l, HW = 921600 / 4^l; Q, K, V from
    N(0, 1); temperature U(0.5, 2). Attention map, then attn . V as the per-image mix
    (blockdiag(A^T), the Restormer fold) through linear_per_image."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(40 + lvl)
    c, heads = 48 * 2 ** lvl, 2 ** lvl
    qkv = rnd(g, 1, h, w, 3 * c, dtype=dt)
    t = torch.rand(heads, generator=g) * 1.5 + 0.5
    a = hip.channel_attention(qkv.cuda(), heads, t.cuda())
    ra = REF.channel_attention(qkv, heads, t)
    assert_fp32(a.cpu(), ra, rel=1e-5 if dt == torch.float32 else 1e-4, what=f"mdta attention l{lvl} {dt}")
    bd = torch.zeros(1, c, c)
    for hh in range(heads):
        bd[:, hh * 48:(hh + 1) * 48, hh * 48:(hh + 1) * 48] = ra[:, hh].transpose(1, 2)
    got = hip.linear_per_image(qkv.cuda()[..., 2 * c:], bd.cuda(), out_dtype=torch.float32)
    assert_fp32(got.cpu(), REF.linear_per_image(qkv[..., 2 * c:], bd, out_dtype=torch.float32), rel=1e-5,
                what=f"mdta attn.V l{lvl} {dt}")


def _blockdiag(blocks):
    """The block-diagonal [N, C, C] matrix of per-head blocks [N, heads, ch, ch]."""
    n, heads, ch, _ = blocks.shape
    bd = torch.zeros(n, heads * ch, heads * ch, dtype=torch.float32)
    for hh in range(heads):
        bd[:, hh * ch:(hh + 1) * ch, hh * ch:(hh + 1) * ch] = blocks[:, hh].float()
    return bd


def _blockdiag_t(a):
    """blockdiag(A_h^T) of an attention map [N, heads, ch, ch]: the per-image matrix the
    Restormer block applies to v (python/clarus/models/restormer/__init__.py:203-208)."""
    return _blockdiag(a.transpose(-1, -2))


@pytest.mark.parametrize("lvl,h,w", CONFIG4)
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_config4_attention_apply(lvl, h, w, dt, hip_bf16, hip_f32):
    """HipOps.attention_apply (the config-4 attn . V the benchmark times: one batched GEMM launch
    per image, the heads as the batch, v read from qkv with pixel stride 3C) against the oracle's
    linear_per_image(v, blockdiag(A^T)), at every config-4 level. As in the benchmark, the maps A
    are passed in the activation dtype; fp32 output, then the backend's own."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(60 + lvl)
    c, heads = 48 * 2 ** lvl, 2 ** lvl
    qkv = rnd(g, 1, h, w, 3 * c, dtype=dt)
    logits = rnd(g, 1, heads, 48, 48, scale=2.0)
    a = torch.softmax(logits, -1)  # a row-stochastic map like channel_attention's
    am = a.to(dt)  # the maps in the activation dtype
    print(f"[attn.V] l{lvl} {dt}", flush=True)
    ref = REF.linear_per_image(qkv[..., 2 * c:], _blockdiag_t(am), out_dtype=torch.float32)
    got = hip.attention_apply(qkv.cuda(), am.cuda(), out_dtype=torch.float32)
    assert_fp32(got.cpu(), ref, rel=1e-5, what=f"attention_apply l{lvl} {dt}")
    got = hip.attention_apply(qkv.cuda(), am.cuda())
    assert got.dtype == dt
    if dt == torch.bfloat16:
        assert_bf16(got.cpu(), ref, what=f"attention_apply l{lvl} bf16 out")
    else:
        assert_fp32(got.cpu(), ref, rel=1e-5, what=f"attention_apply l{lvl} fp32 out")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_attention_apply_batch_and_residual(dt, hip_bf16, hip_f32):
    """Two images (the per-image loop), 4 heads of 24 channels, a residual and a ragged pixel
    count; attn given as [heads, ch, ch] for one image is rejected for two."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(70)
    n, h, w, heads, ch = 2, 13, 29, 4, 24
    c = heads * ch
    qkv = rnd(g, n, h, w, 3 * c, dtype=dt)
    a = torch.softmax(rnd(g, n, heads, ch, ch, scale=2.0), -1)
    res = rnd(g, n, h, w, c, dtype=dt)
    ref = REF.linear_per_image(qkv[..., 2 * c:], _blockdiag_t(a), residual=res, out_dtype=torch.float32)
    got = hip.attention_apply(qkv.cuda(), a.cuda(), residual=res.cuda(), out_dtype=torch.float32)
    assert_fp32(got.cpu(), ref, rel=1e-5, what=f"attention_apply batch 2 + residual {dt}")
    # a map with a transposed (non-contiguous) view gives the same result
    got2 = hip.attention_apply(qkv.cuda(), a.transpose(-1, -2).contiguous().cuda().transpose(-1, -2),
                               residual=res.cuda(), out_dtype=torch.float32)
    assert torch.equal(got, got2)
    from clarus_amd.dispatch import Unsupported
    with pytest.raises(Unsupported):
        hip.attention_apply(qkv.cuda(), a[0].cuda())


@pytest.mark.parametrize("lvl", [0, 2])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_restormer_mix_fold(lvl, dt, hip_bf16, hip_f32):
    """The Restormer block's attention output path (python/clarus/models/restormer/__init__.py:
    203-210): the map from channel_attention, mix = blockdiag(A^T) @ proj.w per image, then
    linear_per_image(v, mix, residual=x, bias=proj.b), all on `hip`, against the same chain on
    the oracle. Level 0 at 180x320 (1 head), level 2 (4 heads) at 90x160."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(80 + lvl)
    c, heads = 48 * 2 ** lvl, 2 ** lvl
    h, w = (180, 320) if lvl == 0 else (90, 160)
    qkv = rnd(g, 1, h, w, 3 * c, dtype=dt)
    t = torch.rand(heads, generator=g) * 1.5 + 0.5
    proj_w, proj_b = rnd(g, c, c, scale=c ** -0.5), rnd(g, c, scale=0.1)
    x = rnd(g, 1, h, w, c, dtype=dt)
    a_hip = hip.channel_attention(qkv.cuda(), heads, t.cuda())
    mix_hip = _blockdiag_t(a_hip.cpu()).cuda() @ proj_w.cuda()
    got = hip.linear_per_image(qkv.cuda()[..., 2 * c:], mix_hip, residual=x.cuda(), out_dtype=torch.float32,
                               bias=proj_b.cuda())
    a_ref = REF.channel_attention(qkv, heads, t)
    mix_ref = _blockdiag_t(a_ref) @ proj_w
    ref = REF.linear_per_image(qkv[..., 2 * c:], mix_ref, residual=x, out_dtype=torch.float32, bias=proj_b)
    # the map carries the attention's own error (1e-4 relative for bf16 q / k, as in test_config4_mdta)
    assert_fp32(got.cpu(), ref, rel=1e-5 if dt == torch.float32 else 1e-4, what=f"restormer mix l{lvl} {dt}")


# ------------------------------------------------------------------ patch DFT ops
@pytest.mark.parametrize("h,w", [(64, 96), (45, 81), (16, 8)])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_patch_filter(h, w, dt, hip_bf16, hip_f32):
    """Non-symmetric random filter (irfft2's v = 0 / 4 handling matters), reflect padding for
    sizes that are not multiples of 8, residual."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(3)
    c = 40
    x, f, res = rnd(g, 2, h, w, c, dtype=dt), rnd(g, c, 8, 5), rnd(g, 2, h, w, c, dtype=dt)
    got = hip.patch_filter(x.cuda(), f.cuda(), residual=res.cuda(), out_dtype=torch.float32)
    assert_fp32(got.cpu(), REF.patch_filter(x, f, residual=res), rel=1e-5, what=f"patch_filter {h}x{w} {dt}")


CONFIG3 = [(48, 720, 1280), (96, 360, 640), (192, 180, 320)]


@pytest.mark.parametrize("c,h,w", CONFIG3)
def test_config3_patch_filter(c, h, w, hip_f32):
    """fp32 patches [1, C, H/8, W/8, 8, 8] (stored NHWC), fwd DFT 64 -> 80,
    seeded frequency-domain filter, inverse 80 -> 64."""
    g = gen(30 + c)
    x, f = torch.randn(1, h, w, c, generator=g), torch.randn(c, 8, 5, generator=g)
    got = hip_f32.patch_filter(x.cuda(), f.cuda())
    assert_fp32(got.cpu(), REF.patch_filter(x, f), rel=1e-5, what=f"config3 C{c}")


@pytest.mark.parametrize("h,w,k,nout,ln,res", [(64, 96, 48, 288, True, False), (40, 64, 192, 256, True, False),
                                               (90, 45, 144, 48, False, True), (52, 76, 96, 96, "rms", True)])
def test_linear_patch_filter(h, w, k, nout, ln, res, hip_bf16):
    """tools/test_kernels.py:237-245 cases. With LN over K >= HipOps.split_min_k the normalised
    rows are rounded once to bf16, as the reference's GPU path does (ops/triton_cuda.py:269-271):
    then the bf16 rule holds against that rounding emulated on the oracle, and the fp32 oracle
    (rows not rounded) is met within 2e-2 absolute beyond the output's own rounding to bf16."""
    from clarus_amd.hip_ops import HipOps
    g = gen(4)
    x, f = rnd(g, 1, h, w, k).bfloat16(), rnd(g, nout, 8, 5)
    wl, b = rnd(g, k, nout, scale=k ** -0.5).bfloat16(), rnd(g, nout)
    rr = rnd(g, 1, h, w, nout).bfloat16() if res else None
    got = hip_bf16.linear_patch_filter(x.cuda(), wl.cuda(), b.cuda(), f.cuda(), ln=ln, ln_eps=1e-5,
                                       residual=rr.cuda() if res else None)
    ref = REF.linear_patch_filter(x, wl, b, f, ln=ln, ln_eps=1e-5, residual=rr)
    what = f"linear_patch_filter {h}x{w} k{k} ln={ln}"
    rounded = (ln and not HipOps.prologue_split and HipOps.split_min_k <= k <= 2048 and k % 32 == 0)
    if not rounded:
        assert_bf16(got.cpu(), ref, what)
        return
    xr = REF.ln(x.float(), 1e-5, rms=(ln == "rms")).to(torch.bfloat16)  # the rows the GPU path rounds
    assert_bf16(got.cpu(), REF.linear_patch_filter(xr, wl, b, f, ln=False, residual=rr), what + " (rounded rows)")
    ref32 = TorchRef(torch.float32, "cpu").linear_patch_filter(x, wl, b, f, ln=ln, ln_eps=1e-5, residual=rr)
    d = assert_abs(got, ref32, what=what + " vs the fp32 oracle")
    print(f"[lpf] {what}: max|d| vs the fp32 oracle {d:.3e} (2e-2 absolute beyond the output rounding)")


# FFTformer DFFN project_in + filter (python/clarus/models/fftformer/__init__.py:160-161): K = c,
# N = 2 * hidden = 6c, LayerNorm eps 1e-5, at levels 0 / 1 / 3 (c = 48 / 96 / 384; K = 384 takes
# the rounded rows pass), on 180 x 320 or smaller images; EVSSM EDFFN project_out + filter
# (python/clarus/models/evssm/__init__.py:158): K = 144, N = 48, no LayerNorm, residual.
LPF_SHAPES = [(180, 320, 48, 288, True, False), (90, 161, 96, 576, True, False), (45, 83, 384, 2304, True, False),
              (180, 320, 144, 48, False, True), (93, 150, 144, 48, "rms", True)]


@pytest.mark.parametrize("h,w,k,nout,ln,res", LPF_SHAPES)
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_linear_patch_filter_fused_model_shapes(h, w, k, nout, ln, res, dt, hip_bf16, hip_f32):
    """The one-kernel linear_patch_filter (clarus_hip_linear_patch_filter) at the FFTformer / EVSSM
    call shapes against the oracle (fp32: 1e-5 relative; bf16: the bf16 rule, against the rows
    rounded once to bf16 where the rows pass runs), and against the two-op path on the GPU (the
    same arithmetic up to fp32 summation order)."""
    from clarus_amd import _lib
    from clarus_amd.hip_ops import HipOps
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(50 + k)
    x, f = rnd(g, 1, h, w, k).to(dt), rnd(g, nout, 8, 5)
    wl, b = rnd(g, k, nout, scale=k ** -0.5).to(dt), rnd(g, nout, scale=0.1)
    rr = rnd(g, 1, h, w, nout).to(dt) if res else None
    dv = [None if t is None else t.cuda() for t in (x, wl, b, f, rr)]
    print(f"[lpf] {dt} {h}x{w} k{k} n{nout} ln={ln} res={res}", flush=True)
    got = hip.linear_patch_filter(*dv[:4], ln=ln, ln_eps=1e-5, residual=dv[4])
    assert "lpf_kernel" in _lib.last_kernel(), _lib.last_kernel()
    saved = HipOps.fuse_patch_filter
    try:
        HipOps.fuse_patch_filter = False
        two = hip.linear_patch_filter(*dv[:4], ln=ln, ln_eps=1e-5, residual=dv[4])
    finally:
        HipOps.fuse_patch_filter = saved
    what = f"fused linear_patch_filter {dt} {h}x{w} k{k} ln={ln}"
    rounded = (bool(ln) and dt == torch.bfloat16 and not HipOps.prologue_split and HipOps.split_min_k <= k <= 2048
               and k % 32 == 0)
    xr = REF.ln(x.float(), 1e-5, rms=(ln == "rms")).to(torch.bfloat16) if rounded else x
    ref = REF.linear_patch_filter(xr, wl, b, f, ln=False if rounded else ln, ln_eps=1e-5, residual=rr)
    if dt == torch.float32:
        assert_fp32(got.cpu(), ref, rel=1e-5, what=what)
        assert_fp32(got.cpu(), two.cpu(), rel=1e-5, what=what + " vs two ops")
    else:
        ref32 = REF.linear(xr, wl, b, ln=False if rounded else ln, ln_eps=1e-5, out_dtype=torch.float32)
        ref32 = TorchRef(torch.float32, "cpu").patch_filter(ref32, f, residual=rr)
        assert_bf16(got.cpu(), ref32, what)
        # both outputs rounded to bf16 from fp32 values that differ by summation order only
        assert_abs(got, two.float(), what=what + " vs two ops", ulps=1.0)


def test_linear_patch_filter_bench_shape(hip_bf16):
    """The bench's FFTformer level-0 DFFN row as timed (workloads.fftformer_dffn_case: 720 x 1280,
    LayerNorm eps 1e-5, 48 -> 288, bf16, its seeded inputs) against the fp32 oracle: the bf16 rule
    (2e-2 absolute up to rounding flips, checked per 1/8 of the output), and 2e-2 absolute beyond
    the output's rounding."""
    from clarus_amd import _lib, workloads as wl
    case = wl.fftformer_dffn_case(hip_bf16, "cuda")
    print(f"[lpf] bench workload {case.name}", flush=True)
    got = case.run().cpu()
    kern = _lib.last_kernel()
    h = case.cpu
    ref32 = TorchRef(torch.float32, "cpu").linear_patch_filter(h["x"], h["w"], h["b"], h["f"], ln=True, ln_eps=1e-5)
    assert got.dtype == torch.bfloat16 and got.shape == ref32.shape == (1, 720, 1280, 288)
    flips = 0
    for part in range(8):  # 90 image rows at a time
        sl = slice(90 * part, 90 * (part + 1))
        flips += assert_bf16(got[:, sl], ref32[:, sl], what=f"lpf bench shape rows {sl}")[1]
    d = assert_abs(got, ref32, what="lpf bench shape")
    print(f"[lpf] bench workload ({kern}): max|d| {d:.3e}, rounding flips {flips}")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_patch_corr(dt, hip_bf16, hip_f32):
    """tools/test_kernels.py:246-247 (q, k channel slices) and the stride cases of
    tools/test_ops_contracts.py:128-141 (batch stride 2HWC, batch stride 0, channel slice,
    H/W-transposed view)."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(5)
    x = rnd(g, 2, 64, 96, 288, dtype=dt)
    assert_fp32(hip.patch_corr(x.cuda(), 96).cpu(), REF.patch_corr(x, 96), rel=1e-5, what=f"patch_corr {dt}")
    c = 32
    base = rnd(g, 4, 16, 24, 2 * c + 16, dtype=dt)
    bd = base.cuda()
    for name, fn in [("batch stride 2HWC", lambda t: t[::2]), ("batch stride 0", lambda t: t[:1].expand(3, -1, -1, -1)),
                     ("channel slice", lambda t: t[..., 8:8 + 2 * c]), ("H/W transposed", lambda t: t.transpose(1, 2))]:
        assert_fp32(hip.patch_corr(fn(bd), c).cpu(), REF.patch_corr(fn(base), c), rel=1e-5, what=f"patch_corr {name}")
