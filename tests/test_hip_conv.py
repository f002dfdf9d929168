"""GPU parity: implicit-GEMM 3x3 convolutions (conv3x3, ending) and intro vs the oracle.

Cases follow tools/test_kernels.py:134-191 (channel-slice in / out, LeakyReLU, out_scale,
residual, nearest-x2 input, NCHW fp32 ending with global residual, intro 3 -> C) and BASELINE
config 5 (RRDBNet dense block convs on a 256x384 feature map and the x2 up-convs).
"""
from __future__ import annotations

import pytest
import torch

from _tol import BF16_ABS, assert_bf16, assert_fp32, bf16_ulp
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


def check(got, ref32, what):
    if got.dtype == torch.bfloat16:
        return assert_bf16(got, ref32, what)
    return assert_fp32(got.float(), ref32, what=what)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_conv3x3_plain(dt, hip_bf16, hip_f32):
    """cout 27 (no padding needed), odd sizes."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(1)
    x, w, b = rnd(g, 2, 19, 27, 64, dtype=dt), rnd(g, 27, 64, 3, 3, scale=0.1, dtype=dt), rnd(g, 27)
    got = hip.conv3x3(x.cuda(), w.cuda(), b.cuda(), out_dtype=torch.float32)
    assert_fp32(got.cpu(), REF.conv3x3(x, w, b), what=f"conv3x3 cout27 {dt}")


def test_conv3x3_slices_lrelu_scale_res(hip_bf16):
    """Input / output channel slices of one buffer, LeakyReLU, out_scale, residual."""
    g = gen(2)
    n, h, w = 2, 21, 34
    buf = rnd(g, n, h, w, 96, dtype=torch.bfloat16)
    wt, b, res = rnd(g, 32, 64, 3, 3, scale=0.05, dtype=torch.bfloat16), rnd(g, 32), rnd(g, n, h, w, 32,
                                                                                          dtype=torch.bfloat16)
    ref = REF.conv3x3(buf[..., :64], wt, b, act="lrelu", out_scale=0.2, residual=res, out_dtype=torch.float32)
    bd = buf.cuda()
    got = hip_bf16.conv3x3(bd[..., :64], wt.cuda(), b.cuda(), act="lrelu", out_scale=0.2, residual=res.cuda(),
                           out=bd[..., 64:])
    assert got.data_ptr() == bd[..., 64:].data_ptr()
    check(bd[..., 64:].cpu(), ref, "conv3x3 slice+lrelu+scale+res")
    assert torch.equal(bd[..., :64].cpu(), buf[..., :64]), "input slice was modified"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_conv3x3_up2(dt, hip_bf16, hip_f32):
    """Nearest-x2 upsample fused into the input addressing, cout 40."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(3)
    x, w, b = rnd(g, 2, 21, 34, 48, dtype=dt), rnd(g, 40, 48, 3, 3, scale=0.05, dtype=dt), rnd(g, 40)
    got = hip.conv3x3(x.cuda(), w.cuda(), b.cuda(), up2=True, act="lrelu")
    check(got.cpu(), REF.conv3x3(x, w, b, up2=True, act="lrelu"), f"conv3x3 up2 {dt}")


@pytest.mark.parametrize("cin,cout,up2,h,w,n,bias", [(64, 32, False, 13, 45, 2, True), (96, 64, False, 8, 32, 1, True),
                                                      (64, 64, True, 11, 19, 2, True), (192, 64, False, 9, 40, 1, True),
                                                      (32, 48, True, 5, 7, 1, True), (128, 40, False, 17, 33, 1, True),
                                                      (64, 64, True, 19, 13, 1, False), (64, 40, False, 10, 70, 2, False)])
def test_conv3x3_halo_shapes(cin, cout, up2, h, w, n, bias, hip_bf16):
    """bf16 convs with cin % 32 == 0 (the halo-tile kernel): ragged 8 x 32 tiles (16 x 32 with the
    x2 upsample), several tiles per workgroup (a tile's stores are issued during the next tile's
    first chunk), batch 2, x2 upsample, output channels that are not a multiple of the 32 /
    64-channel tile, LeakyReLU, out_scale, a residual, and no bias (the kernel's bias table then
    holds zeros)."""
    from clarus_amd import _lib
    g = gen(13)
    x = rnd(g, n, h, w, cin, dtype=torch.bfloat16)
    wt = rnd(g, cout, cin, 3, 3, scale=(cin * 9) ** -0.5, dtype=torch.bfloat16)
    b = rnd(g, cout) if bias else None
    H, W = (2 * h, 2 * w) if up2 else (h, w)
    res = rnd(g, n, H, W, cout, dtype=torch.bfloat16)
    got = hip_bf16.conv3x3(x.cuda(), wt.cuda(), None if b is None else b.cuda(), act="lrelu", out_scale=0.5,
                           residual=res.cuda(), up2=up2)
    assert _lib.last_kernel().startswith("conv_halo_kernel"), _lib.last_kernel()
    ref = REF.conv3x3(x, wt, b, act="lrelu", out_scale=0.5, residual=res, up2=up2, out_dtype=torch.float32)
    check(got.cpu(), ref, f"conv3x3 halo cin{cin} cout{cout} up2={up2} {n}x{h}x{w} bias={bias}")


@pytest.mark.parametrize("tile", [12, 4])
def test_conv3x3_kernels_agree(tile, hip_bf16):
    """Through the C ABI: the halo-tile kernel (12) and an implicit-GEMM tile (4) on one problem
    with channel slices, fp32 output, against the oracle."""
    import ctypes

    from clarus_amd import _lib
    lib = _lib.load()
    g = gen(14)
    n, h, w, cin, cout = 1, 21, 37, 96, 32
    buf = rnd(g, n, h, w, 128, dtype=torch.bfloat16)
    wt = rnd(g, cout, cin, 3, 3, scale=(cin * 9) ** -0.5, dtype=torch.bfloat16)
    b = rnd(g, cout)
    ref = REF.conv3x3(buf[..., :cin], wt, b, act="lrelu", out_dtype=torch.float32)
    wtk = wt.permute(0, 2, 3, 1).reshape(cout, 9 * cin).contiguous().cuda()  # W^T [cout][(ky, kx, cin)]
    bd, bias = buf.cuda(), b.cuda()
    out = torch.empty(n, h, w, cout, device="cuda")
    args = _lib.ConvArgs(x=bd.data_ptr(), wt=wtk.data_ptr(), out=out.data_ptr(), bias=bias.data_ptr(),
                         batch=n, h=h, w=w, cin=cin, cout=cout, ldx=128, ldo=cout, ldr=0,
                         x_dtype=_lib.BF16, w_dtype=_lib.BF16, o_dtype=_lib.F32, act=_lib.ACT_LRELU,
                         out_scale=1.0, slope=0.2, tile=tile)
    _lib.check(lib.clarus_hip_conv3x3(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
               "conv3x3")
    assert_fp32(out.cpu(), ref, rel=1e-5, what=f"conv3x3 tile {tile}")


def test_ending_and_intro(hip_bf16):
    """ending: fp32 input at |x| ~ 300 (implicit GEMM) and bf16 input (halo-tile kernel, 16-channel
    tile, NCHW fp32 stores), NCHW fp32 output + global residual; intro 3 -> 64 / 128 (fp32 MFMA
    kernel) and 48 (FMA kernel)."""
    g = gen(4)
    n, h, w = 2, 19, 27
    x3 = torch.rand(n, 3, h, w, generator=g)
    for xdt, mag in ((torch.float32, 300.0), (torch.bfloat16, 1.0)):
        xe = rnd(g, n, h, w, 64, scale=mag).to(xdt)
        we, be = rnd(g, 3, 64, 3, 3, scale=0.1, dtype=torch.bfloat16), rnd(g, 3)
        got = hip_bf16.ending(xe.cuda(), we.cuda(), be.cuda(), x3.cuda())
        assert_fp32(got.cpu(), REF.ending(xe, we, be, x3), what=f"ending {xdt} NCHW + res")
    for c in (64, 128, 48):
        wi, bi = rnd(g, c, 3, 3, 3, scale=0.3), rnd(g, c)
        got = hip_bf16.intro(x3.cuda(), wi.cuda(), bi.cuda(), out_dtype=torch.float32)
        assert_fp32(got.cpu(), REF.intro(x3, wi, bi, out_dtype=torch.float32), what=f"intro 3->{c}")
        got = hip_bf16.intro(x3.cuda(), wi.cuda(), bi.cuda())
        check(got.cpu(), REF.intro(x3, wi, bi, out_dtype=torch.float32), what=f"intro 3->{c} bf16")


@pytest.mark.parametrize("mag", [2.0 ** -18, 1.0, 6e4, 1e7])
def test_conv3x3_fp32_input_range(mag, hip_bf16):
    """fp32 input, bf16 weights, per-row relative vs float64 (tools/test_kernel_contracts.py:119-126)."""
    g = gen(5)
    x = rnd(g, 2, 10, 14, 48, scale=mag)
    w = rnd(g, 32, 48, 3, 3, scale=0.1, dtype=torch.bfloat16)
    got = hip_bf16.conv3x3(x.cuda(), w.cuda(), None, out_dtype=torch.float32).cpu().double().reshape(-1, 32)
    ref = torch.nn.functional.conv2d(x.double().permute(0, 3, 1, 2), w.double(), padding=1)
    ref = ref.permute(0, 2, 3, 1).reshape(-1, 32)
    row_rel = ((got - ref).abs().amax(1) / ref.abs().amax(1)).max().item()
    assert row_rel < 1e-4, row_rel


def test_config5_dense_block(hip_bf16):
    """one RRDB dense block on a 1x256x384 feature map (64 features, growth
    32) inside one [1, 256, 384, 192] NHWC buffer, convs 64/96/128/160 -> 32 (+ LeakyReLU) into
    the next slice, then 192 -> 64 * 0.2 + x into a second buffer. Weights kaiming-normal x 0.1."""
    g = gen(0)
    h, w = 256, 384
    buf = torch.zeros(1, h, w, 192).bfloat16()
    buf[..., :64] = torch.randn(1, h, w, 64, generator=g).bfloat16()
    ws = []
    for cin in (64, 96, 128, 160):
        ws.append(((torch.randn(32, cin, 3, 3, generator=g) * (2.0 / (cin * 9)) ** 0.5) * 0.1).bfloat16())
    w5 = ((torch.randn(64, 192, 3, 3, generator=g) * (2.0 / (192 * 9)) ** 0.5) * 0.1).bfloat16()
    bs = [torch.zeros(32) for _ in range(4)] + [torch.zeros(64)]
    ref_buf = buf.clone()
    bd = buf.cuda()
    for i, cin in enumerate((64, 96, 128, 160)):
        hip_bf16.conv3x3(bd[..., :cin], ws[i].cuda(), bs[i].cuda(), act="lrelu", out=bd[..., cin:cin + 32])
        r = REF.conv3x3(ref_buf[..., :cin], ws[i], bs[i], act="lrelu", out_dtype=torch.float32)
        check(bd[..., cin:cin + 32].cpu(), r, f"config5 conv{i + 1} {cin}->32")
        ref_buf[..., cin:cin + 32] = bd[..., cin:cin + 32].cpu()  # continue from identical inputs
    out = torch.empty(1, h, w, 192, dtype=torch.bfloat16, device="cuda")
    hip_bf16.conv3x3(bd, w5.cuda(), bs[4].cuda(), out_scale=0.2, residual=bd[..., :64], out=out[..., :64])
    r = REF.conv3x3(ref_buf, w5, bs[4], out_scale=0.2, residual=ref_buf[..., :64], out_dtype=torch.float32)
    check(out[..., :64].cpu(), r, "config5 conv5 192->64 *0.2 + x")


@pytest.mark.parametrize("h,w", [(256, 384), (512, 768)])
def test_config5_upconv(h, w, hip_bf16):
    """BASELINE config 5 up-convs: nearest x2 + 3x3 64 -> 64 + LeakyReLU (out 512x768, 1024x1536)."""
    g = gen(7)
    x = torch.randn(1, h, w, 64, generator=g).bfloat16()
    wt = ((torch.randn(64, 64, 3, 3, generator=g) * (2.0 / 576) ** 0.5) * 0.1).bfloat16()
    b = torch.zeros(64)
    got = hip_bf16.conv3x3(x.cuda(), wt.cuda(), b.cuda(), act="lrelu", up2=True)
    check(got.cpu(), REF.conv3x3(x, wt, b, act="lrelu", up2=True, out_dtype=torch.float32), f"upconv {h}x{w}")


# ------------------------------------------------------------------ depthwise 3x3 (next op on the NAFNet path)
@pytest.mark.parametrize("c", [96, 528, 640])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("gate,act,dil", [(True, None, 1), ("gelu", None, 1), (False, None, 1),
                                          (False, "gelu", 1), (False, None, 2)])
def test_dwconv(dt, gate, act, dil, c, hip_bf16, hip_f32):
    """Depthwise 3x3 + SimpleGate / GELU gate / GELU / dilation 2 (tools/test_kernels.py:110-121,
    193-199), odd sizes (two images of 37 x 53, partial tiles at both edges): bf16 with a gate
    takes the LDS-tiled kernel; otherwise 96 channels take the sliding-window kernel (dilation
    1), 528 and 640 the per-pixel one."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(8)
    x, w, b = rnd(g, 2, 37, 53, c, dtype=dt), rnd(g, c, 1, 3, 3), rnd(g, c)
    got = hip.dwconv(x.cuda(), w.cuda(), b.cuda(), dil=dil, gate=gate, act=act)
    ref = TorchRef(torch.float32, "cpu").dwconv(x, w, b, dil=dil, gate=gate, act=act)
    check(got.cpu(), ref, f"dwconv gate={gate} act={act} dil={dil} {dt}")


@pytest.mark.parametrize("h,w,c", [(90, 160, 1024), (45, 80, 2048), (180, 320, 512)])
def test_dwconv_nafnet_wide_levels(h, w, c, hip_bf16):
    """NAFNet-w64 720p levels 3, 4 and 2 (dwconv of conv1's 2c channels -> SimpleGate -> c) on the
    LDS-tiled kernel."""
    from clarus_amd import _lib
    g = gen(11)
    x, wt, b = rnd(g, 1, h, w, c, dtype=torch.bfloat16), rnd(g, c, 1, 3, 3), rnd(g, c)
    got = hip_bf16.dwconv(x.cuda(), wt.cuda(), b.cuda(), gate=True)
    assert _lib.last_kernel().startswith("dw_tile_kernel gate=1"), _lib.last_kernel()
    check(got.cpu(), TorchRef(torch.float32, "cpu").dwconv(x, wt, b, gate=True), f"dwconv {h}x{w}x{c} gate")


@pytest.mark.parametrize("level", [3, 0])
def test_dwconv_bench_rows(level, hip_bf16):
    """The bench's NAFNet depthwise rows as timed (workloads.nafnet_dw_case: 90 x 160 x 1024 and
    720 x 1280 x 128, SimpleGate, bias) against the oracle."""
    from clarus_amd import _lib, workloads as wl
    case = wl.nafnet_dw_case(hip_bf16, torch.device("cuda"), level)
    got = case.run()
    assert _lib.last_kernel().startswith("dw_tile_kernel gate=1"), _lib.last_kernel()
    ref = case.cpu_run(TorchRef(torch.float32, "cpu"))
    check(got.cpu(), ref, case.name)


@pytest.mark.parametrize("n,h,w,c", [(1, 1, 1, 16), (1, 5, 3, 96), (3, 7, 17, 128), (1, 13, 33, 2064)])
@pytest.mark.parametrize("gate", [True, "gelu"])
def test_dwconv_tile_edges(n, h, w, c, gate, hip_bf16):
    """The LDS-tiled kernel (bf16 input with a gate) at its edges: a single pixel, images smaller
    than one 6 x 16 tile, three images whose tiles end inside the image in both directions, and
    a channel slice that is partly past the outputs (1032 = 16 x 64 + 8 output channels); no
    bias in the GELU-gate cases."""
    from clarus_amd import _lib
    g = gen(13)
    x, wt = rnd(g, n, h, w, c, dtype=torch.bfloat16), rnd(g, c, 1, 3, 3)
    b = None if gate == "gelu" else rnd(g, c)
    got = hip_bf16.dwconv(x.cuda(), wt.cuda(), None if b is None else b.cuda(), gate=gate)
    assert _lib.last_kernel().startswith("dw_tile_kernel"), _lib.last_kernel()
    check(got.cpu(), TorchRef(torch.float32, "cpu").dwconv(x, wt, b, gate=gate), f"dwconv {n}x{h}x{w}x{c} gate={gate}")


def test_dwconv_bf16_in_fp32_out(hip_bf16):
    """bf16 input with an fp32 output (a combination HipOps does not produce), through the C ABI:
    640 channels, no gate and with the gate, two images of 37 x 53, against the oracle's fp32
    result."""
    import ctypes
    from clarus_amd import _lib
    g = gen(12)
    n, h, w, c = 2, 37, 53, 640
    x, wt, b = rnd(g, n, h, w, c, dtype=torch.bfloat16), rnd(g, c, 1, 3, 3), rnd(g, c)
    taps = wt.float().reshape(c, 9).t().contiguous().cuda()
    for gate in (0, 1):
        cout = c // 2 if gate else c
        out = torch.empty(n, h, w, cout, device="cuda", dtype=torch.float32)
        xc, bc = x.cuda(), b.cuda()
        _lib.check(hip_bf16.lib.clarus_hip_dwconv3x3(
            xc.data_ptr(), _lib.BF16, taps.data_ptr(), bc.data_ptr(), out.data_ptr(), _lib.F32, n, h, w, c, 1, gate, 0,
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "dwconv3x3")
        torch.cuda.synchronize()
        ref = TorchRef(torch.float32, "cpu").dwconv(x, wt, b, gate=bool(gate))
        assert_fp32(out.cpu(), ref, what=f"dwconv bf16 -> fp32 gate={gate}")


@pytest.mark.parametrize("n,h,w,full", [(2, 13, 37, True), (1, 5, 3, False), (1, 6, 30, True),
                                        (1, 720, 1280, True)])
def test_linear_dwconv(n, h, w, full, hip_bf16):
    """linear_dwconv on clarus_hip_ln_gemm_dwconv (NAFNet level-0 first half: LN -> 64 -> 128 ->
    depthwise 3x3 -> SimpleGate): partial tiles at both image edges, an image smaller than one
    tile, exactly one tile, two images, biases absent, and 720p. The oracle runs the two ops with
    the 1x1 conv's output rounded to bf16 as the unfused path stores it (fp32 products: the kernel
    feeds the LayerNorm rows as hi + lo pairs)."""
    from clarus_amd import _lib
    g = gen(14)
    x = (rnd(g, n, h, w, 64) + 0.3).bfloat16()
    wt = (rnd(g, 64, 128) / 8).bfloat16()
    b = rnd(g, 128, scale=0.1) if full else None
    dw, dwb = rnd(g, 128, 1, 3, 3, scale=0.3), (rnd(g, 128, scale=0.1) if full else None)
    got = hip_bf16.linear_dwconv(x.cuda(), wt.cuda(), None if b is None else b.cuda(), dw.cuda(),
                                 None if dwb is None else dwb.cuda())
    assert _lib.last_kernel().startswith("ln_dw_kernel"), _lib.last_kernel()
    check_linear_dwconv(got.cpu(), x, wt, b, dw, dwb, f"linear_dwconv {n}x{h}x{w}")


def check_linear_dwconv(got, x, wt, b, dw, dwb, what):
    """got (bf16) against the oracle's two ops with t rounded to bf16. The kernel rounds its own t,
    summed in another order, so an element of t may sit one bf16 step from the oracle's (a rounding
    flip of the intermediate); elementwise the difference is held to what such flips can cause,
    |a1| e2 + |a2| e1 + e1 e2 with e = |taps| * ulp(t) through the depthwise conv (a1, a2: the gate
    halves), plus one output rounding step. Elements beyond 2e-2 of the output scale may only be
    such flips, at most 1e-3 of them."""
    ref32 = TorchRef(torch.float32, "cpu")
    t32 = ref32.linear(x, wt, b, ln=True)
    t = t32.bfloat16()
    ref = ref32.dwconv(t, dw, dwb, gate=True).double()
    a = ref32.dwconv(t, dw, dwb, gate=False).double()
    e = ref32.dwconv(bf16_ulp(t32.float()), dw.abs(), None, gate=False).double()
    c = a.shape[-1] // 2
    a1, a2, e1, e2 = a[..., :c], a[..., c:], e[..., :c], e[..., c:]
    bound = a1.abs() * e2 + a2.abs() * e1 + e1 * e2 + bf16_ulp(ref.float()).double() + 1e-5 * ref.abs().max()
    d = (got.double() - ref).abs()
    assert bool((d <= bound).all()), f"{what}: {int((d > bound).sum())} elements beyond the bound; max {d.max():.3e}"
    far = int((d > BF16_ABS * ref.abs().clamp_min(1.0)).sum())
    assert far <= max(1, 1e-3 * d.numel()), f"{what}: {far} elements beyond 2e-2 of their scale"
    print(f"[linear_dwconv] {what}: max |d| {d.max():.3e}, {far} beyond 2e-2 of their scale")


def test_linear_dwconv_unfused_shapes(hip_bf16):
    """Shapes the fused kernel does not take (128 channels) run the two ops, bit for bit."""
    from clarus_amd import _lib
    g = gen(15)
    x = rnd(g, 1, 9, 11, 128, dtype=torch.bfloat16).cuda()
    wt, b = (rnd(g, 128, 256) / 11).bfloat16().cuda(), rnd(g, 256).cuda()
    dw, dwb = rnd(g, 256, 1, 3, 3).cuda(), rnd(g, 256).cuda()
    got = hip_bf16.linear_dwconv(x, wt, b, dw, dwb)
    assert not _lib.last_kernel().startswith("ln_dw_kernel")
    want = hip_bf16.dwconv(hip_bf16.linear(x, wt, b, ln=True), dw, dwb, gate=True)
    assert torch.equal(got, want)


def test_dwconv_nafnet_720p(hip_bf16):
    """NAFNet level 0: 1x720x1280x128 -> SimpleGate -> 64 channels."""
    g = gen(9)
    x, w, b = rnd(g, 1, 720, 1280, 128, dtype=torch.bfloat16), rnd(g, 128, 1, 3, 3), rnd(g, 128)
    got = hip_bf16.dwconv(x.cuda(), w.cuda(), b.cuda(), gate=True)
    check(got.cpu(), TorchRef(torch.float32, "cpu").dwconv(x, w, b, gate=True), "dwconv 720p gate")


# ------------------------------------------------------------------ TLC local mean (NAFNet SCA input)
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("h,w,k", [(37, 53, 13), (37, 53, (26, 53)), (20, 30, 64), (33, 33, 33), (9, 150, 5)])
def test_boxmean(dt, h, w, k, hip_bf16, hip_f32):
    """Valid-window local mean vs the oracle's prefix-sum form (tools/test_model_contracts.py:
    149-163 windows), odd sizes, windows clamped to the map, a 1 x W output row."""
    hip = hip_bf16 if dt == torch.bfloat16 else hip_f32
    g = gen(10)
    x = (1.5 + rnd(g, 2, h, w, 24)).to(dt)
    got = hip.boxmean(x.cuda(), k)
    ref = TorchRef(torch.float32, "cpu").boxmean(x, k)
    assert (got.pt, got.pl, got.H, got.W) == (ref.pt, ref.pl, ref.H, ref.W)
    assert got.data.shape == ref.data.shape
    check(got.data.cpu(), ref.data.float(), f"boxmean {h}x{w} k={k} {dt}")


def test_boxmean_exact_float64():
    """fp32 input: every window sum against a float64 brute force (the HIP kernel accumulates in
    fp64, so it is held to 2e-7 relative, tighter than the prefix-sum oracle itself)."""
    from clarus_amd.hip_ops import HipOps
    hip = HipOps(torch.float32, torch.device("cuda", 0))
    g = gen(11)
    x = 100 + rnd(g, 1, 40, 60, 16)
    got = hip.boxmean(x.cuda(), (17, 23)).data.cpu().double()
    xd = x.double()
    s = torch.nn.functional.pad(xd.cumsum(2).cumsum(1), (0, 0, 1, 0, 1, 0))
    ref = (s[:, 17:, 23:] + s[:, :-17, :-23] - s[:, :-17, 23:] - s[:, 17:, :-23]) / (17 * 23)
    assert ((got - ref).abs() / ref.abs()).max().item() < 2e-7


@pytest.mark.parametrize("h,w,c,k", [(720, 1280, 64, 384), (360, 640, 128, 192), (600, 1024, 64, 300)])
def test_boxmean_nafnet_levels(h, w, c, k, hip_bf16):
    """NAFNet-w64 levels 0 and 1 at 720p: windows 384 / 192 (maps 337 x 897 / 169 x 449), 32
    threads per line block; and a 300 window whose passes keep all of a thread's rows in
    registers (19 bf16 rows of the vertical pass in the 24-row form, 10 fp32 rows of the
    horizontal pass in the 16-row form)."""
    g = gen(12)
    x = rnd(g, 1, h, w, c, dtype=torch.bfloat16)
    got = hip_bf16.boxmean(x.cuda(), k)
    ref = TorchRef(torch.float32, "cpu").boxmean(x, k)
    assert got.data.shape == (1, h - k + 1, w - k + 1, c)
    check(got.data.cpu(), ref.data.float(), f"boxmean {h}x{w} k={k}")
