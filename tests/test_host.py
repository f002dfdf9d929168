"""CPU: the host side of the HIP backend.

  * the dispatch contract (clarus_amd.dispatch, restating python/clarus/ops/__init__.py):
    fallback on Unsupported, the last backend re-raises, overrides, served counters, report(),
    BackendUnavailable skips, registration by decorator and by path, Backend.cached;
  * HipOps refuses to construct off-GPU (BackendUnavailable, never a silent CPU path);
  * the DFT matrices the patch kernels use, against numpy.fft and torch.fft;
  * the NAFNet harness (weight folding + forward wiring) against an unfolded float64 NAFNet
    written from the upstream block definition, and the TLC windows known answer
    (tools/test_model_contracts.py:149-163).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from clarus_amd import dispatch
from clarus_amd.dft import dft_matrices, filter_gains
from clarus_amd.dispatch import Backend, BackendUnavailable, Ops, Unsupported, register_backend
from oracle.torch_ref import TorchRef


# ------------------------------------------------------------------ dispatch
class _Declines(Backend):
    name = "declines"

    def linear(self, x, *a, **k):
        if x.shape[-1] != 4:
            raise Unsupported("only K = 4")
        return "fast"

    def only_here(self, x):
        raise Unsupported("never")


class _All(Backend):
    name = "all"

    def linear(self, x, *a, **k):
        return "slow"

    def dwconv(self, x):
        return "dw"


class _Unavailable(Backend):
    name = "unavailable"

    def __init__(self, dtype, device):
        raise BackendUnavailable("not on this device")


@pytest.fixture(autouse=True)
def _registered():
    register_backend("declines")(_Declines)
    register_backend("all")(_All)
    register_backend("unavailable")(_Unavailable)
    register_backend("oracle_by_path", "tests.test_host:_OracleBackend")
    yield


def test_fallback_and_counters():
    logs = []
    ops = Ops(["unavailable", "declines", "all"], torch.float32, torch.device("cpu"), log=logs.append)
    assert [b.name for b in ops.backends] == ["declines", "all"]
    assert "unavailable" in ops.skipped and logs
    assert ops.linear(torch.zeros(1, 1, 1, 4)) == "fast"
    assert ops.linear(torch.zeros(1, 1, 1, 8)) == "slow"
    assert ops.dwconv(None) == "dw"
    rep = ops.report()
    assert rep["ops"]["linear"] == {"all": 1, "declines": 1} and rep["ops"]["dwconv"] == {"all": 1}
    with pytest.raises(Unsupported):  # the last backend's Unsupported propagates
        ops.only_here(None)
    with pytest.raises(AttributeError):
        ops.not_an_op


def test_overrides():
    ops = Ops(["declines", "all"], torch.float32, torch.device("cpu"), overrides={"linear": "all"},
              log=lambda *a: None)
    assert ops.linear(torch.zeros(1, 1, 1, 4)) == "slow"
    with pytest.raises(ValueError):
        Ops(["all"], torch.float32, torch.device("cpu"), overrides={"linear": "declines"}, log=lambda *a: None)
    with pytest.raises(RuntimeError):
        Ops(["unavailable"], torch.float32, torch.device("cpu"), log=lambda *a: None)
    with pytest.raises(ValueError):
        Ops(["no_such_backend"], torch.float32, torch.device("cpu"), log=lambda *a: None)


def test_cached_relayout_once():
    b = _All(torch.float32, torch.device("cpu"))
    w = torch.randn(4, 3)
    calls = []
    f = lambda t: calls.append(1) or t.t().contiguous()  # noqa: E731
    assert torch.equal(b.cached(w, "t", f), w.t())
    b.cached(w, "t", f)
    assert len(calls) == 1


def test_hip_backend_unavailable_on_cpu():
    """Off a gfx950 device the hip backend refuses to exist (Ops logs and skips it); it never
    runs a CPU path in its place."""
    from clarus_amd.hip_ops import HipOps
    with pytest.raises(BackendUnavailable):
        HipOps(torch.bfloat16, torch.device("cpu"))
    ops = Ops(["hip", "oracle_by_path"], torch.bfloat16, torch.device("cpu"), log=lambda *a: None)
    assert "hip" in ops.skipped and [b.name for b in ops.backends] == ["oracle"]


def test_host_clarus_absent():
    assert dispatch._host is None and dispatch.Unsupported is dispatch._Unsupported


# ------------------------------------------------------------------ DFT matrices
def test_dft_matrices_vs_numpy_and_torch():
    fwd, inv = dft_matrices(8)
    assert fwd.shape == (80, 64) and inv.shape == (64, 80)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 8, 8))
    spec = np.fft.rfft2(x)                                # [5, 8, 5]
    got = x.reshape(5, 64) @ fwd.T                       # [5, 80]
    assert np.allclose(got[:, 0::2], spec.real.reshape(5, 40), atol=1e-12)
    assert np.allclose(got[:, 1::2], spec.imag.reshape(5, 40), atol=1e-12)
    # inverse of arbitrary (non-Hermitian) coefficients: numpy and torch agree with Inv
    c = rng.standard_normal((5, 80))
    z = c[:, 0::2] + 1j * c[:, 1::2]
    ref_np = np.fft.irfft2(z.reshape(5, 8, 5), s=(8, 8)).reshape(5, 64)
    ref_t = torch.fft.irfft2(torch.from_numpy(z.reshape(5, 8, 5)), s=(8, 8)).reshape(5, 64).numpy()
    assert np.allclose(c @ inv.T, ref_np, atol=1e-12)
    assert np.allclose(c @ inv.T, ref_t, atol=1e-12)
    # round trip on real patches
    assert np.allclose((x.reshape(5, 64) @ fwd.T) @ inv.T, x.reshape(5, 64), atol=1e-12)


def test_filter_gains_match_the_oracle_patch_filter():
    """y = Inv (g * (Fwd x)) reproduces irfft2(rfft2(x) * f) (the oracle) for a random,
    non-symmetric real filter."""
    g = torch.Generator().manual_seed(0)
    x, f = torch.randn(1, 8, 8, 3, generator=g), torch.randn(3, 8, 5, generator=g)
    fwd, inv = dft_matrices(8)
    gains = filter_gains(f.numpy())                       # [3, 80]
    xs = x[0].double().numpy().reshape(64, 3)             # pixel-major
    y = np.stack([inv @ (gains[c] * (fwd @ xs[:, c])) for c in range(3)], axis=1).reshape(8, 8, 3)
    ref = TorchRef().patch_filter(x, f)[0].double().numpy()
    assert np.abs(y - ref).max() < 1e-5


# ------------------------------------------------------------------ NAFNet harness
class _OracleBackend(Backend):
    """The oracle behind the dispatch contract (test use)."""
    name = "oracle"

    def __init__(self, dtype, device):
        super().__init__(dtype, device)
        self._r = TorchRef(dtype, device)

    def __getattr__(self, op):
        if op.startswith("_"):
            raise AttributeError(op)
        return getattr(self._r, op)


def _layernorm2d(x, w, b, eps=1e-6):
    mu = x.mean(1, keepdim=True)
    var = (x - mu).pow(2).mean(1, keepdim=True)
    return (x - mu) / (var + eps).sqrt() * w.view(1, -1, 1, 1) + b.view(1, -1, 1, 1)


def _upstream_nafnet64(sd, enc, mid, dec, x, tlc_kernel):
    """Unfolded NAFNetLocal in float64, written from the upstream block definition (NCHW,
    LayerNorm2d, depthwise conv, SimpleGate, local-average-pool SCA, beta / gamma residuals)."""
    sd = {k: v.double() for k, v in sd.items()}

    def local_mean(t, k):
        kh, kw = min(t.shape[2], k[0]), min(t.shape[3], k[1])
        m = F.avg_pool2d(t, (kh, kw), stride=1)
        ph, pw = t.shape[2] - m.shape[2], t.shape[3] - m.shape[3]
        return F.pad(m, (pw // 2, pw - pw // 2, ph // 2, ph - ph // 2), mode="replicate")

    def block(t, p, level):
        y = _layernorm2d(t, sd[f"{p}.norm1.weight"], sd[f"{p}.norm1.bias"])
        y = F.conv2d(y, sd[f"{p}.conv1.weight"], sd[f"{p}.conv1.bias"])
        y = F.conv2d(y, sd[f"{p}.conv2.weight"], sd[f"{p}.conv2.bias"], padding=1, groups=y.shape[1])
        a, b = y.chunk(2, 1)
        y = a * b
        y = y * F.conv2d(local_mean(y, tlc_kernel(level)), sd[f"{p}.sca.1.weight"], sd[f"{p}.sca.1.bias"])
        y = F.conv2d(y, sd[f"{p}.conv3.weight"], sd[f"{p}.conv3.bias"])
        t2 = t + y * sd[f"{p}.beta"]
        y = _layernorm2d(t2, sd[f"{p}.norm2.weight"], sd[f"{p}.norm2.bias"])
        y = F.conv2d(y, sd[f"{p}.conv4.weight"], sd[f"{p}.conv4.bias"])
        a, b = y.chunk(2, 1)
        y = F.conv2d(a * b, sd[f"{p}.conv5.weight"], sd[f"{p}.conv5.bias"])
        return t2 + y * sd[f"{p}.gamma"]

    inp = x.double()
    t = F.conv2d(inp, sd["intro.weight"], sd["intro.bias"], padding=1)
    skips = []
    for i, n in enumerate(enc):
        for j in range(n):
            t = block(t, f"encoders.{i}.{j}", i)
        skips.append(t)
        t = F.conv2d(t, sd[f"downs.{i}.weight"], sd[f"downs.{i}.bias"], stride=2)
    for j in range(mid):
        t = block(t, f"middle_blks.{j}", len(enc))
    for i, n in enumerate(dec):
        t = F.pixel_shuffle(F.conv2d(t, sd[f"ups.{i}.0.weight"]), 2)
        t = t + skips[len(enc) - 1 - i]
        for j in range(n):
            t = block(t, f"decoders.{i}.{j}", len(enc) - 1 - i)
    return F.conv2d(t, sd["ending.weight"], sd["ending.bias"], padding=1) + inp


def test_nafnet_harness_vs_unfolded_float64():
    from clarus_amd.nafnet import NAFNet, random_state_dict
    enc, mid, dec = [1, 1], 1, [1, 1]
    sd = random_state_dict(8, enc, mid, dec, seed=3)
    ops = Ops(["oracle_by_path"], torch.float32, torch.device("cpu"), log=lambda *a: None)
    model = NAFNet(ops, width=8, enc=enc, mid=mid, dec=dec, tlc=(33, 33), state_dict=sd)
    x = torch.rand(1, 3, 32, 48, generator=torch.Generator().manual_seed(1))
    got = model.forward(x)
    ref = _upstream_nafnet64(sd, enc, mid, dec, x, model.tlc_kernel)
    err = ((got.double() - ref).abs().max() / ref.abs().max()).item()
    assert err < 1e-5, err


def test_nafnet_tlc_windows_known_answer():
    """train 33 with two levels: windows (53, 53), (26, 26), (13, 13)
    (tools/test_model_contracts.py:159-160)."""
    from clarus_amd.nafnet import NAFNet
    ops = Ops(["oracle_by_path"], torch.float32, torch.device("cpu"), log=lambda *a: None)
    m = NAFNet(ops, width=4, enc=[1, 1], mid=1, dec=[1, 1], tlc=(33, 33))
    assert {m.tlc_kernel(level) for level in range(3)} == {(53, 53), (26, 26), (13, 13)}
    # NAFNet-GoPro-w64 at train 256: 384 / 192 / 96 / 48 / 24 per level
    m64 = NAFNet(ops, width=4, enc=[1, 1, 1, 1], mid=1, dec=[1, 1, 1, 1])
    assert [m64.tlc_kernel(level)[0] for level in range(5)] == [384, 192, 96, 48, 24]


@pytest.mark.parametrize("gate", [False, True])
def test_ln_gemm_weight_packing_matches_header(gate):
    """HipOps._frag_pack (torch gather / permute; the packing of _w2p and _wr_pack) against the
    fragment order clarus_hip_gemm_ln_gemm documents in include/clarus_hip.h, evaluated element by
    element at sampled positions:
    packed[P][w][s][b][l][e] = W^T[row(P, 64 w + 32 b + l % 32)][16 s + 8 (l / 32) + e]."""
    from clarus_amd.hip_ops import HipOps

    n2w = 1024
    w = torch.randn(512, n2w, generator=torch.Generator().manual_seed(5))
    packed = HipOps._frag_pack(w, gate).reshape(-1)
    assert packed.numel() == n2w * 512
    wt = w.t()
    rng = np.random.default_rng(0)
    for _ in range(3000):
        P, wv, s, b, l, e = (int(rng.integers(0, m)) for m in (n2w // 512, 8, 32, 2, 64, 8))
        i = l % 32
        j = 16 * ((i // 4) % 2) + 4 * (i // 8) + i % 4
        row = b * (n2w // 2) + 256 * P + 32 * wv + j if gate else 512 * P + 64 * wv + 32 * b + j
        flat = ((((P * 8 + wv) * 32 + s) * 2 + b) * 64 + l) * 8 + e
        assert packed[flat].item() == wt[row, 16 * s + 8 * (l // 32) + e].item()
    # every W^T element lands exactly once
    assert torch.equal(packed.sort().values, w.reshape(-1).sort().values)


@pytest.mark.parametrize("gate,n", [(True, 128), (True, 256), (False, 96), (False, 256), (False, 1024)])
def test_wr_weight_padding(gate, n):
    """HipOps._wr_pack: the weight padded with zero columns (gate: each half to a multiple of 256,
    else to a multiple of 512) before the fragment packing, so the packed halves of a gated weight
    start at row 256 * ceil(n / 256) and the padding rows are zero."""
    from clarus_amd.hip_ops import HipOps

    class Stub:
        _frag_pack = staticmethod(HipOps._frag_pack)

        def cached(self, t, tag, fn):
            return fn(t)

    k = 128
    w = torch.randn(k, 2 * n if gate else n, generator=torch.Generator().manual_seed(6)) + 3  # no zeros
    packed = HipOps._wr_pack(Stub(), w, gate)
    half = -(-n // 256) * 256
    nw = 2 * half if gate else -(-n // 512) * 512
    assert packed.numel() == k * nw
    wt = torch.zeros(nw, k)
    if gate:
        wt[:n], wt[half:half + n] = w[:, :n].t(), w[:, n:].t()
    else:
        wt[:n] = w.t()
    assert torch.equal(packed, HipOps._frag_pack(wt.t().contiguous(), gate))
    assert int((packed == 0).sum()) == k * (nw - (2 * n if gate else n))


def _mfma32(a_lanes: np.ndarray, b_lanes: np.ndarray) -> np.ndarray:
    """A 32x32 MFMA as the lanes feed it: lane l supplies A[l % 32][kp (l // 32) + i] and
    B[kp (l // 32) + i][l % 32] for its kp values (kp = 8 for 32x32x16 bf16, 1 for 32x32x2 fp32);
    returns the lanes' accumulator elements, lane l element j = D[8 (j // 4) + 4 (l // 32) + j % 4][l % 32]."""
    kp = a_lanes.shape[1]
    a = np.zeros((32, 2 * kp))
    b = np.zeros((2 * kp, 32))
    for l in range(64):
        a[l % 32, kp * (l // 32):kp * (l // 32) + kp] = a_lanes[l]
        b[kp * (l // 32):kp * (l // 32) + kp, l % 32] = b_lanes[l]
    d = a @ b
    return np.array([[d[8 * (j // 4) + 4 * (l // 32) + j % 4, l % 32] for j in range(16)] for l in range(64)])


@pytest.mark.parametrize("c,kp", [(32, 8), (64, 8), (128, 8), (32, 1), (64, 1)])
def test_ffn_fragment_packing(c, kp):
    """clarus_hip_ffn's data flow, emulated lane by lane on the packed weights (HipOps._ffn_pack1 /
    _ffn_pack2) with 32x32 MFMAs as the lanes feed them (kp = 8: the bf16 instructions, kp = 1: the
    fp32 ones, 8 / 16 per fragment): the gated accumulators of the first product used directly as
    the second product's B operand, the residual taken from the lane's own x fragments and the
    output channel of each element as the kernel stores it. In exact arithmetic this must equal
    x + scale * (SG(x w1 + b1) w2 + b2) for one 32-pixel unit; a wrong k order in w2p, a wrong
    output permutation or a wrong residual slot fails it."""
    from clarus_amd.hip_ops import HipOps
    g = torch.Generator().manual_seed(11)
    x = torch.randn(32, c, generator=g, dtype=torch.float64)
    w1 = torch.randn(c, 2 * c, generator=g, dtype=torch.float64)
    w2 = torch.randn(c, c, generator=g, dtype=torch.float64)
    b1 = torch.randn(2 * c, generator=g, dtype=torch.float64)
    b2 = torch.randn(c, generator=g, dtype=torch.float64)
    sc = torch.randn(c, generator=g, dtype=torch.float64)
    h = x @ w1 + b1
    want = (x + sc * ((h[:, :c] * h[:, c:]) @ w2 + b2)).numpy()
    w1p, w2p = HipOps._ffn_pack1(w1).numpy(), HipOps._ffn_pack2(w2).numpy()
    assert w1p.shape == (2 * c // 32, c // 16, 64, 8) and w2p.shape == (c // 32, c // 32, 64, 16)
    xn = x.numpy()
    lanes = np.arange(64)
    # x fragment s of lane l: channels 16 s + 8 (l // 32) .. + 7 of pixel l % 32
    xf = np.stack([np.stack([xn[l % 32, 16 * s + 8 * (l // 32):16 * s + 8 * (l // 32) + 8] for l in lanes])
                   for s in range(c // 16)])                                  # [s, 64, 8]

    def product(wfr, bfr):  # wfr / bfr: [64, 8 * n] lane operands, fed kp values per instruction
        acc = np.zeros((64, 16))
        for q in range(0, wfr.shape[1], kp):
            acc += _mfma32(wfr[:, q:q + kp], bfr[:, q:q + kp])
        return acc

    tg = c // 32
    u = []
    for t in range(tg):
        ga = product(np.concatenate([w1p[t, s] for s in range(c // 16)], 1), np.concatenate(list(xf), 1))
        gb = product(np.concatenate([w1p[t + tg, s] for s in range(c // 16)], 1), np.concatenate(list(xf), 1))
        hid = np.array([[32 * t + 8 * (j // 4) + 4 * (l // 32) + j % 4 for j in range(16)] for l in lanes])
        u.append((ga + b1.numpy()[hid]) * (gb + b1.numpy()[c + hid]))
    got = np.zeros((32, c))
    for t2 in range(tg):
        acc = product(np.concatenate([w2p[t2, t] for t in range(tg)], 1), np.concatenate(u, 1))
        for l in lanes:
            for j in range(16):
                ch = 32 * t2 + 16 * (j // 8) + 8 * (l // 32) + j % 8
                res = xf[2 * t2 + j // 8, l, j % 8]
                assert res == xn[l % 32, ch]
                got[l % 32, ch] = (acc[l, j] + b2.numpy()[ch]) * sc.numpy()[ch] + res
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10 * np.abs(want).max())  # fp64 summation order


def test_ln_dw_fragment_packing():
    """clarus_hip_ln_gemm_dwconv's 1x1 conv, emulated lane by lane on the packed weight
    (HipOps._ln_dw_pack) with 32x32x16 MFMAs as the lanes feed them: B operand = the lane's x
    fragments (pixel l % 32, channels 16 s + 8 (l // 32) ..), accumulator element j of output block
    T = channel 32 T + 16 (j // 8) + 8 (l // 32) + j % 8 of the lane's pixel, as the kernel writes
    the t tile. Exact arithmetic must give x w for one 32-pixel row."""
    from clarus_amd.hip_ops import HipOps
    g = torch.Generator().manual_seed(13)
    x = torch.randn(32, 64, generator=g, dtype=torch.float64)
    w = torch.randn(64, 128, generator=g, dtype=torch.float64)
    want = (x @ w).numpy()
    wp = HipOps._ln_dw_pack(w).numpy()
    assert wp.shape == (4, 4, 64, 8)
    xn = x.numpy()
    xf = np.concatenate([np.stack([xn[l % 32, 16 * s + 8 * (l // 32):16 * s + 8 * (l // 32) + 8] for l in range(64)])
                         for s in range(4)], 1)  # [64, 32]: step s in columns 8 s .. 8 s + 7
    got = np.zeros((32, 128))
    for t in range(4):
        wt = np.concatenate([wp[t, s] for s in range(4)], 1)
        acc = sum(_mfma32(wt[:, q:q + 8], xf[:, q:q + 8]) for q in range(0, 32, 8))
        for l in range(64):
            for j in range(16):
                got[l % 32, 32 * t + 16 * (j // 8) + 8 * (l // 32) + j % 8] = acc[l, j]
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10 * np.abs(want).max())


def test_linear_gate_linear_unfused_is_two_linears():
    """Backends without the fused kernel run linear_gate_linear as its two linear ops: the gated
    LN GEMM, then the second GEMM with the scale and the input as residual."""
    calls = []

    class B(Backend):
        name = "rec2"

        def linear(self, x, w, bias=None, **kw):
            calls.append(kw)
            y = x @ w
            return y[:, :4] * y[:, 4:] if kw.get("gate") else y

    b = B(torch.float32, torch.device("cpu"))
    x, w1, w2, sc = torch.randn(3, 4), torch.randn(4, 8), torch.randn(4, 4), torch.randn(4)
    out = b.linear_gate_linear(x, w1, None, w2, None, scale=sc, ln="rms", ln_eps=1e-5, out_dtype=torch.float32)
    h = x @ w1
    assert torch.equal(out, (h[:, :4] * h[:, 4:]) @ w2)
    assert calls[0] == {"ln": "rms", "gate": True, "ln_eps": 1e-5}
    assert calls[1]["residual"] is x and calls[1]["scale"] is sc and calls[1]["out_dtype"] == torch.float32


def test_linear_ln_linear_unfused_is_two_linears():
    """Backends without the fused kernel run linear_ln_linear as the two ops."""
    calls = []

    class B(Backend):
        name = "rec"

        def linear(self, x, w, bias=None, **kw):
            calls.append(kw)
            return x @ w

    b = B(torch.float32, torch.device("cpu"))
    x, w1, w2 = torch.randn(3, 4), torch.randn(4, 4), torch.randn(4, 6)
    y, u = b.linear_ln_linear(x, w1, residual=x, w2=w2, gate2=True, ln="rms", ln_eps=1e-5)
    assert torch.equal(y, x @ w1) and torch.equal(u, (x @ w1) @ w2)
    assert calls[0]["residual"] is x and calls[1] == {"ln": "rms", "gate": True, "ln_eps": 1e-5}


def test_pair_default_for_a_host_backend_base():
    """Inside a clarus installation Backend is clarus's own class, which has no linear_ln_linear:
    the two-linear default is attached to it, so every backend answers the op."""
    class HostBase:  # a host's backend base without the op
        def __init__(self, dtype, device):
            self.dtype, self.device = dtype, device

    dispatch.give_pair_default(HostBase)
    assert HostBase.linear_ln_linear is dispatch.linear_ln_linear_unfused
    assert HostBase.linear_gate_linear is dispatch.linear_gate_linear_unfused
    assert HostBase.linear_dwconv is dispatch.linear_dwconv_unfused

    class Own(HostBase):
        def linear_ln_linear(self, *a, **k):
            return "own"
    dispatch.give_pair_default(Own)  # a class with its own op keeps it
    assert Own(torch.float32, "cpu").linear_ln_linear() == "own"


class _PlainOracle:
    """A backend that does not derive from Backend and has no linear_ln_linear."""
    name = "plain_oracle"

    def __init__(self, dtype, device):
        self.dtype, self.device = dtype, device
        self._r = TorchRef(dtype, device)

    def __getattr__(self, op):
        if op.startswith("_") or op in ("linear_ln_linear", "linear_gate_linear", "linear_dwconv"):
            raise AttributeError(op)
        return getattr(self._r, op)


def test_nafnet_pairs_match_the_reference_call_pattern():
    """The harness's fused calls (at the pair width: conv3 -> conv4, conv5 -> next conv1 in a
    stage of two blocks; at other widths the feed-forward half conv4 -> conv5) give exactly the
    reference block's five-linear result (fused_pairs=False) on the oracle, and the harness falls
    back to the linear calls when no backend has the fused ops."""
    from clarus_amd.nafnet import NAFNet, random_state_dict
    register_backend("plain_oracle")(_PlainOracle)
    enc, mid, dec = [2, 1], 2, [1, 2]
    sd = random_state_dict(8, enc, mid, dec, seed=4)
    x = torch.rand(1, 3, 24, 40, generator=torch.Generator().manual_seed(2))
    outs = []
    for backend, fused in (("oracle_by_path", True), ("oracle_by_path", False), ("plain_oracle", True)):
        ops = Ops([backend], torch.float32, torch.device("cpu"), log=lambda *a: None)
        model = NAFNet(ops, width=8, enc=enc, mid=mid, dec=dec, tlc=(24, 40), state_dict=sd, fused_pairs=fused)
        model.pair_width = 16  # the enc1 / dec0 width of this model (512 at NAFNet-w64 level 3)
        outs.append(model.forward(x))
        calls = ops.report()["ops"]
        for op in ("linear_ln_linear", "linear_gate_linear", "linear_dwconv"):
            assert (op in calls) == (fused and backend == "oracle_by_path"), (op, calls)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
