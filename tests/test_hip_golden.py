"""GPU: the `hip` backend against golden vectors written by the reference implementation
(tests/golden/make_golden.py; the CPU side of the same fixtures is tests/test_golden.py).

* The tiny NAFNetLocal forward (the reference model adapter on its PyTorch backend) run through
  clarus_amd.nafnet.NAFNet on `hip`: fp32 activations within 1e-5 of the output scale; bf16
  activations with |dPSNR| <= 1e-3 dB against a synthetic target (north star), and every
  GEMM-family op, the depthwise conv and the box mean served by `hip`.
* The reference's linear_patch_filter calls on `hip`: fp32 within 1e-5 relative, bf16 outputs by the
  bf16 rule against the oracle's fp32 value before the final cast (the fixture rounds to it).
* The reference's combined-epilogue TorchOps calls on `hip`: fp32 backends within 1e-5
  relative, bf16 backends within 1e-5 relative where the reference output is fp32 and by the
  bf16 rule (2e-2 absolute, rounding flips allowed) where it is bf16.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from clarus_amd import spatial_torch  # noqa: F401  (registers "torch" for pixel (un)shuffle etc.)
from clarus_amd.dispatch import Ops, Unsupported
from clarus_amd.nafnet import psnr
from oracle.torch_ref import Small, TorchRef
from tests._tol import assert_bf16, assert_fp32
from tests.test_golden import (DT, load_freq_fixture, load_nafnet_fixture, load_ops_fixture, run_combined,
                               run_linear_patch_filter, tiny_nafnet)

pytestmark = pytest.mark.gpu

HIP_OPS = {"linear", "down", "up", "intro", "ending", "dwconv", "boxmean"}


@pytest.mark.parametrize("tag", ["fp32", "bf16"])
def test_hip_nafnet_tiny_vs_reference(tag, gpu_device):
    tiny, sd, t = load_nafnet_fixture()
    print(f"[golden] NAFNet tiny {tag}", flush=True)
    ops = Ops(["hip", "torch"], DT[tag], gpu_device, log=print)
    assert "hip" in ops.by_name, ops.skipped
    y = tiny_nafnet(ops, tiny, sd).forward(t["input"].to(gpu_device)).float().cpu()
    torch.cuda.synchronize()
    ref = t[f"out_{tag}"]
    served = ops.report()["ops"]
    for op in HIP_OPS:
        assert list(served.get(op, {"hip": 0})) == ["hip"], (op, served.get(op))
    if tag == "fp32":
        e = assert_fp32(y, ref, what="NAFNet tiny fp32")
        print(f"[golden] NAFNet tiny fp32 rel err {e:.2e}")
        return
    x = t["input"]
    gt = F.avg_pool2d(x, 3, stride=1, padding=1, count_include_pad=False)
    p_hip, p_ref = psnr(y.clamp(0, 1), gt), psnr(ref.clamp(0, 1), gt)
    print(f"[golden] NAFNet tiny bf16: PSNR hip {p_hip:.6f} ref {p_ref:.6f} |d| {abs(p_hip - p_ref):.2e} "
          f"max|dy| {(y - ref).abs().max().item():.3e}")
    assert abs(p_hip - p_ref) <= 1e-3


@pytest.mark.parametrize("tag", ["fp32", "bf16"])
def test_hip_combined_ops_vs_reference(tag, gpu_device):
    t = load_ops_fixture()
    print(f"[golden] combined ops {tag}", flush=True)
    ops = Ops(["hip"], DT[tag], gpu_device, log=print)
    assert "hip" in ops.by_name, ops.skipped
    got = run_combined(ops, t, tag, gpu_device)
    torch.cuda.synchronize()
    for case, y in got.items():
        ref = t[f"{case}_{tag}.y"]
        assert y.dtype == ref.dtype and y.shape == ref.shape, case
        if ref.dtype == torch.float32:
            e = assert_fp32(y.cpu(), ref, what=f"{case} {tag}")
            print(f"[golden] {case} {tag} rel err {e:.2e}")
        else:
            # the one bf16-output case (lin2) is judged against the oracle's fp32 value before
            # its cast; that value rounds to the fixture bit for bit
            a = {k.split(".")[1]: v for k, v in t.items() if k.startswith(f"{case}_{tag}.")}
            r32 = TorchRef(DT[tag], "cpu").linear(a["x"], a["w"], a["b"], ln="rms", scale=a["s"],
                                                  residual=a["res"], out_dtype=torch.float32)
            assert case == "lin2" and torch.equal(r32.to(ref.dtype), ref)
            d, flips = assert_bf16(y.cpu(), r32, what=f"{case} {tag}")
            print(f"[golden] {case} {tag} max|d| {d:.2e} flips {flips}")


def test_hip_declines_ln_with_mul_like_the_reference(gpu_device):
    """LayerNorm and TLC-map prologues together go to the next backend, as in the reference's
    Triton adapter (python/clarus/ops/triton_cuda.py:88-89)."""
    t = load_ops_fixture()
    ops = Ops(["hip"], torch.float32, gpu_device, log=print)
    g = {k.split(".")[1]: v.to(gpu_device) for k, v in t.items() if k.startswith("lin1_fp32.")}
    with pytest.raises(Unsupported):
        ops.linear(g["x"], g["w"], g["b"], ln=True, gate=True, mul=Small(g["map"], 2, 3, 9, 13))


@pytest.mark.parametrize("tag", ["fp32", "bf16"])
def test_hip_linear_patch_filter_vs_reference(tag, gpu_device):
    print(f"[golden] linear_patch_filter {tag}", flush=True)
    ops = Ops(["hip"], DT[tag], gpu_device, log=print)
    assert "hip" in ops.by_name, ops.skipped
    for key, (a, ln) in load_freq_fixture().items():
        if not key.endswith(tag):
            continue
        y = run_linear_patch_filter(ops, a, ln, gpu_device).cpu()
        ref = a["y"]
        assert y.dtype == ref.dtype and y.shape == ref.shape, key
        if tag == "fp32":
            e = assert_fp32(y, ref, what=key)
            print(f"[golden] {key} rel err {e:.2e}")
        else:
            # the oracle's fp32 value before the cast, on this host's CPU: the fixture (written on
            # another CPU, whose summation order may differ in the last fp32 bits) must be a
            # rounding of it up to rounding flips; tests/test_golden.py pins it bit for bit
            r32 = run_linear_patch_filter(TorchRef(DT[tag], "cpu"), a, ln, "cpu", out_fp32=True)
            assert_bf16(ref, r32, what=key + " (fixture vs this host's oracle)")
            d, flips = assert_bf16(y, r32, what=key)
            print(f"[golden] {key} max|d| {d:.2e} flips {flips}")
    assert list(ops.report()["ops"]["linear_patch_filter"]) == ["hip"]
