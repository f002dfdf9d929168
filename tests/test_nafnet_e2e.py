"""GPU: NAFNet-GoPro-w64 (NAFNetLocal, enc [1, 1, 1, 28], mid 1, dec [1, 1, 1, 1]) forward at
720p in bf16, the GEMM-family ops on the HIP backend, against the same harness running every op
on the oracle (the reference PyTorch backend's semantics) on the GPU.

Criterion (north star): PSNR of the restored image against a synthetic ground truth agrees
within 1e-3 dB between the two op chains; the outputs also agree to a small max difference.
Every GEMM-family op of the forward must have been served by `hip`. With the harness's fused
calls, every level-3 pair (linear_ln_linear) must have run as one fused kernel: 29 conv3 -> conv4
pairs (28 encoder blocks and one decoder block at width 512) and 27 conv5 -> next conv1 pairs
(within the 28-block encoder stage), 56 per forward; and so must the feed-forward half
(linear_gate_linear) of the level-0 and level-1 blocks (widths 64 and 128), 4 per forward, and
the level-0 conv1 -> depthwise conv (linear_dwconv), 2 per forward. The reference's unchanged
block (five linear calls, fused_pairs=False) is held to the same PSNR criterion.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from clarus_amd import spatial_torch  # noqa: F401  (registers "torch" for the non-GEMM ops)
from clarus_amd.dispatch import Backend, Ops, register_backend
from clarus_amd.nafnet import NAFNet, psnr
from oracle.torch_ref import TorchRef

pytestmark = pytest.mark.gpu

GEMM_OPS = {"linear", "down", "up", "intro", "ending"}
FUSED_PAIRS_PER_FORWARD = 29 + 27
FUSED_FFN_PER_FORWARD = 4  # levels 0 and 1: encoder block and decoder block each
FUSED_LN_DW_PER_FORWARD = 2  # level 0 conv1 -> depthwise conv: encoder block and decoder block


class _OracleBackend(Backend):
    name = "oracle"

    def __init__(self, dtype, device):
        super().__init__(dtype, device)
        self._r = TorchRef(dtype, device)

    def __getattr__(self, op):
        if op.startswith("_"):
            raise AttributeError(op)
        return getattr(self._r, op)


@pytest.mark.parametrize("h,w,fused", [(256, 384, True), (720, 1280, True), (720, 1280, False)])
def test_nafnet_w64_psnr_parity(h, w, fused, gpu_device):
    register_backend("oracle")(_OracleBackend)
    dev = gpu_device
    ops_hip = Ops(["hip", "torch"], torch.bfloat16, dev, log=print)
    assert "hip" in ops_hip.by_name, ops_hip.skipped
    ops_ref = Ops(["oracle"], torch.bfloat16, dev, log=print)
    m_hip = NAFNet(ops_hip, seed=0, fused_pairs=fused)
    m_ref = NAFNet(ops_ref, seed=0)
    print(f"[e2e] NAFNet-w64 {h}x{w} fused_pairs={fused}", flush=True)
    g = torch.Generator().manual_seed(7)
    x = torch.rand(1, 3, h, w, generator=g).to(dev)
    gt = F.avg_pool2d(x, 3, stride=1, padding=1, count_include_pad=False)  # synthetic target
    y_hip = m_hip.forward(x).float()
    y_ref = m_ref.forward(x).float()
    assert torch.isfinite(y_hip).all() and torch.isfinite(y_ref).all()
    p_hip = psnr(y_hip.clamp(0, 1), gt)
    p_ref = psnr(y_ref.clamp(0, 1), gt)
    diff = (y_hip - y_ref).abs().max().item()
    print(f"NAFNet-w64 {h}x{w}: PSNR hip {p_hip:.5f} dB, oracle {p_ref:.5f} dB, |dPSNR| {abs(p_hip - p_ref):.2e}, "
          f"max|dy| {diff:.3e}, output range [{y_ref.min().item():.3f}, {y_ref.max().item():.3f}]")
    served = ops_hip.report()["ops"]
    for op in GEMM_OPS | ({"linear_ln_linear", "linear_gate_linear", "linear_dwconv"} if fused else set()):
        assert list(served.get(op, {"hip": 0})) == ["hip"], (op, served.get(op))
    launches = ops_hip.by_name["hip"].pair_launches
    assert launches == {"gemm_ln_gemm": FUSED_PAIRS_PER_FORWARD if fused else 0, "gemm_ln_rows": 0}, launches
    assert ops_hip.by_name["hip"].ffn_launches == (FUSED_FFN_PER_FORWARD if fused else 0)
    assert ops_hip.by_name["hip"].ln_dw_launches == (FUSED_LN_DW_PER_FORWARD if fused else 0)
    assert ("linear_ln_linear" in served) == fused and ("linear_gate_linear" in served) == fused
    assert abs(p_hip - p_ref) <= 1e-3
