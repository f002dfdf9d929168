"""GPU: the NAFNet-w64 forward on `hip` captured in one HIP graph and replayed.

Every kernel here has a fixed reduction order and the library records no memset nodes, so each
replay must reproduce the eager forward bit for bit; the replays are interleaved with eager work
and host synchronisations (a graph replayed once can hide state that only a later replay
exposes). The captured forward includes the fused residual GEMM -> LayerNorm -> GEMM pairs
(clarus_hip_gemm_ln_gemm) and their packed second weights, which the eager warm-up builds.
"""
from __future__ import annotations

import pytest
import torch

from clarus_amd import spatial_torch  # noqa: F401  (registers "torch" for the non-GEMM ops)
from clarus_amd.dispatch import Ops
from clarus_amd.nafnet import NAFNet

pytestmark = pytest.mark.gpu


def test_nafnet_graph_replays_match_eager(gpu_device):
    dev = gpu_device
    ops = Ops(["hip", "torch"], torch.bfloat16, dev, log=print)
    assert "hip" in ops.by_name, ops.skipped
    model = NAFNet(ops, seed=0)
    g = torch.Generator().manual_seed(3)
    x = torch.rand(1, 3, 192, 320, generator=g).to(dev)
    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        eager = model.forward(x).clone()  # warm-up: weight re-layouts
        eager2 = model.forward(x).clone()
    torch.cuda.synchronize()
    assert torch.equal(eager, eager2), "eager forwards differ"
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y = model.forward(x)
    torch.cuda.synchronize()
    served = ops.report()["ops"]
    for op in ("linear", "linear_ln_linear"):
        assert list(served.get(op, {})) == ["hip"], (op, served.get(op))
    assert ops.by_name["hip"].pair_launches["gemm_ln_gemm"] > 0
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep}: max|d| {(y - eager).abs().max().item():.3e}"
        # eager work between replays on the same buffers' allocator
        z = model.forward(x)
        torch.cuda.synchronize()
        assert torch.equal(z, eager), f"eager forward after replay {rep} differs"
