"""GPU: capture safety of the `hip` backend under clarus's worker discipline.

clarus's worker builds each static-shape entry on its own stream: buffers are allocated and
initialised there, the pipeline runs eagerly (weight re-layouts, scratch), and then it is
captured into a graph (python/clarus/worker.py:113-150). Its smoke test poisons the current
stream's allocator pool with NaN-filled freed blocks and keeps that stream busy before entries
are created lazily (tools/worker_smoke.py:93-102, 184-191): anything the backend allocated or
initialised on the wrong stream would then read poisoned memory, or be overwritten late.

Here: a fresh `hip` backend (empty weight caches) runs the NAFNet-w64 forward on a worker stream
while the default stream is stalled behind NaN-poisoned frees; the eager results and every graph
replay (interleaved with eager work and host synchronisations) must equal the forward computed
beforehand on a clean backend, bit for bit.
"""
from __future__ import annotations

import pytest
import torch

from clarus_amd import spatial_torch  # noqa: F401  (registers "torch" for the non-GEMM ops)
from clarus_amd.dispatch import Ops
from clarus_amd.nafnet import NAFNet

pytestmark = pytest.mark.gpu


def _poison_and_stall(dev):
    """NaN-filled blocks freed into the current stream's pool, then ~0.2 s of queued spinning on
    that stream (no host synchronisation)."""
    junk = [torch.full((1 << 17,), float("nan"), device=dev) for _ in range(64)]  # 64 x 512 KiB
    junk += [torch.full((1 << 24,), float("nan"), device=dev) for _ in range(4)]  # 4 x 64 MiB
    del junk
    torch.cuda._sleep(int(4e8))


@pytest.mark.parametrize("fused_pairs", [True, False])
def test_nafnet_lazy_capture_on_worker_stream(fused_pairs, gpu_device):
    dev = gpu_device
    g = torch.Generator().manual_seed(5)
    x = torch.rand(1, 3, 192, 320, generator=g).to(dev)
    clean = NAFNet(Ops(["hip", "torch"], torch.bfloat16, dev, log=print), seed=0, fused_pairs=fused_pairs)
    ref = clean.forward(x).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()

    ops = Ops(["hip", "torch"], torch.bfloat16, dev, log=print)  # fresh backend: nothing cached yet
    model = NAFNet(ops, seed=0, fused_pairs=fused_pairs)
    torch.cuda.synchronize()
    print(f"[capture] fused_pairs={fused_pairs}: poison + stall the default stream", flush=True)
    _poison_and_stall(dev)
    worker = torch.cuda.Stream(dev)
    pool = torch.cuda.graph_pool_handle()
    with torch.cuda.stream(worker):
        inp = torch.zeros_like(x)  # allocated and initialised on the worker stream
        inp.copy_(x)
        eager = model.forward(inp).clone()  # lazy weight re-layouts and scratch, on the worker stream
        eager2 = model.forward(inp).clone()
        worker.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=pool, stream=worker):
            y = model.forward(inp)
    torch.cuda.synchronize()
    assert torch.equal(eager, ref), f"eager on the worker stream: max|d| {(eager - ref).abs().max().item():.3e}"
    assert torch.equal(eager2, ref)
    served = ops.report()["ops"]
    for op in ("linear", "down", "up", "intro", "ending", "dwconv", "boxmean") + (("linear_ln_linear",) if fused_pairs else ()):
        assert list(served.get(op, {})) == ["hip"], (op, served.get(op))
    for rep in range(3):
        with torch.cuda.stream(worker):
            graph.replay()
        worker.synchronize()
        assert torch.equal(y, ref), f"replay {rep}: max|d| {(y - ref).abs().max().item():.3e}"
        _poison_and_stall(dev)  # poison again between replays; the graph's memory is its own pool's
        with torch.cuda.stream(worker):
            z = model.forward(inp)
        torch.cuda.synchronize()
        assert torch.equal(z, ref), f"eager forward after replay {rep} differs"
