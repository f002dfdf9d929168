"""GPU: clarus_hip_channel_attention_noalloc (static device scratch, no allocation) against
clarus_hip_channel_attention (caller workspace), both called through the C ABI.

Two calls in a row on the same device, the second on a smaller input, so the second call
runs on partials the first one left in the shared static array; both must equal the workspace
entry point's output bit for bit (same kernels, fixed summation order). The size limit is
checked on the host before anything launches (tests/test_abi.py covers it without a GPU).
The no-allocation property itself: the device's free memory (hipMemGetInfo through torch) is
the same before and after further calls, and the call captured in a HIP graph replays to the
same result.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from clarus_amd import _lib

pytestmark = pytest.mark.gpu


def _with_workspace(lib, qkv, temp, n, hw, c, heads):
    out = torch.empty((n, heads, c // heads, c // heads), dtype=torch.float32, device=qkv.device)
    need = lib.clarus_hip_channel_attention_workspace(n, hw, c, heads)
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=qkv.device)  # the counters start at zero
    _lib.check(lib.clarus_hip_channel_attention(qkv.data_ptr(), _lib.dtype_code(qkv.dtype), temp.data_ptr(),
                                                out.data_ptr(), n, hw, c, heads, ws.data_ptr(), ws.numel(),
                                                torch.cuda.current_stream().cuda_stream), "channel_attention")
    return out


def _no_alloc(lib, qkv, temp, n, hw, c, heads):
    out = torch.empty((n, heads, c // heads, c // heads), dtype=torch.float32, device=qkv.device)
    _lib.check(lib.clarus_hip_channel_attention_noalloc(qkv.data_ptr(), _lib.dtype_code(qkv.dtype), temp.data_ptr(),
                                                        out.data_ptr(), n, hw, c, heads,
                                                        torch.cuda.current_stream().cuda_stream),
               "channel_attention_noalloc")
    return out


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_channel_attention_noalloc_matches_workspace_entry(dt, gpu_device):
    lib = _lib.load()
    g = torch.Generator().manual_seed(5)
    # (batch, h, w, c, heads): Restormer level 1 at 720p (2 heads of 48), then a smaller ragged
    # case with 4 heads of 24 over 2 images
    cases = [(1, 360, 640, 96, 2), (2, 37, 53, 96, 4)]
    for n, h, w, c, heads in cases:
        print(f"[noalloc] {dt} batch {n} {h}x{w} c {c} heads {heads}", flush=True)
        need = lib.clarus_hip_channel_attention_workspace(n, h * w, c, heads)
        assert 0 < need <= _lib.CHANNEL_ATTENTION_SCRATCH_MAX
        qkv = torch.randn(n, h, w, 3 * c, generator=g).to(dt).to(gpu_device)
        temp = (torch.rand(heads, generator=g) * 1.5 + 0.5).to(gpu_device)
        want = _with_workspace(lib, qkv, temp, n, h * w, c, heads)
        got = _no_alloc(lib, qkv, temp, n, h * w, c, heads)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), (got - want).abs().max().item()
        # rows of a softmax sum to one (catches a result read from stale partials that happens to
        # match a stale workspace too)
        assert torch.allclose(got.sum(-1), torch.ones_like(got.sum(-1)), atol=1e-5)


def test_channel_attention_noalloc_allocates_nothing(gpu_device):
    lib = _lib.load()
    g = torch.Generator().manual_seed(6)
    n, h, w, c, heads = 1, 180, 320, 192, 4
    qkv = torch.randn(n, h, w, 3 * c, generator=g).bfloat16().to(gpu_device)
    temp = (torch.rand(heads, generator=g) * 1.5 + 0.5).to(gpu_device)
    want = _with_workspace(lib, qkv, temp, n, h * w, c, heads)
    out = torch.empty_like(want)

    def call():
        _lib.check(lib.clarus_hip_channel_attention_noalloc(qkv.data_ptr(), _lib.dtype_code(qkv.dtype),
                                                            temp.data_ptr(), out.data_ptr(), n, h * w, c, heads,
                                                            torch.cuda.current_stream().cuda_stream),
                   "channel_attention_noalloc")
    call()  # the first call on the device resolves the static array's address
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(gpu_device)[0]
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info(gpu_device)[0]
    print(f"[noalloc] device free bytes before {free0}, after {free1}", flush=True)
    assert free1 == free0 and torch.equal(out, want)
    # captured in a HIP graph (no allocation may happen inside a capture) and replayed
    side = torch.cuda.Stream(gpu_device)
    side.wait_stream(torch.cuda.current_stream(gpu_device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call()
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
    assert torch.cuda.mem_get_info(gpu_device)[0] >= free1 - (64 << 20)  # the graph object itself only
