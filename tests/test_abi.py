"""CPU: the C-ABI library loads, exports every entry point include/clarus_hip.h declares, its
struct layouts match the ctypes binding, and argument validation rejects bad calls before any
launch (those calls never touch a GPU)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from clarus_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "clarus_hip.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(clarus_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} is not built: run __graft_entry__.build()")
    return _lib.load()


def test_header_declares_the_bound_functions():
    assert declared_functions() == sorted(_lib.SIGNATURES), "binding and header disagree"


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [f for f in declared_functions() if not hasattr(raw, f)]
    assert not missing, missing


def test_abi_version_and_struct_sizes(lib):
    assert lib.clarus_hip_abi_version() == _lib.ABI_VERSION
    assert lib.clarus_hip_sizeof_gemm_args() == ctypes.sizeof(_lib.GemmArgs)
    assert lib.clarus_hip_sizeof_conv_args() == ctypes.sizeof(_lib.ConvArgs)


def test_validation_rejects_before_launch(lib):
    assert lib.clarus_hip_gemm(None, None) == _lib.EINVAL
    assert b"null" in lib.clarus_hip_last_error()
    a = _lib.GemmArgs(a=16, wt=16, c=16, m=10, n=8, k=12, batch=1, lda=12, ldc=8)
    assert lib.clarus_hip_gemm(ctypes.byref(a), None) == _lib.EINVAL  # K % 8 != 0
    assert b"multiple of 8" in lib.clarus_hip_last_error()
    cv = _lib.ConvArgs(x=16, wt=16, out=16, batch=1, h=4, w=4, cin=12, cout=8, ldx=12, ldo=8)
    assert lib.clarus_hip_conv3x3(ctypes.byref(cv), None) == _lib.EINVAL  # cin % 8 != 0
    assert lib.clarus_hip_channel_attention(16, 1, 16, 16, 1, 64, 30, 2, 16, 0, None) == _lib.EINVAL
    # more heads than one launch's arrival counters cover (496), a workspace short of the size
    assert lib.clarus_hip_channel_attention(16, 1, 16, 16, 1, 64, 512 * 8, 512, 16, 1 << 30, None) == _lib.EINVAL
    assert b"heads" in lib.clarus_hip_last_error()
    need = lib.clarus_hip_channel_attention_workspace(1, 64, 96, 2)
    assert need > 64 * 1024  # the counters come first
    assert lib.clarus_hip_channel_attention(16, 1, 16, 16, 1, 64, 96, 2, 16, need - 16, None) == _lib.EINVAL
    assert b"scratch" in lib.clarus_hip_last_error()
    assert lib.clarus_hip_patch_corr(16, 0, 0, 0, 0, 16, 16, 16, 1, 12, 16, 8, None) == _lib.EINVAL  # h % 8
    a = _lib.GemmArgs(a=16, m=10, k=64, batch=1, lda=64, pro=0, a_dtype=_lib.BF16)
    assert lib.clarus_hip_rows_split(ctypes.byref(a), 16, None) == _lib.EINVAL  # bf16 rows, no prologue
    assert b"fp32" in lib.clarus_hip_last_error()
    a.pro = 9
    assert lib.clarus_hip_rows_prologue(ctypes.byref(a), 16, None) == _lib.EINVAL  # unknown prologue
    assert b"rows_prologue" in lib.clarus_hip_last_error()
    a = _lib.GemmArgs(a=16, wt=16, c=16, m=10, n=256, k=64, batch=1, lda=64, ldc=256,
                      a_dtype=_lib.BF16, w_dtype=_lib.BF16)
    assert lib.clarus_hip_gemm_ln_rows(ctypes.byref(a), 16, 1e-6, 0, None) == _lib.EINVAL  # N != 512
    assert b"512" in lib.clarus_hip_last_error()
    a.n, a.ldc = 512, 512
    assert lib.clarus_hip_gemm_ln_gemm(ctypes.byref(a), 1e-6, 0, 16, None, 16, 768, 1, None) == _lib.EINVAL  # n2w
    assert b"n2w" in lib.clarus_hip_last_error()
    a.k, a.lda, a.res, a.ldr, a.r_dtype = 512, 512, 16, 512, _lib.BF16
    assert lib.clarus_hip_gemm_ln_gemm_w1p(ctypes.byref(a), 16, 1e-6, 0, 16, None, 16, 1024, 1, None) == _lib.EINVAL
    assert b"fp32 residual" in lib.clarus_hip_last_error()
    a.r_dtype = _lib.F32
    assert lib.clarus_hip_gemm_ln_gemm_w1p(ctypes.byref(a), 16, 1e-6, 0, 16, None, 16, 768, 1, None) == _lib.EINVAL
    assert b"n2w" in lib.clarus_hip_last_error()
    a = _lib.GemmArgs(a=16, c=16, m=10, n=512, k=384, batch=1, lda=384, ldc=512, a_dtype=_lib.BF16,
                      w_dtype=_lib.BF16, c_dtype=_lib.BF16)
    assert lib.clarus_hip_gemm_wp(ctypes.byref(a), 16, None) == _lib.EINVAL  # K not 256 / 512 / 1024
    assert b"K = 256, 512 or 1024" in lib.clarus_hip_last_error()
    a.k, a.lda, a.n, a.ldc = 512, 512, 256, 256
    assert lib.clarus_hip_gemm_wp(ctypes.byref(a), 16, None) == _lib.EINVAL  # 256 W^T rows
    a.gate = 1
    a.pro = _lib.PRO_MUL
    assert lib.clarus_hip_gemm_wp(ctypes.byref(a), 16, None) == _lib.EINVAL  # a prologue other than LN / RMS
    assert b"LayerNorm / RMS without a residual" in lib.clarus_hip_last_error()
    a.pro, a.res, a.r_dtype, a.ldr = _lib.PRO_LN, 16, _lib.F32, 256
    assert lib.clarus_hip_gemm_wp(ctypes.byref(a), 16, None) == _lib.EINVAL  # LN with a residual
    assert b"LayerNorm / RMS without a residual" in lib.clarus_hip_last_error()
    a.pro, a.res = _lib.PRO_MUL, 0
    assert lib.clarus_hip_gemm_wp(ctypes.byref(a), 16, None) == _lib.EINVAL  # the map prologue without a residual
    assert b"map prologue with a residual" in lib.clarus_hip_last_error()
    a.res = 16
    assert lib.clarus_hip_gemm_wp(ctypes.byref(a), 16, None) == _lib.EINVAL  # ... without a map
    assert b"bf16 map" in lib.clarus_hip_last_error()
    a.pro, a.res, a.a_dtype = 0, 0, _lib.F32
    assert lib.clarus_hip_gemm_wp(ctypes.byref(a), 16, None) == _lib.EINVAL  # fp32 A
    assert b"bf16 A" in lib.clarus_hip_last_error()
    a = _lib.GemmArgs(a=16, c=16, m=64, n=256, k=512, batch=1, lda=512, ldc=256, a_dtype=_lib.BF16,
                      w_dtype=_lib.BF16, c_dtype=_lib.BF16)
    assert lib.clarus_hip_gemm_wr(ctypes.byref(a), 16, None) == _lib.EINVAL  # K = 512
    assert b"K = 128 or 256" in lib.clarus_hip_last_error()
    a.k, a.lda, a.res, a.ldr, a.r_dtype, a.gate, a.n = 256, 256, 16, 128, _lib.F32, 1, 128
    assert lib.clarus_hip_gemm_wr(ctypes.byref(a), 16, None) == _lib.EINVAL  # gated 128 with a residual
    assert b"residual" in lib.clarus_hip_last_error()
    a.gate, a.n, a.ldc, a.ldr = 0, 512, 512, 512
    assert lib.clarus_hip_gemm_wr(ctypes.byref(a), 16, None) == _lib.EINVAL  # fp32 residual, 512 outputs
    a.pro = _lib.PRO_LN
    assert lib.clarus_hip_gemm_wr(ctypes.byref(a), 16, None) == _lib.EINVAL  # LN with a residual
    assert b"LayerNorm / RMS without a residual" in lib.clarus_hip_last_error()
    a.pro, a.res = _lib.PRO_MUL, 0
    assert lib.clarus_hip_gemm_wr(ctypes.byref(a), 16, None) == _lib.EINVAL  # the map prologue without a map
    assert b"bf16 map" in lib.clarus_hip_last_error()
    a.gate = 1
    assert lib.clarus_hip_gemm_wr(ctypes.byref(a), 16, None) == _lib.EINVAL  # ... with the gate
    assert b"map prologue without the gate" in lib.clarus_hip_last_error()
    # clarus_hip_ffn: c, dtype, prologue, alignment and overlap are checked before any launch
    ffn = lib.clarus_hip_ffn
    assert ffn(16, 1 << 20, _lib.BF16, 16, None, 16, None, None, 64, 256, 1, 1e-6, 1.0, None) == _lib.EINVAL
    assert b"c = 32 or 64, or 128 in bf16" in lib.clarus_hip_last_error()
    assert ffn(16, 1 << 20, _lib.F32, 16, None, 16, None, None, 64, 128, 1, 1e-6, 1.0, None) == _lib.EINVAL
    assert ffn(16, 1 << 20, 7, 16, None, 16, None, None, 64, 64, 1, 1e-6, 1.0, None) == _lib.EINVAL
    assert ffn(16, 1 << 20, _lib.BF16, 16, None, 16, None, None, 64, 64, 2, 1e-6, 1.0, None) == _lib.EINVAL  # mul
    assert ffn(16, 1 << 20, _lib.BF16, 24, None, 16, None, None, 64, 64, 1, 1e-6, 1.0, None) == _lib.EINVAL
    assert b"16-byte" in lib.clarus_hip_last_error()
    assert ffn(1 << 20, (1 << 20) + 4096, _lib.BF16, 16, None, 16, None, None, 64, 64, 0, 0.0, 1.0, None) == _lib.EINVAL
    assert b"overlap" in lib.clarus_hip_last_error()
    assert ffn(None, 16, _lib.F32, 16, None, 16, None, None, 64, 32, 0, 0.0, 1.0, None) == _lib.EINVAL
    # clarus_hip_ln_gemm_dwconv: 64 channels only, alignment, overlap, size
    lndw = lib.clarus_hip_ln_gemm_dwconv
    assert lndw(16, 1 << 24, 16, None, 16, None, 1, 8, 8, 128, 1e-6, None) == _lib.EINVAL
    assert b"c = 64 only" in lib.clarus_hip_last_error()
    assert lndw(24, 1 << 24, 16, None, 16, None, 1, 8, 8, 64, 1e-6, None) == _lib.EINVAL
    assert b"16-byte" in lib.clarus_hip_last_error()
    assert lndw(1 << 20, (1 << 20) + 4096, 16, None, 16, None, 1, 8, 8, 64, 1e-6, None) == _lib.EINVAL
    assert b"overlap" in lib.clarus_hip_last_error()
    assert lndw(16, 1 << 24, 16, None, 16, None, 1, 1 << 14, 1 << 14, 64, 1e-6, None) == _lib.EINVAL
    assert lndw(16, 1 << 24, None, None, 16, None, 1, 8, 8, 64, 1e-6, None) == _lib.EINVAL
    assert lib.clarus_hip_channel_attention_workspace(1, 0, 48, 1) == 0
    assert lib.clarus_hip_channel_attention_workspace(1, 921600, 48, 1) > 0


def test_noalloc_attention_rejects_oversized_shapes_before_launch(lib):
    """clarus_hip_channel_attention_noalloc checks the partials' size against its static scratch on
    the host, before it looks up the device array or launches anything."""
    big = (64, 65536, 512, 8)  # batch, hw, c, heads: 496 (image, head) trees of 3 records of 64 x 64 per launch
    need = lib.clarus_hip_channel_attention_workspace(*big)
    assert need > _lib.CHANNEL_ATTENTION_SCRATCH_MAX
    assert lib.clarus_hip_channel_attention_noalloc(16, _lib.BF16, 16, 16, *big, None) == _lib.EINVAL
    msg = lib.clarus_hip_last_error()
    assert b"static scratch" in msg and str(need).encode() in msg
    assert lib.clarus_hip_channel_attention_noalloc(16, 1, 16, 16, 1, 64, 30, 2, None) == _lib.EINVAL  # width 15
    assert lib.clarus_hip_channel_attention_noalloc(None, 1, 16, 16, 1, 64, 32, 2, None) == _lib.EINVAL
    # the largest config-4 level needs well under the maximum
    for hw, c, heads in ((921600, 48, 1), (230400, 96, 2), (57600, 192, 4), (14400, 384, 8)):
        assert 0 < lib.clarus_hip_channel_attention_workspace(1, hw, c, heads) <= _lib.CHANNEL_ATTENTION_SCRATCH_MAX
