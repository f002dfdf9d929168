"""ctypes binding of libclarus_hip.so (declarations: include/clarus_hip.h).

The structures below mirror ClarusGemmArgs / ClarusConvArgs field by field; `load()` checks
their sizes against the library's own sizeof and the ABI version before handing it out.
torch is imported first so that the process's HIP runtime is torch's (the library links the
same soname, libamdhip64.so.7, and binds to the already-loaded copy).
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads torch's HIP runtime before the kernel library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libclarus_hip.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "clarus_hip.h")

ABI_VERSION = 2
OK, EINVAL, ELAUNCH = 0, 1, 2
F32, BF16 = 0, 1
PRO_NONE, PRO_LN, PRO_MUL, PRO_RMS, PRO_LNMUL = 0, 1, 2, 3, 5
PRO_ROUND = 0x100  # or-ed into pro: the prologue output may be rounded once to bf16
A_ROWS, A_S2D = 0, 1
C_ROWS, C_SHUFFLE, C_NCHW = 0, 1, 2
ACT_NONE, ACT_GELU, ACT_LRELU = 0, 1, 2
CHANNEL_ATTENTION_SCRATCH_MAX = 16 << 20  # bytes of clarus_hip_channel_attention_noalloc's static scratch

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("a", _vp), ("wt", _vp), ("c", _vp), ("bias", _vp), ("scale", _vp), ("res", _vp),
        ("small", _vp), ("m2", _vp), ("lnw", _vp), ("lnb", _vp), ("stats", _vp),
        ("m", _i64), ("n", _i64), ("k", _i64), ("batch", _i64),
        ("lda", _i64), ("ldc", _i64), ("ldr", _i64), ("ldm2", _i64),
        ("a_bstride", _i64), ("w_bstride", _i64), ("c_bstride", _i64), ("r_bstride", _i64),
        ("a_dtype", _i32), ("w_dtype", _i32), ("c_dtype", _i32), ("r_dtype", _i32),
        ("s_dtype", _i32), ("m2_dtype", _i32),
        ("h", _i32), ("w", _i32), ("oh", _i32), ("ow", _i32), ("pt", _i32), ("pl", _i32),
        ("pro", _i32), ("a_mode", _i32), ("c_mode", _i32), ("gate", _i32), ("act", _i32),
        ("m2_act", _i32),
        ("ln_eps", _f32), ("out_scale", _f32), ("slope", _f32),
        ("tile", _i32),
    ]


class ConvArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("wt", _vp), ("out", _vp), ("bias", _vp), ("res", _vp),
        ("batch", _i64), ("h", _i64), ("w", _i64), ("cin", _i64), ("cout", _i64),
        ("ldx", _i64), ("ldo", _i64), ("ldr", _i64),
        ("x_dtype", _i32), ("w_dtype", _i32), ("o_dtype", _i32), ("r_dtype", _i32),
        ("act", _i32), ("up2", _i32), ("c_mode", _i32),
        ("out_scale", _f32), ("slope", _f32),
        ("tile", _i32),
    ]


# name -> (restype, argtypes); every function declared in include/clarus_hip.h
SIGNATURES = {
    "clarus_hip_gemm": (_i32, [ctypes.POINTER(GemmArgs), _vp]),
    "clarus_hip_rows_split": (_i32, [ctypes.POINTER(GemmArgs), _vp, _vp]),
    "clarus_hip_rows_prologue": (_i32, [ctypes.POINTER(GemmArgs), _vp, _vp]),
    "clarus_hip_gemm_ln_rows": (_i32, [ctypes.POINTER(GemmArgs), _vp, _f32, _i32, _vp]),
    "clarus_hip_gemm_ln_gemm": (_i32, [ctypes.POINTER(GemmArgs), _f32, _i32, _vp, _vp, _vp, _i64, _i32, _vp]),
    "clarus_hip_gemm_wp": (_i32, [ctypes.POINTER(GemmArgs), _vp, _vp]),
    "clarus_hip_gemm_wr": (_i32, [ctypes.POINTER(GemmArgs), _vp, _vp]),
    "clarus_hip_ffn": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _f32, _vp]),
    "clarus_hip_ln_gemm_dwconv": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp]),
    "clarus_hip_gemm_ln_gemm_w1p": (_i32, [ctypes.POINTER(GemmArgs), _vp, _f32, _i32, _vp, _vp, _vp, _i64, _i32, _vp]),
    "clarus_hip_conv3x3": (_i32, [ctypes.POINTER(ConvArgs), _vp]),
    "clarus_hip_intro3x3": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _vp]),
    "clarus_hip_channel_attention_workspace": (ctypes.c_size_t, [_i64, _i64, _i64, _i64]),
    "clarus_hip_channel_attention": (_i32, [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp,
                                            ctypes.c_size_t, _vp]),
    "clarus_hip_channel_attention_noalloc": (_i32, [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "clarus_hip_patch_filter": (_i32, [_vp, _i32, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _i32,
                                       _i64, _i64, _i64, _i64, _vp]),
    "clarus_hip_linear_patch_filter": (_i32, [_vp, _i32, _vp, _i32, _vp, _i32, _f32, _vp, _vp, _vp, _vp, _i32, _vp,
                                              _i32, _i64, _i64, _i64, _i64, _i64, _vp]),
    "clarus_hip_patch_corr": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64,
                                     _i64, _i64, _vp]),
    "clarus_hip_dwconv3x3": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _i32,
                                    _vp]),
    "clarus_hip_boxmean_workspace": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "clarus_hip_boxmean": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _vp, ctypes.c_size_t,
                                  _vp]),
    "clarus_hip_psnr_ssim_workspace": (ctypes.c_size_t, [_i64, _i64]),
    "clarus_hip_psnr_ssim": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp, ctypes.c_size_t, _vp]),
    "clarus_hip_selective_scan_workspace": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "clarus_hip_selective_scan": (_i32, [_vp, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp,
                                         ctypes.c_size_t, _vp]),
    "clarus_hip_abi_version": (_i32, []),
    "clarus_hip_sizeof_gemm_args": (ctypes.c_size_t, []),
    "clarus_hip_sizeof_conv_args": (ctypes.c_size_t, []),
    "clarus_hip_last_error": (ctypes.c_char_p, []),
    "clarus_hip_last_kernel": (ctypes.c_char_p, []),
}

_LIB = None


def load(path: str = LIB_PATH):
    """The bound library (loaded once). Raises RuntimeError when it is missing or does not
    match this binding."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (run clarus_amd.build.build_lib() or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    missing = [name for name in SIGNATURES if not hasattr(lib, name)]
    if missing:
        raise RuntimeError(f"{path} lacks {missing}: rebuild it")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.clarus_hip_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {lib.clarus_hip_abi_version()} != {ABI_VERSION}")
    if lib.clarus_hip_sizeof_gemm_args() != ctypes.sizeof(GemmArgs):
        raise RuntimeError("ClarusGemmArgs layout differs between the library and the binding")
    if lib.clarus_hip_sizeof_conv_args() != ctypes.sizeof(ConvArgs):
        raise RuntimeError("ClarusConvArgs layout differs between the library and the binding")
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise RuntimeError with the library's message for a nonzero return code."""
    if rc != OK:
        msg = _LIB.clarus_hip_last_error().decode(errors="replace") if _LIB is not None else ""
        kind = {EINVAL: "invalid arguments", ELAUNCH: "launch failed"}.get(rc, f"error {rc}")
        raise RuntimeError(f"{what}: {kind}: {msg}")


def last_kernel() -> str:
    """Kernel the calling thread's last launching GEMM / conv entry point chose."""
    return _LIB.clarus_hip_last_kernel().decode() if _LIB is not None else ""


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise ValueError(f"no kernel dtype for {dt}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
