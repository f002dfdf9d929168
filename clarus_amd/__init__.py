"""clarus_amd: MI355X (gfx950) HIP kernels for clarus's GEMM-shaped operator family.

The `hip` operator backend (clarus_amd.hip_ops.HipOps) plugs into clarus's per-operator
dispatch (clarus_amd.dispatch mirrors its contract) and runs the ops on hand-written HIP
kernels in libclarus_hip.so (C ABI: include/clarus_hip.h, bound by clarus_amd._lib).
"""
__version__ = "0.1.0"
