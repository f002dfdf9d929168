"""`hip` operator backend: clarus's GEMM-family ops on MI355X (gfx950) HIP kernels.

Registers as backend "hip" in the per-operator dispatch (python/clarus/ops/__init__.py:41-51),
so a runtime config `backends: [hip, torch]` runs these kernels and falls back to the PyTorch
reference backend for anything they decline. Each op has the signature and semantics of the
reference backend (python/clarus/ops/torch_ref.py) and the acceptance rules of the Triton
adapter (python/clarus/ops/triton_cuda.py): arguments the kernels do not handle raise
`Unsupported` BEFORE anything is launched; a failure inside the library raises RuntimeError.

Ops served: linear, down, up, intro, ending, conv3x3, channel_attention, linear_per_image,
patch_filter, linear_patch_filter, patch_corr, ln_mul_linear (the GEMM family), plus dwconv
(depthwise 3x3 + gates) and boxmean (the other ops of the NAFNet forward), selective_scan
(EVSSM's state-space scan), attention_apply (MDTA attn . V) and linear_ln_linear (a residual
GEMM and the LayerNorm GEMM on its output).

Capture safety: kernels launch on torch's current stream, scratch comes from torch's
allocator, weight re-layouts are computed once through `Backend.cached` (in the eager warm-up
pass), and no call synchronises.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .dft import dft_matrices
from .dispatch import (Backend, BackendUnavailable, Unsupported, linear_dwconv_unfused, linear_gate_linear_unfused,
                       linear_ln_linear_unfused, register_backend)
from .geometry import box_geometry, is_small, make_small

_KDT = (torch.bfloat16, torch.float32)


# ------------------------------------------------------------------ acceptance predicates
def _dense(*ts) -> bool:
    """All given tensors (None skipped) are contiguous."""
    return all(t is None or t.is_contiguous() for t in ts)


def _same(t, shape) -> bool:
    """t is None, or contiguous with exactly `shape`."""
    return t is None or (t.is_contiguous() and tuple(t.shape) == tuple(shape))


def _pix_rows(t: torch.Tensor) -> bool:
    """NHWC addressable as pixel * stride(2) + channel: unit channel stride and one uniform
    pixel stride across rows and images (a channel slice of a wider buffer qualifies)."""
    n, h, w, _ = t.shape
    s = t.stride()
    return s[3] == 1 and (h == 1 or s[1] == w * s[2]) and (n == 1 or s[0] == h * w * s[2])


def _kdt(*ts) -> bool:
    return all(t is None or t.dtype in _KDT for t in ts)


def _vec16(t: torch.Tensor, *strides: int) -> bool:
    """Base pointer and the given element strides keep 16-byte alignment."""
    es = t.element_size()
    return t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in strides)


@register_backend("hip")
class HipOps(Backend):
    name = "hip"
    # linear with a prologue (LN / RMS / TLC map) and bf16 weights runs the prologue as a
    # separate pass from this K on, then a plain bf16 GEMM; shorter rows keep the prologue inside
    # the streaming kernels. NAFNet-w64 720p bf16 forward at thresholds 128 / 256: 9.17-9.22 /
    # 9.29-9.30 ms (rounded rows); 10.68 / 10.51 ms with split rows.
    split_min_k = 128
    # The pass rounds the prologue output once to bf16 (clarus_hip_rows_prologue, then the GEMM
    # with K), as the reference's GPU path does (ops/triton_cuda.py:104-110, kernels/gemm.py:
    # 164-186). True writes [hi | lo] rows instead (clarus_hip_rows_split, K' = 2K on [W | W]):
    # fp32-accurate products at twice the MFMA work and A bytes (forward 10.88 vs 9.27 ms).
    prologue_split = False
    # linear_ln_linear (a residual GEMM and the LayerNorm GEMM on its output, an explicit op the
    # caller asks for) runs the pair as one kernel (clarus_hip_gemm_ln_gemm) when the first GEMM
    # has N = 512 and W2 is a bf16 [512, 512 j] weight, or the first GEMM with the LN rows of its
    # output written by its epilogue (clarus_hip_gemm_ln_rows) and then the second GEMM on those
    # rows when only the first fits; False runs the two linear ops.
    fuse_ln_rows = True
    # The fused pair with K = 512 and an fp32 residual on clarus_hip_gemm_ln_gemm_w1p (both weights
    # streamed into registers, the residual staged in LDS during the first GEMM); False keeps it on
    # clarus_hip_gemm_ln_gemm (the first GEMM's weights staged through LDS).
    pair_w1p = True
    # With pair_w1p, the first GEMM's TLC-map multiply (NAFNet conv3) inside that kernel on each A
    # chunk in LDS (the separate pass's operand bit for bit); False keeps the separate pass.
    pair_mul = True
    # Plain bf16 GEMMs with K = 256, 512 or 1024 (>= wstream_min_k) and W^T rows a multiple of 512 on
    # clarus_hip_gemm_wp (W^T packed once per weight and streamed from L2 into registers, the
    # residual staged in LDS during the K loop); False keeps them on clarus_hip_gemm.
    wstream = True
    wstream_min_k = 256
    wstream_min_tiles = 200  # (64-pixel tile, 512-row pass) workgroups: fewer leave CUs idle
    wstream_gate_only = False
    # LayerNorm / RMS linear without a residual at K = 256 / 512 (bf16 or fp32 rows, bf16
    # weights): the prologue inside clarus_hip_gemm_wp's 128-pixel kernel on whole rows (the
    # separate pass's operand bit for bit, without its round trip through HBM), while that
    # kernel's (tile, pass) count covers 3/4 of the compute units; False, or fewer tiles, keep the
    # separate pass. Reference-block NAFNet-w64 forward: level 3 conv1 and conv4.
    wstream_prologue = True
    # TLC-map multiply linear with a residual, bf16 rows and map, K <= 512, whose rows the separate
    # pass would feed to clarus_hip_gemm_wp's 64-pixel ring: the multiply inside that kernel on each
    # A chunk in LDS (the pass's operand bit for bit); False keeps the separate pass. Reference-
    # block NAFNet-w64 forward: level-3 conv3.
    wstream_mul = True
    # The same multiply inside clarus_hip_gemm_wr (no gate; at K = 256 one half pass, N <= 256)
    # where the separate pass would feed that kernel: NAFNet level-2 conv3.
    wres_mul = True
    # Plain bf16 GEMMs with K in wres_ks on clarus_hip_gemm_wr (persistent workgroups, each keeping
    # its 512-row W^T pass in registers for all of its pixel tiles, the next A tile copied during the
    # current one); False or other K keep them on the kernels above.
    wres = True
    wres_ks = (128, 256)
    # N = 128 with a bf16 residual on clarus_hip_gemm_wr when the map prologue rides along (128
    # residual channels staged per tile): NAFNet level-1 conv3, whose separate 23 us map pass it
    # replaces. Plain c128 c->c + residual stays on clarus_hip_gemm (config-2 c128 c->c: 39.9-40.4
    # us there against 40.5-40.6 on clarus_hip_gemm_wr).
    wres_res128 = True
    # LayerNorm / RMS linear without a residual, bf16 rows and weights, K in wres_ks: the prologue
    # inside clarus_hip_gemm_wr on each A tile in LDS (the separate pass's operand bit for bit,
    # without its round trip through HBM); False keeps the separate pass (K = 128) or the 128-pixel
    # kernel's prologue (K = 256). NAFNet-w64 levels 1 and 2, conv1 and conv4.
    wres_prologue = True
    # linear_patch_filter as one kernel (GEMM output straight into the patch DFT); False runs
    # linear (fp32 output) and patch_filter as two ops.
    fuse_patch_filter = True
    # linear_gate_linear (NAFNet's feed-forward half-block and the config-1 chain, an explicit op
    # the caller asks for) as one kernel (clarus_hip_ffn) for c = 32 / 64 channels (and 128 in bf16)
    # with weights of the activation dtype; False (or other shapes) runs its two linear ops.
    fuse_ffn = True
    # linear_dwconv (NAFNet's conv1 with LayerNorm -> depthwise 3x3 -> SimpleGate, an explicit op the
    # caller asks for) as one kernel (clarus_hip_ln_gemm_dwconv) for bf16 x of 64 channels; False (or
    # other shapes) runs its two ops.
    fuse_ln_dwconv = True
    # Short-K prologue GEMMs (K < split_min_k) on the ring streaming kernel round the prologue
    # output once to bf16 too (CLARUS_PRO_ROUND) instead of taking hi + lo pairs.
    round_short_prologue = False

    def __init__(self, dtype, device):
        super().__init__(dtype, device)
        dev = torch.device(device)
        if torch.version.hip is None:
            raise BackendUnavailable("needs a ROCm build of torch")
        if dev.type != "cuda":
            raise BackendUnavailable(f"needs a HIP device (torch type 'cuda'), got {dev}")
        if dtype not in _KDT:
            raise BackendUnavailable(f"runs bf16 / fp32 activations, got {dtype}")
        if not torch.cuda.is_available():
            raise BackendUnavailable("no HIP device is visible")
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        arch = torch.cuda.get_device_properties(dev).gcnArchName.split(":")[0]
        if arch != "gfx950":
            raise BackendUnavailable(f"kernels are built for gfx950, device is {arch}")
        try:
            self.lib = _lib.load()
        except (OSError, RuntimeError) as exc:
            raise BackendUnavailable(f"libclarus_hip.so: {exc}") from exc
        self.dev = dev
        self._cus = None  # compute units of dev, looked up on first use
        # launches of the fused pair kernel (clarus_hip_gemm_ln_gemm) and of the LN-rows GEMM
        # (clarus_hip_gemm_ln_rows) made by linear_ln_linear; counters only, never read by the dispatch
        self.pair_launches = {"gemm_ln_gemm": 0, "gemm_ln_rows": 0}
        self.ffn_launches = 0  # linear_gate_linear calls served by clarus_hip_ffn
        self.ln_dw_launches = 0  # linear_dwconv calls served by clarus_hip_ln_gemm_dwconv
        self._ca_ws = {}  # (device, stream) -> zeroed channel-attention workspace (counters stay zero)

    # ------------------------------------------------------------------ plumbing
    def cached(self, t: torch.Tensor, tag: str, fn):
        """Weight re-layout computed once per (tensor, tag).

        Keyed like the base class on the storage address, plus strides and dtype, and the entry
        keeps a reference to the source tensor: while an entry lives its address cannot be
        recycled by the caching allocator for a different weight, and an in-place update of the
        weight (its version counter) recomputes the entry."""
        key = (t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype, tag)
        hit = self._cache.get(key)
        if hit is None or hit[1] != t._version:
            hit = (t, t._version, fn(t))
            self._cache[key] = hit
        return hit[2]

    def _stream(self, t: torch.Tensor) -> int:
        return torch.cuda.current_stream(t.device).cuda_stream

    def _bias(self, b):
        """fp32 contiguous copy of a (weight-like) vector, once per tensor."""
        if b is None:
            return None
        if b.dtype == torch.float32 and b.is_contiguous():
            return b
        return self.cached(b, "f32", lambda t: t.float().contiguous())

    def _wt(self, w: torch.Tensor) -> torch.Tensor:
        """[K, N] weight -> W^T [N, K] (K contiguous), kept in its dtype."""
        return self.cached(w, "wt", lambda t: t.t().contiguous())

    def _wt2(self, w: torch.Tensor) -> torch.Tensor:
        """[K, N] weight -> [W | W]^T [N, 2K]: the weights of the split-operand GEMM, whose
        A rows are [hi | lo] (clarus_hip_rows_split)."""
        return self.cached(w, "wt2", lambda t: torch.cat([t.t(), t.t()], dim=1).contiguous())

    def _mats(self, device):
        key = ("dft8", str(device))
        m = self._cache.get(key)
        if m is None:
            fwd, inv = dft_matrices(8)
            m = (torch.tensor(fwd, dtype=torch.float32, device=device).contiguous(),
                 torch.tensor(inv, dtype=torch.float32, device=device).contiguous())
            self._cache[key] = m
        return m

    def _gemm(self, what, *, a, wt, c, m, n, k, lda, ldc, bias=None, scale=None, res=None, ldr=0,
              gate=False, act=0, pro=0, a_mode=0, c_mode=0, batch=1, a_bs=0, w_bs=0, c_bs=0, r_bs=0,
              small=None, geom=(0, 0, 0, 0, 0, 0), m2=None, ldm2=0, lnw=None, lnb=None, m2_act=0,
              ln_eps=1e-6, out_scale=1.0, tile=0, wp=None):
        h, w, oh, ow, pt, pl = geom
        stats = None
        if (pro & 0xff) in (_lib.PRO_LN, _lib.PRO_RMS, _lib.PRO_LNMUL) and k > 128 and batch == 1 and wp is None:
            stats = torch.empty(2 * m, device=a.device, dtype=torch.float32)  # row statistics scratch
        args = _lib.GemmArgs(
            a=a.data_ptr(), wt=wt.data_ptr(), c=c.data_ptr(), bias=_lib.ptr(bias), scale=_lib.ptr(scale),
            res=_lib.ptr(res), small=_lib.ptr(small), m2=_lib.ptr(m2), lnw=_lib.ptr(lnw), lnb=_lib.ptr(lnb),
            stats=_lib.ptr(stats),
            m=m, n=n, k=k, batch=batch, lda=lda, ldc=ldc, ldr=ldr, ldm2=ldm2,
            a_bstride=a_bs, w_bstride=w_bs, c_bstride=c_bs, r_bstride=r_bs,
            a_dtype=_lib.dtype_code(a.dtype), w_dtype=_lib.dtype_code(wt.dtype), c_dtype=_lib.dtype_code(c.dtype),
            r_dtype=_lib.dtype_code(res.dtype) if res is not None else 0,
            s_dtype=_lib.dtype_code(small.dtype) if small is not None else 0,
            m2_dtype=_lib.dtype_code(m2.dtype) if m2 is not None else 0,
            h=h, w=w, oh=oh, ow=ow, pt=pt, pl=pl, pro=pro, a_mode=a_mode, c_mode=c_mode, gate=int(gate),
            act=act, m2_act=m2_act, ln_eps=ln_eps, out_scale=out_scale, slope=0.0, tile=tile)
        if wp is not None:  # the same GEMM with W^T also packed: ("wp" | "wr", packed weight)
            fn = self.lib.clarus_hip_gemm_wr if wp[0] == "wr" else self.lib.clarus_hip_gemm_wp
            _lib.check(fn(ctypes.byref(args), wp[1].data_ptr(), self._stream(a)), what)
        else:
            _lib.check(self.lib.clarus_hip_gemm(ctypes.byref(args), self._stream(a)), what)
        return c

    def _wp_for(self, a, w, k, nout, gate, act, m, res=None, res128=False):
        """("wr" | "wp", W^T packed) when this plain bf16 GEMM goes to clarus_hip_gemm_wr /
        clarus_hip_gemm_wp, else None. Square plain GEMMs that clarus_hip_gemm serves on its W-slice
        kernel (N = K = 128 / 256 / 512, no residual, gate or activation, M <= 80000: the NAFNet SCA
        GEMMs on the TLC map) stay there: cold, us, 75881 x 128 x 128: 16.3 against 18.0 on
        clarus_hip_gemm_wr; 19125 x 256 x 256: 14.3 against 16.0. (Other shapes, e.g. conv1's
        N = 2K, were not measured on it and keep the kernels below.)"""
        nw = (2 if gate else 1) * nout
        if (res is None and not gate and act == 0 and nout == k and m <= 80000 and k in (128, 256, 512)
                and a.dtype == torch.bfloat16 and w.dtype == torch.bfloat16):
            return None
        if (self.wres and k in self.wres_ks and a.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
                and act in (0, _lib.ACT_GELU) and nout % 16 == 0
                and (res is None or (nout % 256 == 0 if gate else (nout == 256 or (res.dtype == torch.bfloat16
                                                                                     and ((nout == 128 and res128)
                                                                                          or nout % 512 == 0)))))):
            return "wr", self._wr_pack(w, bool(gate))
        if not (self.wstream and a.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
                and k >= self.wstream_min_k and k in (256, 512, 1024) and nw % 512 == 0
                and act in (0, _lib.ACT_GELU) and (gate or not self.wstream_gate_only)
                and -(-m // 64) * (nw // 512) >= self.wstream_min_tiles):
            return None
        return "wp", self._w2p(w, bool(gate))

    def _wr_prologue(self, x, w, pro, k, nout, gate, act, res):
        """("wr", W^T packed) when this LayerNorm / RMS linear runs with its prologue inside
        clarus_hip_gemm_wr (see wres_prologue): the shapes whose separate pass would feed that
        kernel, else None."""
        if not (self.wres and self.wres_prologue and not self.prologue_split and res is None
                and pro in (_lib.PRO_LN, _lib.PRO_RMS) and k in self.wres_ks and x.dtype == torch.bfloat16
                and w.dtype == torch.bfloat16 and act in (0, _lib.ACT_GELU) and nout % 16 == 0
                and (gate or act != 0 or nout != k)):
            return None
        return "wr", self._wr_pack(w, bool(gate))

    def _wp_mul(self, x, w, pro, sm, k, nout, gate, act, m, res):
        """("wp" | "wr", W^T packed) when this map-prologue linear runs with the multiply inside the
        kernel its separate pass would feed (see wstream_mul, wres_mul), else None."""
        if not (not self.prologue_split and pro == _lib.PRO_MUL and sm is not None and sm.dtype == torch.bfloat16
                and x.dtype == torch.bfloat16 and k <= 512):
            return None
        wp = self._wp_for(x, w, k, nout, gate, act, m, res, res128=self.wres_res128)
        if wp is None:
            return None
        if wp[0] == "wp":
            return wp if self.wstream_mul and res is not None else None
        return wp if self.wres_mul and not gate and (k == 128 or nout <= 256) else None

    def _wp_prologue(self, x, w, pro, k, nout, gate, act, m, res):
        """("wp", W^T packed) when this LayerNorm / RMS linear runs with its prologue inside
        clarus_hip_gemm_wp (see wstream_prologue), else None."""
        nw = (2 if gate else 1) * nout
        if not (self.wstream and self.wstream_prologue and not self.prologue_split and res is None
                and pro in (_lib.PRO_LN, _lib.PRO_RMS) and k in (256, 512) and nw % 512 == 0
                and x.dtype in (torch.bfloat16, torch.float32) and w.dtype == torch.bfloat16
                and act in (0, _lib.ACT_GELU)):
            return None
        if self._cus is None:
            self._cus = torch.cuda.get_device_properties(self.dev).multi_processor_count
        if 4 * -(-m // 128) * (nw // 512) < 3 * self._cus:
            return None
        return "wp", self._w2p(w, bool(gate))

    # ------------------------------------------------------------------ GEMMs
    def _linear_plan(self, x, w, bias, ln, act, gate, scale, residual, mul, out_dtype):
        """Acceptance rules of linear (ops/triton_cuda.py:84-112): raises Unsupported, else
        returns (n, h, wd, k, nout, odt, map tensor, prologue code, map geometry)."""
        if ln and mul is not None:
            raise Unsupported("linear: LayerNorm and mul prologues together")
        if act not in (None, "gelu") or ln not in (False, True, "rms"):
            raise Unsupported(f"linear: act={act!r} ln={ln!r}")
        n, h, wd, k = x.shape
        if gate and w.shape[1] % 2:
            raise Unsupported("linear: gate needs an even number of weight columns")
        nout = w.shape[1] // 2 if gate else w.shape[1]
        odt = out_dtype or self.dtype
        sm = mul.data if mul is not None else None
        if not (_dense(x, w, bias, scale) and _same(residual, (n, h, wd, nout))
                and (sm is None or (sm.is_contiguous() and tuple(sm.shape[::3]) == (n, k)
                                    and (mul.H, mul.W) == (h, wd)))):
            raise Unsupported("linear: contiguous x / weights / mul map, residual of the output's shape")
        if not (_kdt(x, w, residual, sm) and odt in _KDT and w.shape[0] == k and k % 8 == 0
                and _vec16(x) and (sm is None or _vec16(sm))):
            raise Unsupported("linear: bf16 / fp32 operands, K % 8 == 0, 16-byte aligned rows")
        pro = _lib.PRO_NONE
        geom = (0, 0, 0, 0, 0, 0)
        if ln:
            pro = _lib.PRO_RMS if ln == "rms" else _lib.PRO_LN
        elif sm is not None:
            pro = _lib.PRO_MUL
            geom = (h, wd, sm.shape[1], sm.shape[2], mul.pt, mul.pl)
        return n, h, wd, k, nout, odt, sm, pro, geom

    def _prologue_pass(self, w, pro, k) -> bool:
        """A prologue over this K with these weights runs as a separate pass over the rows (the
        reference's ln_rows / mul_small, ops/triton_cuda.py:104-110), then a plain bf16 GEMM."""
        return pro != _lib.PRO_NONE and w.dtype == torch.bfloat16 and self.split_min_k <= k <= 2048 and k % 32 == 0

    def _prologue_rows(self, x, pro, sm, geom, ln_eps, m, k, split=None):
        """The prologue applied to every row, rounded once to bf16 ([m, K]), or as [hi | lo] bf16
        ([m, 2K]) with prologue_split (or split=True)."""
        split = self.prologue_split if split is None else split
        kk = 2 * k if split else k
        rows = torch.empty((m, kk), device=x.device, dtype=torch.bfloat16)
        hh, ww, oh, ow, pt, pl = geom
        args = _lib.GemmArgs(a=x.data_ptr(), m=m, k=k, batch=1, lda=k, a_dtype=_lib.dtype_code(x.dtype),
                             pro=pro, ln_eps=float(ln_eps), small=_lib.ptr(sm),
                             s_dtype=_lib.dtype_code(sm.dtype) if sm is not None else 0,
                             h=hh, w=ww, oh=oh, ow=ow, pt=pt, pl=pl)
        fn = self.lib.clarus_hip_rows_split if split else self.lib.clarus_hip_rows_prologue
        _lib.check(fn(ctypes.byref(args), rows.data_ptr(), self._stream(x)), "linear")
        return rows

    def linear(self, x, w, bias=None, ln=False, act=None, gate=False, scale=None,
               residual=None, mul=None, out_dtype=None, ln_eps=1e-6):
        if is_small(x):
            return x.with_data(self.linear(x.data, w, bias, ln, act, gate, scale, residual, mul, out_dtype, ln_eps))
        n, h, wd, k, nout, odt, sm, pro, geom = self._linear_plan(x, w, bias, ln, act, gate, scale, residual, mul,
                                                                  out_dtype)
        out = torch.empty((n, h, wd, nout), device=x.device, dtype=odt)
        if out.numel() == 0:
            return out
        epi = dict(bias=self._bias(bias), scale=self._bias(scale), res=residual, ldr=nout, gate=gate,
                   act=_lib.ACT_GELU if act == "gelu" else 0)
        m = n * h * wd
        if self._prologue_pass(w, pro, k):
            wpp = (self._wr_prologue(x, w, pro, k, nout, gate, epi["act"], residual)
                   or self._wp_prologue(x, w, pro, k, nout, gate, epi["act"], m, residual)
                   or self._wp_mul(x, w, pro, sm, k, nout, gate, epi["act"], m, residual))
            if wpp is not None:
                return self._gemm("linear", a=x, wt=self._wt(w), c=out, m=m, n=nout, k=k, lda=k, ldc=nout, pro=pro,
                                  small=sm, geom=geom, ln_eps=float(ln_eps), wp=wpp, **epi)
            # the separate prologue pass of triton_cuda.py:104-110 (ln_rows / mul_small), then a
            # plain bf16 GEMM: rows rounded once to bf16 (K), or as [hi | lo] (K' = 2K)
            rows = self._prologue_rows(x, pro, sm, geom, ln_eps, m, k)
            kk = rows.shape[1]
            wt = self._wt2(w) if self.prologue_split else self._wt(w)
            wp = None if self.prologue_split else self._wp_for(rows, w, kk, nout, gate, epi["act"], m, residual)
            return self._gemm("linear", a=rows, wt=wt, c=out, m=m, n=nout, k=kk, lda=kk, ldc=nout, wp=wp, **epi)
        if pro != _lib.PRO_NONE and w.dtype == torch.bfloat16 and self.round_short_prologue and not self.prologue_split:
            pro |= _lib.PRO_ROUND
        wp = self._wp_for(x, w, k, nout, gate, epi["act"], m, residual) if pro == _lib.PRO_NONE else None
        return self._gemm("linear", a=x, wt=self._wt(w), c=out, m=m, n=nout, k=k, lda=k, ldc=nout, pro=pro,
                          small=sm, geom=geom, ln_eps=float(ln_eps), wp=wp, **epi)

    # ---- a residual GEMM and the LayerNorm GEMM on its output (linear_ln_linear)
    @staticmethod
    def _frag_pack(t: torch.Tensor, gate: bool) -> torch.Tensor:
        """[K, n2w] weight (n2w % 512 == 0) -> W^T in the MFMA fragment order of
        clarus_hip_gemm_ln_gemm, clarus_hip_gemm_wp and clarus_hip_gemm_wr ([pass][wave][16-k step]
        [block][lane][8], the rows of a block permuted so a lane accumulates 16 consecutive
        channels; with gate block 0 / 1 of a wave are the two halves' rows of the same channels)."""
        wt = t.t().contiguous()  # [n2w, K]
        n2w, kk = wt.shape
        dv = wt.device
        wv = torch.arange(8, device=dv).view(1, 8, 1, 1)
        b = torch.arange(2, device=dv).view(1, 1, 2, 1)
        i = torch.arange(32, device=dv).view(1, 1, 1, 32)
        j = 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3)
        pas = torch.arange(n2w // 512, device=dv).view(-1, 1, 1, 1)
        rows = (b * (n2w // 2) + 256 * pas + 32 * wv + j) if gate else (512 * pas + 64 * wv + 32 * b + j)
        f = wt[rows]                                          # [pass, w, b, l32, K]
        f = f.view(n2w // 512, 8, 2, 32, kk // 16, 2, 8)      # k = 16 s + 8 hl + e
        return f.permute(0, 1, 4, 2, 5, 3, 6).contiguous()    # [pass, w, s, b, hl, l32, e]

    def _w2p(self, w2: torch.Tensor, gate: bool) -> torch.Tensor:
        """[K, n2w] weight -> W^T packed (_frag_pack), computed once per weight."""
        return self.cached(w2, "w2p_gate" if gate else "w2p", lambda t: self._frag_pack(t, gate))

    def _wr_pack(self, w: torch.Tensor, gate: bool) -> torch.Tensor:
        """[K, N] (gate: [K, 2 N]) weight -> W^T padded for clarus_hip_gemm_wr (gate: each half to a
        multiple of 256 columns, else to a multiple of 512; zeros), then packed (_frag_pack)."""
        def pack(t):
            kk, nw = t.shape
            if gate:
                n = nw // 2
                z = t.new_zeros(kk, -(-n // 256) * 256 - n)
                tp = torch.cat([t[:, :n], z, t[:, n:], z], dim=1)
            else:
                tp = torch.cat([t, t.new_zeros(kk, -(-nw // 512) * 512 - nw)], dim=1)
            return self._frag_pack(tp.contiguous(), gate)
        return self.cached(w, "wr_gate" if gate else "wr", pack)

    def _pair_first(self, x, w, bias, scale, residual, mul, out_dtype, ln, mul_in=False):
        """The first GEMM of linear_ln_linear on the LN-rows kernel: (A rows, W^T, output,
        epilogue, m) when it fits (bf16 backend, plain bf16 rows after any prologue pass, N = 512,
        K % 64 == 0, a residual, no gate / activation), else None. mul_in: a bf16 TLC map at K = 512
        stays with x (pro = MUL in the epilogue args) for the pair kernel to apply."""
        if not (self.fuse_ln_rows and not self.prologue_split and self.dtype == torch.bfloat16
                and ln in (True, "rms") and not is_small(x) and residual is not None):
            return None
        try:
            n, h, wd, k, nout, odt, sm, pro, geom = self._linear_plan(x, w, bias, False, None, False, scale,
                                                                      residual, mul, out_dtype)
        except Unsupported:
            return None
        if not (nout == 512 and k % 64 == 0 and w.dtype == torch.bfloat16 and n * h * wd > 0):
            return None
        m = n * h * wd
        inside = (mul_in and pro == _lib.PRO_MUL and k == 512 and sm.dtype == torch.bfloat16
                  and x.dtype == torch.bfloat16)
        if inside:
            a = x
        elif pro != _lib.PRO_NONE:
            if not self._prologue_pass(w, pro, k):
                return None
            a = self._prologue_rows(x, pro, sm, geom, 1e-6, m, k)
        elif x.dtype == torch.bfloat16:
            a = x
        else:
            return None
        out = torch.empty((n, h, wd, nout), device=x.device, dtype=odt)
        hh, ww, oh, ow, pt, pl = geom if inside else (0, 0, 0, 0, 0, 0)
        epi = _lib.GemmArgs(
            a=a.data_ptr(), wt=self._wt(w).data_ptr(), c=out.data_ptr(), bias=_lib.ptr(self._bias(bias)),
            scale=_lib.ptr(self._bias(scale)), res=residual.data_ptr(), m=m, n=nout, k=k, batch=1, lda=k, ldc=nout,
            ldr=nout, a_dtype=_lib.BF16, w_dtype=_lib.BF16, c_dtype=_lib.dtype_code(odt),
            r_dtype=_lib.dtype_code(residual.dtype), out_scale=1.0, pro=_lib.PRO_MUL if inside else 0,
            small=_lib.ptr(sm) if inside else None, s_dtype=_lib.BF16 if inside else 0,
            h=hh, w=ww, oh=oh, ow=ow, pt=pt, pl=pl)
        return a, out, epi, m

    def linear_ln_linear(self, x, w, bias=None, scale=None, residual=None, mul=None, out_dtype=None,
                         w2=None, bias2=None, gate2=False, ln=True, ln_eps=1e-6):
        """y = linear(x, w, bias, scale=, residual=, mul=, out_dtype=), then u = linear(y, w2,
        bias2, ln=ln, gate=gate2, ln_eps=ln_eps); returns (y, u). One kernel
        (clarus_hip_gemm_ln_gemm) when the first GEMM fits the LN-rows kernel and W2 is a bf16
        [512, 512 j] weight; the first GEMM writing the LN rows of its output and a plain GEMM
        on them when only the first fits; otherwise the two linear ops."""
        pairable = w2 is not None and w2.dtype == torch.bfloat16 and w2.dim() == 2 and w2.shape[0] == 512
        b2 = self._bias(bias2) if pairable else None
        # the first GEMM's TLC-map multiply inside clarus_hip_gemm_ln_gemm_w1p (the branch below that
        # takes it: W2 [512, 512 j], an fp32 residual, K = 512 checked in _pair_first)
        mul_in = (pairable and self.pair_mul and self.pair_w1p and mul is not None and residual is not None
                  and residual.dtype == torch.float32 and w2.shape[1] % 512 == 0 and w2.is_contiguous()
                  and (b2 is None or _vec16(b2)))
        first = self._pair_first(x, w, bias, scale, residual, mul, out_dtype, ln, mul_in) if pairable else None
        if first is None:
            return linear_ln_linear_unfused(self, x, w, bias, scale, residual, mul, out_dtype, w2, bias2, gate2,
                                            ln, ln_eps)
        a, y, args, m = first
        rms = int(ln == "rms")
        b2 = self._bias(bias2)
        fused = (w2.dtype == torch.bfloat16 and w2.dim() == 2 and w2.shape[0] == 512 and w2.shape[1] % 512 == 0
                 and w2.is_contiguous() and (b2 is None or _vec16(b2)))
        n, h, wd, _ = y.shape
        if fused:
            n2w = w2.shape[1]
            u = torch.empty((n, h, wd, n2w // 2 if gate2 else n2w), device=x.device, dtype=torch.bfloat16)
            if args.k == 512 and residual.dtype == torch.float32 and self.pair_w1p:
                # both weights streamed into registers, the residual staged in LDS during the K loop
                _lib.check(self.lib.clarus_hip_gemm_ln_gemm_w1p(
                    ctypes.byref(args), self._w2p(w, False).data_ptr(), float(ln_eps), rms,
                    self._w2p(w2, bool(gate2)).data_ptr(), _lib.ptr(b2), u.data_ptr(), n2w, int(bool(gate2)),
                    self._stream(a)), "linear_ln_linear")
            else:
                _lib.check(self.lib.clarus_hip_gemm_ln_gemm(
                    ctypes.byref(args), float(ln_eps), rms, self._w2p(w2, bool(gate2)).data_ptr(), _lib.ptr(b2),
                    u.data_ptr(), n2w, int(bool(gate2)), self._stream(a)), "linear_ln_linear")
            self.pair_launches["gemm_ln_gemm"] += 1
            return y, u
        rows = torch.empty((n, h, wd, 512), device=x.device, dtype=torch.bfloat16)
        _lib.check(self.lib.clarus_hip_gemm_ln_rows(ctypes.byref(args), rows.data_ptr(), float(ln_eps), rms,
                                                    self._stream(a)), "linear_ln_linear")
        self.pair_launches["gemm_ln_rows"] += 1
        # the rows are LN(y) rounded once to bf16: what linear(y, ln=...) feeds its GEMM for K = 512
        return y, self.linear(rows, w2, bias2, gate=gate2)

    # ---- the feed-forward half-block (linear_gate_linear)
    @staticmethod
    def _ffn_pack1(w1: torch.Tensor) -> torch.Tensor:
        """w1 [c, 2c] (linear layout) -> clarus_hip_ffn's fragment order:
        w1p[T][s][l][i] = w1[16 s + 8 (l // 32) + i][32 T + l % 32]."""
        c = w1.shape[0]
        dv = w1.device
        lv = torch.arange(64, device=dv).view(1, 1, 64, 1)
        t1 = torch.arange(2 * c // 32, device=dv).view(-1, 1, 1, 1)
        s = torch.arange(c // 16, device=dv).view(1, -1, 1, 1)
        i = torch.arange(8, device=dv).view(1, 1, 1, 8)
        return w1[16 * s + 8 * (lv // 32) + i, 32 * t1 + lv % 32].contiguous()

    @staticmethod
    def _ffn_pack2(w2: torch.Tensor) -> torch.Tensor:
        """w2 [c, c] (linear layout) -> clarus_hip_ffn's fragment order: w2p[T2][T][l][j] =
        w2[32 T + 8 (j // 4) + 4 (l // 32) + j % 4][o(T2, l % 32)], o(T2, r) = 32 T2 + 16 (r // 16) +
        8 ((r // 4) % 2) + 4 ((r // 8) % 2) + r % 4."""
        c = w2.shape[0]
        dv = w2.device
        lv = torch.arange(64, device=dv).view(1, 1, 64, 1)
        t2 = torch.arange(c // 32, device=dv).view(-1, 1, 1, 1)
        tg = torch.arange(c // 32, device=dv).view(1, -1, 1, 1)
        j = torch.arange(16, device=dv).view(1, 1, 1, 16)
        r = lv % 32
        o = 32 * t2 + 16 * (r // 16) + 8 * ((r // 4) % 2) + 4 * ((r // 8) % 2) + r % 4
        return w2[32 * tg + 8 * (j // 4) + 4 * (lv // 32) + j % 4, o].contiguous()

    def linear_gate_linear(self, x, w1, b1=None, w2=None, b2=None, scale=None, ln=False, ln_eps=1e-6,
                           out_dtype=None):
        """linear(linear(x, w1, b1, ln=ln, gate=True), w2, b2, scale=scale, residual=x) (the
        feed-forward half of a NAFNet block; the config-1 chain without LN). One kernel
        (clarus_hip_ffn) for dense NHWC x with c = 32 or 64 (or 128 in bf16) in the backend's dtype, weights of that
        dtype and an output of it: the gated intermediate stays in registers, rounded as the
        first linear stores it; with bf16 weights a normalised row is rounded once to bf16 (the
        reference's in-kernel LayerNorm, kernels/gemm.py:165-175). Otherwise, or with
        prologue_split, the two linear ops."""
        c = x.shape[-1] if x.dim() == 4 else 0
        odt = out_dtype or self.dtype
        fits = (self.fuse_ffn and (c in (32, 64) or (c == 128 and x.dtype == torch.bfloat16))
                and x.dtype == self.dtype and odt == x.dtype
                and ln in (False, True, "rms") and not (ln and self.prologue_split)
                and w2 is not None and w1.dtype == x.dtype and w2.dtype == x.dtype
                and tuple(w1.shape) == (c, 2 * c) and tuple(w2.shape) == (c, c)
                and (b1 is None or tuple(b1.shape) == (2 * c,)) and (b2 is None or tuple(b2.shape) == (c,))
                and (scale is None or tuple(scale.shape) == (c,))
                and _dense(x, w1, w2, b1, b2, scale) and _vec16(x))
        if not fits:
            return linear_gate_linear_unfused(self, x, w1, b1, w2, b2, scale=scale, ln=ln, ln_eps=ln_eps,
                                              out_dtype=out_dtype)
        w1p = self.cached(w1, "ffn1", self._ffn_pack1)
        w2p = self.cached(w2, "ffn2", self._ffn_pack2)
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
        pro = {False: _lib.PRO_NONE, True: _lib.PRO_LN, "rms": _lib.PRO_RMS}[ln]
        _lib.check(self.lib.clarus_hip_ffn(
            x.data_ptr(), out.data_ptr(), _lib.dtype_code(x.dtype), w1p.data_ptr(), _lib.ptr(self._bias(b1)),
            w2p.data_ptr(), _lib.ptr(self._bias(b2)), _lib.ptr(self._bias(scale)), x.numel() // c, c, pro,
            float(ln_eps), 1.0, self._stream(x)), "linear_gate_linear")
        self.ffn_launches += 1
        return out

    # ---- the first half of a NAFNet block (linear_dwconv)
    @staticmethod
    def _ln_dw_pack(w: torch.Tensor) -> torch.Tensor:
        """w [64, 128] (linear layout) -> clarus_hip_ln_gemm_dwconv's fragment order:
        w1p[T][s][l][i] = w[16 s + 8 (l // 32) + i][o(T, l % 32)], o(T, r) = 32 T + 16 (r // 16) +
        8 ((r // 4) % 2) + 4 ((r // 8) % 2) + r % 4."""
        k, n = w.shape
        dv = w.device
        lv = torch.arange(64, device=dv).view(1, 1, 64, 1)
        t = torch.arange(n // 32, device=dv).view(-1, 1, 1, 1)
        s = torch.arange(k // 16, device=dv).view(1, -1, 1, 1)
        i = torch.arange(8, device=dv).view(1, 1, 1, 8)
        r = lv % 32
        o = 32 * t + 16 * (r // 16) + 8 * ((r // 4) % 2) + 4 * ((r // 8) % 2) + r % 4
        return w[16 * s + 8 * (lv // 32) + i, o].contiguous()

    def linear_dwconv(self, x, w, bias=None, dw_w=None, dw_b=None, ln=True, gate=True, ln_eps=1e-6):
        """dwconv(linear(x, w, bias, ln=ln), dw_w, dw_b, gate=gate) (the first half of a NAFNet
        block). One kernel (clarus_hip_ln_gemm_dwconv) for dense bf16 NHWC x with 64 channels, a
        bf16 [64, 128] weight, LayerNorm and SimpleGate: the 128-channel intermediate stays in LDS,
        rounded to bf16 as the 1x1 conv stores it. Otherwise the two ops."""
        c = x.shape[-1] if x.dim() == 4 else 0
        fits = (self.fuse_ln_dwconv and self.dtype == torch.bfloat16 and x.dtype == torch.bfloat16 and c == 64
                and ln is True and gate is True and w.dtype == torch.bfloat16 and tuple(w.shape) == (64, 128)
                and dw_w is not None and tuple(dw_w.shape) == (128, 1, 3, 3)
                and (bias is None or tuple(bias.shape) == (128,)) and (dw_b is None or tuple(dw_b.shape) == (128,))
                and _dense(x, w, bias, dw_b) and _vec16(x) and x.numel() * 2 < (1 << 31))
        if not fits:
            return linear_dwconv_unfused(self, x, w, bias, dw_w, dw_b, ln=ln, gate=gate, ln_eps=ln_eps)
        w1p = self.cached(w, "lndw", self._ln_dw_pack)
        taps = self.cached(dw_w, "dw9", lambda t: t.float().reshape(t.shape[0], 9).t().contiguous())
        n, h, wd, _ = x.shape
        out = torch.empty((n, h, wd, 64), device=x.device, dtype=torch.bfloat16)
        _lib.check(self.lib.clarus_hip_ln_gemm_dwconv(
            x.data_ptr(), out.data_ptr(), w1p.data_ptr(), _lib.ptr(self._bias(bias)), taps.data_ptr(),
            _lib.ptr(self._bias(dw_b)), n, h, wd, c, float(ln_eps), self._stream(x)), "linear_dwconv")
        self.ln_dw_launches += 1
        return out

    def down(self, x, w4d, b, out_dtype=None):
        if tuple(w4d.shape[-2:]) != (2, 2) or not _dense(x, b):
            raise Unsupported("down: only 2x2 stride-2 convs, contiguous input")
        n, h, wd, c = x.shape
        cout = w4d.shape[0]
        odt = out_dtype or self.dtype
        if not (_kdt(x, w4d) and odt in _KDT and w4d.shape[1] == c and c % 8 == 0 and h >= 2 and wd >= 2
                and _vec16(x)):
            raise Unsupported("down: bf16 / fp32, cin % 8 == 0, at least 2x2 input")
        wt = self.cached(w4d, "s2d", lambda t: t.permute(0, 2, 3, 1).reshape(t.shape[0], -1).contiguous())
        out = torch.empty((n, h // 2, wd // 2, cout), device=x.device, dtype=odt)
        if x.dtype == torch.float32 and wt.dtype == torch.bfloat16 and not self.prologue_split:
            # fp32 activations with bf16 weights: rounded once to bf16 like the reference's fp32 A
            # operand (kernels/gemm.py:187-193), then the bf16 space-to-depth GEMM
            xb = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
            args = _lib.GemmArgs(a=x.data_ptr(), m=n * h * wd, k=c, batch=1, lda=c, a_dtype=_lib.F32,
                                 pro=_lib.PRO_NONE)
            _lib.check(self.lib.clarus_hip_rows_prologue(ctypes.byref(args), xb.data_ptr(), self._stream(x)), "down")
            x = xb
        return self._gemm("down", a=x, wt=wt, c=out, m=n * (h // 2) * (wd // 2), n=cout, k=4 * c, lda=c, ldc=cout,
                          bias=self._bias(b), a_mode=_lib.A_S2D, geom=(h, wd, 0, 0, 0, 0))

    def up(self, x, w, residual=None, out_dtype=None):
        n, h, wd, c = x.shape
        cq = w.shape[1] // 4
        if w.shape[1] % 16 or not (_dense(x, w) and _same(residual, (n, 2 * h, 2 * wd, cq))):
            raise Unsupported("up: 4 C' % 16 == 0, contiguous x, residual of the output's shape")
        odt = out_dtype or self.dtype
        if not (_kdt(x, w, residual) and odt in _KDT and w.shape[0] == c and c % 8 == 0 and _vec16(x)):
            raise Unsupported("up: bf16 / fp32, K % 8 == 0")
        out = torch.empty((n, 2 * h, 2 * wd, cq), device=x.device, dtype=odt)
        return self._gemm("up", a=x, wt=self._wt(w), c=out, m=n * h * wd, n=4 * cq, k=c, lda=c, ldc=4 * cq,
                          res=residual, c_mode=_lib.C_SHUFFLE, geom=(h, wd, 0, 0, 0, 0))

    # ------------------------------------------------------------------ convolutions
    def _conv_wt(self, w):
        return self.cached(w, "conv3", lambda t: t.permute(0, 2, 3, 1).reshape(t.shape[0], -1).contiguous())

    def intro(self, inp, w, b, out_dtype=None):
        if tuple(w.shape[1:]) != (3, 3, 3) or b is None or inp.dim() != 4 or inp.shape[1] != 3:
            raise Unsupported("intro: 3-channel input, 3x3, bias")
        odt = out_dtype or self.dtype
        if odt not in _KDT or w.shape[0] % 8 or w.shape[0] > 512:
            raise Unsupported("intro: bf16 / fp32 output, cout a multiple of 8 and at most 512")
        n, _, h, wd = inp.shape
        cout = w.shape[0]
        x = inp if (inp.dtype == torch.float32 and inp.is_contiguous()) else inp.float().contiguous()
        wt = self.cached(w, "intro", lambda t: t.permute(2, 3, 1, 0).reshape(27, t.shape[0]).float().contiguous())
        out = torch.empty((n, h, wd, cout), device=inp.device, dtype=odt)
        _lib.check(self.lib.clarus_hip_intro3x3(x.data_ptr(), wt.data_ptr(), self._bias(b).data_ptr(),
                                                out.data_ptr(), _lib.dtype_code(odt), n, h, wd, cout,
                                                self._stream(x)), "intro")
        return out

    def _conv(self, x, w, b, *, odt, act, residual, out_scale, up2, out, slope, nchw=False):
        n, h, wd, cin = x.shape
        cout = w.shape[0]
        hh, ww = (2 * h, 2 * wd) if up2 else (h, wd)
        if out is None:
            shape = (n, cout, hh, ww) if nchw else (n, hh, ww, cout)
            out = torch.empty(shape, device=x.device, dtype=odt)
        args = _lib.ConvArgs(
            x=x.data_ptr(), wt=self._conv_wt(w).data_ptr(), out=out.data_ptr(), bias=_lib.ptr(self._bias(b)),
            res=_lib.ptr(residual), batch=n, h=h, w=wd, cin=cin, cout=cout, ldx=x.stride(2),
            ldo=0 if nchw else out.stride(2), ldr=(residual.stride(2) if (residual is not None and not nchw) else 0),
            x_dtype=_lib.dtype_code(x.dtype), w_dtype=_lib.dtype_code(w.dtype), o_dtype=_lib.dtype_code(out.dtype),
            r_dtype=_lib.dtype_code(residual.dtype) if residual is not None else 0,
            act=_lib.ACT_LRELU if act == "lrelu" else 0, up2=int(bool(up2)),
            c_mode=_lib.C_NCHW if nchw else _lib.C_ROWS, out_scale=float(out_scale), slope=float(slope), tile=0)
        _lib.check(self.lib.clarus_hip_conv3x3(ctypes.byref(args), self._stream(x)), "conv3x3")
        return out

    def ending(self, x, w, b, inp):
        n, h, wd, cin = x.shape
        if (tuple(w.shape[-2:]) != (3, 3) or tuple(inp.shape) != (n, w.shape[0], h, wd) or b is None
                or not _pix_rows(x)):
            raise Unsupported("ending: 3x3 with global residual of the output's shape, NHWC rows")
        if not (_kdt(x, w) and w.shape[1] == cin and cin % 8 == 0 and _vec16(x, x.stride(2))):
            raise Unsupported("ending: bf16 / fp32, cin % 8 == 0, 16-byte pixel rows")
        res = inp if (inp.dtype == torch.float32 and inp.is_contiguous()) else inp.float().contiguous()
        return self._conv(x, w, b, odt=torch.float32, act=None, residual=res, out_scale=1.0, up2=False, out=None,
                          slope=0.2, nchw=True)

    def conv3x3(self, x, w, b=None, out_dtype=None, act=None, residual=None, out_scale=1.0, up2=False,
                out=None, slope=0.2):
        n, h, wd, cin = x.shape
        oshape = (n, 2 * h, 2 * wd, w.shape[0]) if up2 else (n, h, wd, w.shape[0])
        if act not in (None, "lrelu") or tuple(w.shape[-2:]) != (3, 3) or w.shape[1] != cin:
            raise Unsupported("conv3x3: 3x3, activation none / lrelu")
        if not (_pix_rows(x) and all(t is None or (tuple(t.shape) == oshape and _pix_rows(t)) for t in (residual, out))):
            raise Unsupported("conv3x3: NHWC tensors with a uniform pixel stride, residual / out of the output's shape")
        odt = out.dtype if out is not None else (out_dtype or self.dtype)
        if not (_kdt(x, w, residual) and odt in _KDT and cin % 8 == 0 and _vec16(x, x.stride(2))):
            raise Unsupported("conv3x3: bf16 / fp32, cin % 8 == 0, 16-byte pixel rows")
        return self._conv(x, w, b, odt=odt, act=act, residual=residual, out_scale=out_scale, up2=up2, out=out,
                          slope=slope)

    def boxmean(self, x, k):
        """TLC local mean over the valid (kh, kw) windows, returned as the un-padded map (not
        GEMM-shaped; the reference's boxmean, ops/torch_ref.py:133-141)."""
        if x.dim() != 4 or not x.is_contiguous() or x.dtype not in _KDT or x.shape[-1] % 8 or not _vec16(x):
            raise Unsupported("boxmean: contiguous NHWC bf16 / fp32 with channels % 8 == 0")
        n, h, wd, c = x.shape
        k1, k2, oh, ow, pt, pl = box_geometry(h, wd, k)
        out = torch.empty((n, oh, ow, c), device=x.device, dtype=self.dtype)
        nbytes = self.lib.clarus_hip_boxmean_workspace(n, h, wd, c, k1, k2)
        scratch = torch.empty((nbytes + 3) // 4, device=x.device, dtype=torch.float32)
        _lib.check(self.lib.clarus_hip_boxmean(x.data_ptr(), _lib.dtype_code(x.dtype), out.data_ptr(),
                                               _lib.dtype_code(self.dtype), n, h, wd, c, k1, k2, scratch.data_ptr(),
                                               nbytes, self._stream(x)), "boxmean")
        return make_small(out, pt, pl, h, wd)

    def dwconv(self, x, w, b, dil=1, gate=False, act=None):
        """Depthwise 3x3 conv with fused SimpleGate / GELU gate / GELU (not GEMM-shaped; the
        reference serves it from its torch or Triton backend, ops/torch_ref.py:143-155)."""
        kh, kw = w.shape[-2:]
        n, h, wd, c = x.shape
        gcode = {False: 0, None: 0, True: 1, "mul": 1, "gelu": 2}.get(gate, -1)
        cout = c // 2 if gcode else c
        if ((kh, kw) != (3, 3) or tuple(w.shape[:2]) != (c, 1) or gcode < 0 or act not in (None, "gelu")
                or (act == "gelu" and gcode) or dil < 1 or not _dense(x, b)):
            raise Unsupported("dwconv: contiguous 3x3 depthwise, gate none / mul / gelu, act none / gelu")
        if not (_kdt(x) and (gcode == 0 or c % 2 == 0) and cout % 8 == 0 and c % 8 == 0 and _vec16(x)
                and 10 * c * 4 <= 160 * 1024):
            raise Unsupported("dwconv: bf16 / fp32, output channels % 8 == 0")
        taps = self.cached(w, "dw9", lambda t: t.float().reshape(t.shape[0], 9).t().contiguous())
        out = torch.empty((n, h, wd, cout), device=x.device, dtype=self.dtype)
        _lib.check(self.lib.clarus_hip_dwconv3x3(
            x.data_ptr(), _lib.dtype_code(x.dtype), taps.data_ptr(), _lib.ptr(self._bias(b)), out.data_ptr(),
            _lib.dtype_code(self.dtype), n, h, wd, c, int(dil), gcode, _lib.ACT_GELU if act == "gelu" else 0,
            self._stream(x)), "dwconv")
        return out

    # ------------------------------------------------------------------ attention
    def channel_attention(self, qkv, heads, temperature):
        if not qkv.is_contiguous():
            raise Unsupported("channel_attention: contiguous qkv only")
        n, h, wd, c3 = qkv.shape
        c = c3 // 3
        if c3 % 3 or c % heads or not _kdt(qkv) or (c // heads) % 8 or c // heads > 64 or not _vec16(qkv, c):
            raise Unsupported("channel_attention: head width a multiple of 8, <= 64; bf16 / fp32")
        ch = c // heads
        t = temperature.reshape(heads)
        t = t if (t.dtype == torch.float32 and t.is_contiguous()) else t.float().contiguous()
        need = self.lib.clarus_hip_channel_attention_workspace(n, h * wd, c, heads)
        scratch = self._attention_workspace(need, qkv.device)
        out = torch.empty((n, heads, ch, ch), dtype=torch.float32, device=qkv.device)
        _lib.check(self.lib.clarus_hip_channel_attention(qkv.data_ptr(), _lib.dtype_code(qkv.dtype), t.data_ptr(),
                                                         out.data_ptr(), n, h * wd, c, heads, scratch.data_ptr(),
                                                         scratch.numel(), self._stream(qkv)), "channel_attention")
        return out

    def _attention_workspace(self, need: int, device) -> torch.Tensor:
        """Workspace of clarus_hip_channel_attention: its leading arrival counters must be zero when
        a call starts, and every call leaves them zero. Eager calls reuse one zeroed buffer per
        stream (grown, zeroed again, when a call needs more); a call under graph capture gets a
        fresh zeroed buffer of the graph's own pool, its fill recorded before the launch, so every
        replay starts from zero."""
        if torch.cuda.is_current_stream_capturing():
            return torch.zeros(need, dtype=torch.uint8, device=device)
        key = (str(device), torch.cuda.current_stream(device).cuda_stream)
        ws = self._ca_ws.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.zeros(max(need, 1 << 20), dtype=torch.uint8, device=device)
            self._ca_ws[key] = ws
        return ws

    def linear_per_image(self, x, w, residual=None, out_dtype=None, bias=None):
        n, h, wd, k = x.shape
        nout = w.shape[-1]
        if (x.stride(-1) != 1 or x.stride(1) != wd * x.stride(2) or tuple(w.shape[:2]) != (n, k)
                or not (_dense(bias) and _same(residual, (n, h, wd, nout)))):
            raise Unsupported("linear_per_image: NHWC rows with a uniform pixel stride, residual of the output's shape")
        odt = out_dtype or self.dtype
        if not (_kdt(x, w, residual) and odt in _KDT and k % 8 == 0 and _vec16(x, x.stride(2), x.stride(0))):
            raise Unsupported("linear_per_image: bf16 / fp32, K % 8 == 0, 16-byte rows")
        out = torch.empty((n, h, wd, nout), device=x.device, dtype=odt)
        wt = w.transpose(1, 2).contiguous()  # per-image weights change every call: not cached
        return self._gemm("linear_per_image", a=x, wt=wt, c=out, m=h * wd, n=nout, k=k, lda=x.stride(2), ldc=nout,
                          bias=self._bias(bias), res=residual, ldr=nout, batch=n, a_bs=x.stride(0),
                          w_bs=nout * k, c_bs=h * wd * nout, r_bs=h * wd * nout)

    def attention_apply(self, qkv, attn, residual=None, out_dtype=None):
        """attn . V of Restormer's MDTA per head: out[p, hd*ch + j] = sum_i A[n, hd, j, i]
        * v[p, hd*ch + i], with v = qkv[..., 2C:] and A the map channel_attention returns
        [N, heads, ch, ch]. Equals linear_per_image(v, blockdiag(A^T)) (the block-diagonal mix the
        Restormer block builds, python/clarus/models/restormer/__init__.py:203-210) without the
        zero blocks: one batched GEMM launch per image with the heads as the batch, A read as
        the GEMM's transposed weight as it is (no copy when it is contiguous)."""
        n, h, wd, c3 = qkv.shape
        c = c3 // 3
        if attn.dim() == 3:
            attn = attn.unsqueeze(0)
        heads, ch = attn.shape[1], attn.shape[2]
        if (not qkv.is_contiguous() or c3 % 3 or heads * ch != c or tuple(attn.shape) != (n, heads, ch, ch)
                or not _same(residual, (n, h, wd, c))):
            raise Unsupported("attention_apply: contiguous qkv, attn [N, heads, ch, ch], residual of the output's shape")
        odt = out_dtype or self.dtype
        if not (_kdt(qkv, attn, residual) and odt in _KDT and ch % 8 == 0 and _vec16(qkv, c3, ch)):
            raise Unsupported("attention_apply: bf16 / fp32, head width % 8 == 0")
        out = torch.empty((n, h, wd, c), device=qkv.device, dtype=odt)
        wt = attn.contiguous()  # W^T per head [n, heads, j, i] is A itself
        for i in range(n):
            self._gemm("attention_apply", a=qkv[i, ..., 2 * c:], wt=wt[i], c=out[i], m=h * wd, n=ch, k=ch, lda=c3,
                       ldc=c, res=residual[i] if residual is not None else None, ldr=c, batch=heads, a_bs=ch,
                       w_bs=ch * ch, c_bs=ch, r_bs=ch)
        return out

    # ------------------------------------------------------------------ state-space scan (EVSSM)
    def selective_scan(self, u, dbl, dt_w, dt_bias, A, D):
        """Mamba selective scan along each crop's raster sequence, d_state 8 (the reference's
        scan, ops/torch_ref.py:312-341; acceptance as ops/triton_cuda.py:228-235):
        clarus_hip_selective_scan, segments scanned in parallel. Returns fp32 [T, h, w, d]."""
        r, ns = dt_w.shape[1], A.shape[1]
        if (not (u.is_contiguous() and dbl.is_contiguous() and dbl.dtype == torch.float32) or ns != 8
                or tuple(dbl.shape[:3]) != tuple(u.shape[:3]) or dbl.shape[-1] < r + 2 * ns):
            raise Unsupported("selective_scan: contiguous inputs, fp32 dbl, d_state 8")
        t, hh, ww, d = u.shape
        if not (_kdt(u) and 1 <= r <= 16 and tuple(dt_w.shape) == (d, r) and tuple(A.shape) == (d, ns)):
            raise Unsupported("selective_scan: bf16 / fp32 u, 1 <= r <= 16")
        a2 = self.cached(A, "a2", lambda v: (v.float() * 1.4426950408889634).contiguous())
        y = torch.empty(u.shape, device=u.device, dtype=torch.float32)
        if y.numel() == 0:
            return y
        need = self.lib.clarus_hip_selective_scan_workspace(t, hh * ww, d)
        scratch = torch.empty((need + 3) // 4, device=u.device, dtype=torch.float32)
        _lib.check(self.lib.clarus_hip_selective_scan(
            u.data_ptr(), _lib.dtype_code(u.dtype), dbl.data_ptr(), dbl.shape[-1], self._bias(dt_w.reshape(-1)).data_ptr(),
            r, self._bias(dt_bias).data_ptr(), a2.data_ptr(), self._bias(D).data_ptr(), y.data_ptr(), t, hh * ww, d,
            scratch.data_ptr(), need, self._stream(u)), "selective_scan")
        return y

    # ------------------------------------------------------------------ frequency ops
    def patch_filter(self, x, f, residual=None, out_dtype=None):
        n, h, wd, c = x.shape
        pad_h, pad_w = (-h) % 8, (-wd) % 8
        if (f.dim() != 3 or tuple(f.shape) != (c, 8, 5) or not _pix_rows(x) or not _same(residual, (n, h, wd, c))
                or (pad_h and pad_h >= h) or (pad_w and pad_w >= wd)):
            raise Unsupported("patch_filter: 8x8 patches, NHWC rows, residual of the output's shape")
        odt = out_dtype or self.dtype
        if not (_kdt(x, residual) and odt in _KDT):
            raise Unsupported("patch_filter: bf16 / fp32")
        fwd, inv = self._mats(x.device)
        gain = self.cached(f, "gain", lambda t: t.float().reshape(t.shape[0], -1).repeat_interleave(2, dim=1)
                           .contiguous())
        out = torch.empty((n, h, wd, c), device=x.device, dtype=odt)
        _lib.check(self.lib.clarus_hip_patch_filter(
            x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(2), fwd.data_ptr(), inv.data_ptr(), gain.data_ptr(),
            _lib.ptr(residual), _lib.dtype_code(residual.dtype) if residual is not None else 0, out.data_ptr(),
            _lib.dtype_code(odt), n, h, wd, c, self._stream(x)), "patch_filter")
        return out

    def linear_patch_filter(self, x, w, bias, f, ln=False, ln_eps=1e-6, residual=None):
        """patch_filter(linear(x, w, bias, ln) kept fp32, f, residual) in one kernel
        (clarus_hip_linear_patch_filter): the GEMM output goes from the MFMA accumulators
        straight into the patch DFT, never to memory. Prologue arithmetic as linear's: LayerNorm /
        RMS inside the kernel in fp32 for K < split_min_k (or fp32 weights, K <= 256), else the
        rows pass rounded once to bf16 first (the reference's ln_rows for K > 128,
        ops/triton_cuda.py:267-270). fuse_patch_filter = False runs the two ops instead."""
        n, h, wd, k = x.shape
        nout = w.shape[1] if w.dim() == 2 else -1
        if (tuple(f.shape[1:]) != (8, 5) or f.shape[0] != nout or min(h, wd) < 9 or bias is None
                or x.dtype != self.dtype or not _dense(x, w, bias) or not _same(residual, (n, h, wd, nout))):
            raise Unsupported("linear_patch_filter: 8x8 patches, H, W >= 9, contiguous, bias, x in the compute "
                              "dtype, residual of the output's shape")
        if ln not in (False, True, "rms"):
            raise Unsupported(f"linear_patch_filter: ln={ln!r}")
        if not self.fuse_patch_filter:
            y = self.linear(x, w, bias, ln=ln, ln_eps=ln_eps, out_dtype=torch.float32)
            return self.patch_filter(y, f, residual=residual)
        if not (_kdt(x, w, residual) and w.shape[0] == k and k % 8 == 0 and _vec16(x)):
            raise Unsupported("linear_patch_filter: bf16 / fp32 operands, K % 8 == 0, 16-byte aligned rows")
        code = {False: 0, True: 1, "rms": 2}[ln]
        a, kk, wt = x, k, self._wt(w)
        pro = _lib.PRO_RMS if ln == "rms" else _lib.PRO_LN
        if code and (self._prologue_pass(w, pro, k) or k > 256):
            # bf16 weights: rows rounded once (or [hi | lo] with prologue_split), as linear; fp32
            # weights with K > 256 (past the kernel's in-register rows): [hi | lo] rows, fp32-accurate
            split = self.prologue_split or w.dtype != torch.bfloat16
            if not (k <= 2048 and k % 32 == 0):
                raise Unsupported("linear_patch_filter: LayerNorm rows over K > 256 need K % 32 == 0, K <= 2048")
            a = self._prologue_rows(x, pro, None, (0, 0, 0, 0, 0, 0), ln_eps, n * h * wd, k, split=split)
            kk = a.shape[1]
            wt = self._wt2(w) if split else wt
            code = 0
        fwd, inv = self._mats(x.device)
        gain = self.cached(f, "gain", lambda t: t.float().reshape(t.shape[0], -1).repeat_interleave(2, dim=1)
                           .contiguous())
        out = torch.empty((n, h, wd, nout), device=x.device, dtype=self.dtype)
        _lib.check(self.lib.clarus_hip_linear_patch_filter(
            a.data_ptr(), _lib.dtype_code(a.dtype), wt.data_ptr(), _lib.dtype_code(wt.dtype), self._bias(bias).data_ptr(),
            code, float(ln_eps), fwd.data_ptr(), inv.data_ptr(), gain.data_ptr(), _lib.ptr(residual),
            _lib.dtype_code(residual.dtype) if residual is not None else 0, out.data_ptr(), _lib.dtype_code(self.dtype),
            n, h, wd, kk, nout, self._stream(x)), "linear_patch_filter")
        return out

    def patch_corr(self, x, c, p=8):
        n, h, w, cx = x.shape
        if p != 8 or h % 8 or w % 8 or x.stride(-1) != 1 or cx < 2 * c or not _kdt(x):
            raise Unsupported("patch_corr: 8x8 patches, H and W multiples of 8, unit channel stride, >= 2c channels")
        fwd, inv = self._mats(x.device)
        out = torch.empty((n, h, w, c), device=x.device, dtype=torch.float32)
        _lib.check(self.lib.clarus_hip_patch_corr(x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), x.stride(1),
                                                  x.stride(2), fwd.data_ptr(), inv.data_ptr(), out.data_ptr(), n, h,
                                                  w, c, self._stream(x)), "patch_corr")
        return out

    def ln_mul_linear(self, x, ln_w, ln_b, m, w, bias=None, m_act=None, residual=None, ln_eps=1e-5,
                      out_dtype=None):
        n, h, wd, k = x.shape
        if (not _dense(x, ln_w, ln_b, w, bias) or tuple(m.shape) != tuple(x.shape) or not _pix_rows(m)
                or not _same(residual, (n, h, wd, w.shape[1]))):
            raise Unsupported("ln_mul_linear: contiguous x, NHWC m with a uniform pixel stride, "
                              "residual of the output's shape")
        odt = out_dtype or self.dtype
        if not (_kdt(x, m, w, residual) and odt in _KDT and m_act in (None, "gelu") and k % 8 == 0
                and _vec16(x) and _vec16(m, m.stride(2))):
            raise Unsupported("ln_mul_linear: bf16 / fp32, K % 8 == 0, 16-byte rows")
        out = torch.empty((n, h, wd, w.shape[1]), device=x.device, dtype=odt)
        return self._gemm("ln_mul_linear", a=x, wt=self._wt(w), c=out, m=n * h * wd, n=w.shape[1], k=k, lda=k,
                          ldc=w.shape[1], bias=self._bias(bias), res=residual, ldr=w.shape[1], pro=_lib.PRO_LNMUL,
                          m2=m, ldm2=m.stride(2), lnw=self._bias(ln_w), lnb=self._bias(ln_b),
                          m2_act=_lib.ACT_GELU if m_act == "gelu" else 0, ln_eps=float(ln_eps))
