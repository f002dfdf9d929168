"""Write the golden fixtures of tests/golden/ from the reference implementation itself.

Run in the build container only (the reference source is not present on the GPU box, and no
part of it is copied here: the fixtures hold inputs, weights and outputs, nothing else):

    python tests/golden/make_golden.py [/root/reference]

What it pins, and why an import is needed for it: the closed-form and known-answer checks of
tests/test_oracle.py pin every single GEMM-family op, but not how the reference *composes* them.

* nafnet_tiny.safetensors: the reference NAFNetLocal model adapter
  (python/clarus/models/nafnet/__init__.py:60-185: weight fold, TLC windows, residual dtypes,
  block wiring, pad / crop) running on its PyTorch backend (ops/torch_ref.py) on the CPU, on a
  tiny network (width 8, enc [1, 1, 1], mid 1, dec [1, 1, 1], train_size 24x40) and a 30x45
  input that needs padding. Outputs for fp32 and bf16 activations, and the exact seeded state
  dict the model was built from (written to a temporary checkpoint and loaded by the
  reference's own load_checkpoint).
* ops_combined.safetensors: reference TorchOps calls whose epilogue / prologue combinations
  fix an operation order, in fp32 and bf16: torch_ref.py:103-131 linear with a TLC-map
  multiply or LN prologue and bias + gate + GELU + scale + residual, :290-302 ln_mul_linear,
  :178-199 conv3x3 with up2 + act + out_scale + residual, :237-245 linear_per_image with
  bias + residual.

* ops_freq.safetensors: reference TorchOps.linear_patch_filter (torch_ref.py:272-276) calls:
  LayerNorm / RMS / no prologue, with and without a residual, fp32 and bf16 activations, on an
  odd 13x22 or 9x16 image (reflect padding) and a 16x16 one; the fp32 intermediate between the GEMM and
  the filter is what the bf16 cases pin (a rounded intermediate gives other bits).

* metrics.safetensors: the reference's on-device metric semantics on the CPU: its host psnr()
  (basicsr rule, python/clarus/metrics.py:46-56) and TorchMetrics.compute (the fp32 restatement of
  its Triton SSIM, :202-269) on small uint8 image pairs: random, a blurred / noisy pair, one
  with max(pred) <= 1 (peak 1), identical images, odd sizes.

Inputs are drawn from one torch.Generator seeded per case; the generator is in this file, so the
fixtures can be rewritten, but the tests read only the stored tensors.
"""
from __future__ import annotations

import json
import os
import sys
import tempfile

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))

TINY = {"width": 8, "enc": [1, 1, 1], "mid": 1, "dec": [1, 1, 1], "train_size": [1, 3, 24, 40],
        "res_fp32_level": 2, "h": 30, "w": 45}


def _seeded_state_dict(shapes: dict, seed: int) -> dict:
    """Conv weights / biases U(-1/sqrt(fan_in), 1/sqrt(fan_in)); LayerNorm weight 1 + 0.1 N,
    bias 0.1 N; beta / gamma 0.2 N (non-zero, so the residual branches matter); the final conv
    scaled by 0.1 to keep the restored image near the input."""
    g = torch.Generator().manual_seed(seed)
    sd = {}
    for k, shape in shapes.items():
        if k.endswith(("beta", "gamma")):
            v = 0.2 * torch.randn(shape, generator=g)
        elif ".norm" in k:
            v = (1.0 if k.endswith("weight") else 0.0) + 0.1 * torch.randn(shape, generator=g)
        else:
            ws = shapes[k[:-len("bias")] + "weight"] if k.endswith("bias") else shape
            fan_in = ws[1] * ws[2] * ws[3]
            v = (torch.rand(shape, generator=g) * 2 - 1) / fan_in ** 0.5
            if k.startswith("ending."):
                v = v * 0.1
        sd[k] = v.float().contiguous()
    return sd


def nafnet_fixture(ref_root: str) -> tuple[dict, dict]:
    from clarus.models import create_model
    from clarus.models.nafnet import state_dict_shapes
    from clarus.ops import Ops

    sd = _seeded_state_dict(state_dict_shapes(TINY["width"], TINY["enc"], TINY["mid"], TINY["dec"]), seed=11)
    g = torch.Generator().manual_seed(12)
    x = torch.rand(1, 3, TINY["h"], TINY["w"], generator=g)
    out = {"input": x}
    out.update({f"sd.{k}": v for k, v in sd.items()})
    with tempfile.TemporaryDirectory() as tmp:
        ckpt = os.path.join(tmp, "tiny.pth")
        torch.save({"params": sd}, ckpt)
        cfg = {"name": "nafnet", "checkpoint": ckpt,
               "network_g": {"type": "NAFNetLocal", "width": TINY["width"], "enc_blk_nums": TINY["enc"],
                             "middle_blk_num": TINY["mid"], "dec_blk_nums": TINY["dec"],
                             "train_size": TINY["train_size"]},
               "options": {"residual_fp32_from_level": TINY["res_fp32_level"]}}
        for tag, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
            ops = Ops(["torch"], dt, torch.device("cpu"))
            model = create_model(cfg, ops, torch.device("cpu"), dt)
            with torch.no_grad():
                out[f"out_{tag}"] = model.forward(x).float().contiguous()
            out[f"tlc_{tag}"] = torch.tensor([list(model._tlc_kernel(lv)) for lv in range(len(TINY["enc"]) + 1)])
    return out, {"tiny": json.dumps(TINY)}


def ops_fixture(ref_root: str) -> dict:
    from clarus.ops.torch_ref import Small, TorchOps

    out = {}
    for tag, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        r = TorchOps(dt, torch.device("cpu"))
        g = torch.Generator().manual_seed(21)

        def rnd(*s, scale=1.0):
            return (torch.randn(*s, generator=g) * scale)

        # linear: TLC-map multiply -> GEMM -> bias -> gate -> GELU -> scale -> residual
        x = rnd(1, 9, 13, 24).to(dt)
        sm = Small(rnd(1, 4, 6, 24).to(dt), 2, 3, 9, 13)
        w = rnd(24, 64, scale=24 ** -0.5).to(dt)
        b, s = rnd(64, scale=0.1), rnd(32, scale=0.5)
        res = rnd(1, 9, 13, 32).to(dt)
        y = r.linear(x, w, b, act="gelu", gate=True, scale=s, residual=res, mul=sm, out_dtype=torch.float32)
        out.update({f"lin1_{tag}.x": x, f"lin1_{tag}.map": sm.data, f"lin1_{tag}.w": w, f"lin1_{tag}.b": b,
                    f"lin1_{tag}.s": s, f"lin1_{tag}.res": res, f"lin1_{tag}.y": y})
        # linear: LN -> GEMM -> bias -> gate -> GELU -> scale -> residual
        x = rnd(1, 7, 10, 32).to(dt)
        w = rnd(32, 48, scale=32 ** -0.5).to(dt)
        b, s = rnd(48, scale=0.1), rnd(24, scale=0.5)
        res = rnd(1, 7, 10, 24).to(dt)
        y = r.linear(x, w, b, ln=True, act="gelu", gate=True, scale=s, residual=res, out_dtype=torch.float32)
        out.update({f"lin3_{tag}.x": x, f"lin3_{tag}.w": w, f"lin3_{tag}.b": b, f"lin3_{tag}.s": s,
                    f"lin3_{tag}.res": res, f"lin3_{tag}.y": y})
        # linear: RMS prologue, no gate, scale + residual, activation-dtype output
        x = rnd(2, 5, 7, 40).to(dt)
        w = rnd(40, 24, scale=40 ** -0.5).to(dt)
        b, s = rnd(24, scale=0.1), rnd(24, scale=0.5)
        res = rnd(2, 5, 7, 24).to(dt)
        y = r.linear(x, w, b, ln="rms", scale=s, residual=res)
        out.update({f"lin2_{tag}.x": x, f"lin2_{tag}.w": w, f"lin2_{tag}.b": b, f"lin2_{tag}.s": s,
                    f"lin2_{tag}.res": res, f"lin2_{tag}.y": y})
        # ln_mul_linear with a GELU multiplier, bias and residual (eps 1e-5)
        x, m = rnd(1, 6, 11, 32).to(dt), rnd(1, 6, 11, 32).to(dt)
        lw, lb = 1 + rnd(32, scale=0.1), rnd(32, scale=0.1)
        w = rnd(32, 16, scale=32 ** -0.5).to(dt)
        b, res = rnd(16, scale=0.1), rnd(1, 6, 11, 16).to(dt)
        y = r.ln_mul_linear(x, lw, lb, m, w, bias=b, m_act="gelu", residual=res, out_dtype=torch.float32)
        out.update({f"lml_{tag}.x": x, f"lml_{tag}.m": m, f"lml_{tag}.lw": lw, f"lml_{tag}.lb": lb,
                    f"lml_{tag}.w": w, f"lml_{tag}.b": b, f"lml_{tag}.res": res, f"lml_{tag}.y": y})
        # conv3x3: nearest x2 input, LeakyReLU, out_scale, residual
        x = rnd(1, 5, 7, 32).to(dt)
        w = rnd(16, 32, 3, 3, scale=(9 * 32) ** -0.5).to(dt)
        b, res = rnd(16, scale=0.1), rnd(1, 10, 14, 16).to(dt)
        y = r.conv3x3(x, w, b, out_dtype=torch.float32, act="lrelu", residual=res, out_scale=0.2, up2=True)
        out.update({f"c3_{tag}.x": x, f"c3_{tag}.w": w, f"c3_{tag}.b": b, f"c3_{tag}.res": res,
                    f"c3_{tag}.y": y})
        # linear_per_image: per-image weights, bias and residual
        x = rnd(2, 6, 5, 48).to(dt)
        w = rnd(2, 48, 48, scale=48 ** -0.5).to(dt)
        b, res = rnd(48, scale=0.1), rnd(2, 6, 5, 48).to(dt)
        y = r.linear_per_image(x, w, residual=res, out_dtype=torch.float32, bias=b)
        out.update({f"lpi_{tag}.x": x, f"lpi_{tag}.w": w, f"lpi_{tag}.b": b, f"lpi_{tag}.res": res,
                    f"lpi_{tag}.y": y})
    return {k: v.contiguous() for k, v in out.items()}


LPF_CASES = [  # (name, n, h, w, k, c, ln, residual)
    ("lpf_none_res", 1, 13, 22, 16, 24, False, True),
    ("lpf_ln", 1, 13, 22, 16, 24, True, False),
    ("lpf_rms_res", 2, 16, 16, 16, 16, "rms", True),
    ("lpf_ln_res", 1, 9, 16, 32, 16, True, True),
]


def freq_fixture(ref_root: str) -> dict:
    from clarus.ops.torch_ref import TorchOps

    out = {}
    for tag, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        r = TorchOps(dt, torch.device("cpu"))
        g = torch.Generator().manual_seed(31)
        for name, n, h, w, k, c, ln, has_res in LPF_CASES:
            x = torch.randn(n, h, w, k, generator=g).to(dt)
            wt = (torch.randn(k, c, generator=g) * k ** -0.5).to(dt)
            b = torch.randn(c, generator=g) * 0.1
            f = torch.randn(c, 8, 5, generator=g)
            res = torch.randn(n, h, w, c, generator=g).to(dt) if has_res else None
            y = r.linear_patch_filter(x, wt, b, f, ln=ln, ln_eps=1e-5, residual=res)
            key = f"{name}_{tag}"
            out.update({f"{key}.x": x, f"{key}.w": wt, f"{key}.b": b, f"{key}.f": f, f"{key}.y": y})
            if res is not None:
                out[f"{key}.res"] = res
    return {k: v.contiguous() for k, v in out.items()}


METRIC_CASES = [("rand", 23, 37), ("blur", 40, 52), ("small", 17, 29), ("same", 21, 19), ("tall", 64, 11)]


def metrics_fixture(ref_root: str) -> dict:
    from clarus.metrics import TorchMetrics, psnr

    g = torch.Generator().manual_seed(41)
    m = TorchMetrics(torch.device("cpu"))
    out = {}
    for name, h, w in METRIC_CASES:
        if name == "small":
            a = torch.randint(0, 2, (h, w, 3), generator=g, dtype=torch.uint8)
            b = torch.randint(0, 2, (h, w, 3), generator=g, dtype=torch.uint8)
        elif name == "blur":
            b = torch.randint(0, 256, (h, w, 3), generator=g, dtype=torch.uint8)
            a = (b.float() * 0.8 + 20 + 8 * torch.randn(h, w, 3, generator=g)).round().clamp(0, 255).to(torch.uint8)
        else:
            a = torch.randint(0, 256, (h, w, 3), generator=g, dtype=torch.uint8)
            b = a.clone() if name == "same" else torch.randint(0, 256, (h, w, 3), generator=g, dtype=torch.uint8)
        res = torch.zeros(2, dtype=torch.float64)
        m.compute(a, b, res)
        out.update({f"{name}.pred": a, f"{name}.gt": b, f"{name}.torch_metrics": res,
                    f"{name}.psnr": torch.tensor([psnr(a.numpy(), b.numpy())], dtype=torch.float64)})
    return out


def main(ref_root: str = "/root/reference", which: str = "all") -> None:
    sys.path.insert(0, os.path.join(ref_root, "python"))
    torch.manual_seed(0)
    written = []
    if which in ("all", "nafnet"):
        tensors, meta = nafnet_fixture(ref_root)
        save_file(tensors, os.path.join(HERE, "nafnet_tiny.safetensors"), metadata=meta)
        written.append("nafnet_tiny.safetensors")
    if which in ("all", "ops"):
        save_file(ops_fixture(ref_root), os.path.join(HERE, "ops_combined.safetensors"))
        written.append("ops_combined.safetensors")
    if which in ("all", "freq"):
        save_file(freq_fixture(ref_root), os.path.join(HERE, "ops_freq.safetensors"),
                  metadata={"cases": json.dumps(LPF_CASES)})
        written.append("ops_freq.safetensors")
    if which in ("all", "metrics"):
        save_file(metrics_fixture(ref_root), os.path.join(HERE, "metrics.safetensors"),
                  metadata={"cases": json.dumps(METRIC_CASES)})
        written.append("metrics.safetensors")
    for f in written:
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main(*sys.argv[1:])
