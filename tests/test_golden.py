"""Golden vectors written by the reference implementation itself (tests/golden/make_golden.py).

CPU: the oracle and the NAFNet harness reproduce the reference's outputs.
  * the tiny NAFNetLocal forward (reference model adapter on its PyTorch backend) through
    clarus_amd.nafnet.NAFNet with every op on the oracle, fp32 and bf16 activations, and the
    TLC windows the reference computed per level;
  * combined-epilogue calls of the reference TorchOps through the oracle: linear with a
    TLC-map multiply or LN prologue and bias + gate + GELU + scale + residual, RMS linear,
    ln_mul_linear, conv3x3 with up2 + LeakyReLU + out_scale + residual, linear_per_image with
    bias + residual.
  * linear_patch_filter calls of the reference TorchOps (LN / RMS / none, residual or not, fp32
    and bf16, reflect-padded sizes) through the oracle, bit for bit; an oracle that rounded the
    GEMM output to the activation dtype before the filter does not reproduce the bf16 cases.
GPU (tests/test_hip_golden.py): the same fixtures through the `hip` backend.
"""
from __future__ import annotations

import json
import os

import pytest
import torch
from safetensors.torch import load_file, safe_open

from clarus_amd.dispatch import Backend, Ops, register_backend
from clarus_amd.nafnet import NAFNet
from oracle.torch_ref import Small, TorchRef

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


def load_nafnet_fixture():
    path = os.path.join(GOLDEN, "nafnet_tiny.safetensors")
    with safe_open(path, "pt") as f:
        tiny = json.loads(f.metadata()["tiny"])
    t = load_file(path)
    sd = {k[3:]: v for k, v in t.items() if k.startswith("sd.")}
    return tiny, sd, t


def load_ops_fixture():
    return load_file(os.path.join(GOLDEN, "ops_combined.safetensors"))


def load_freq_fixture():
    """{case: (inputs dict, ln mode)} of ops_freq.safetensors."""
    path = os.path.join(GOLDEN, "ops_freq.safetensors")
    with safe_open(path, "pt") as f:
        cases = json.loads(f.metadata()["cases"])
    t = load_file(path)
    out = {}
    for name, *_, ln, _res in cases:
        for tag in DT:
            key = f"{name}_{tag}"
            out[key] = ({k.split(".", 1)[1]: v for k, v in t.items() if k.startswith(key + ".")}, ln)
    return out


def run_linear_patch_filter(r, a, ln, dev, out_fp32=False):
    """linear_patch_filter of one ops_freq case on backend-like `r` (ln_eps 1e-5, as written)."""
    g = {k: v.to(dev) for k, v in a.items()}
    if out_fp32:  # the same chain with the final cast left out (the oracle's value before rounding)
        y = r.linear(g["x"], g["w"], g["b"], ln=ln, ln_eps=1e-5, out_dtype=torch.float32)
        return r.patch_filter(y, g["f"], residual=g.get("res"), out_dtype=torch.float32)
    return r.linear_patch_filter(g["x"], g["w"], g["b"], g["f"], ln=ln, ln_eps=1e-5, residual=g.get("res"))


def tiny_nafnet(ops, tiny, sd):
    return NAFNet(ops, width=tiny["width"], enc=tiny["enc"], mid=tiny["mid"], dec=tiny["dec"],
                  tlc=tuple(tiny["train_size"][-2:]), res_fp32_level=tiny["res_fp32_level"], state_dict=sd)


class _OracleBackend(Backend):
    name = "oracle"

    def __init__(self, dtype, device):
        super().__init__(dtype, device)
        self._r = TorchRef(dtype, device)

    def __getattr__(self, op):
        if op.startswith("_"):
            raise AttributeError(op)
        return getattr(self._r, op)


def run_combined(r, t, tag, dev):
    """Every combined call of ops_combined.safetensors on backend-like `r`: {case: output}."""
    g = {k: v.to(dev) for k, v in t.items() if k.split(".")[0].endswith(tag)}

    def a(case, name):
        return g[f"{case}_{tag}.{name}"]
    out = {}
    sm = Small(a("lin1", "map"), 2, 3, 9, 13)
    out["lin1"] = r.linear(a("lin1", "x"), a("lin1", "w"), a("lin1", "b"), act="gelu", gate=True,
                           scale=a("lin1", "s"), residual=a("lin1", "res"), mul=sm, out_dtype=torch.float32)
    out["lin3"] = r.linear(a("lin3", "x"), a("lin3", "w"), a("lin3", "b"), ln=True, act="gelu", gate=True,
                           scale=a("lin3", "s"), residual=a("lin3", "res"), out_dtype=torch.float32)
    out["lin2"] = r.linear(a("lin2", "x"), a("lin2", "w"), a("lin2", "b"), ln="rms", scale=a("lin2", "s"),
                           residual=a("lin2", "res"))
    out["lml"] = r.ln_mul_linear(a("lml", "x"), a("lml", "lw"), a("lml", "lb"), a("lml", "m"), a("lml", "w"),
                                 bias=a("lml", "b"), m_act="gelu", residual=a("lml", "res"),
                                 out_dtype=torch.float32)
    out["c3"] = r.conv3x3(a("c3", "x"), a("c3", "w"), a("c3", "b"), out_dtype=torch.float32, act="lrelu",
                          residual=a("c3", "res"), out_scale=0.2, up2=True)
    out["lpi"] = r.linear_per_image(a("lpi", "x"), a("lpi", "w"), residual=a("lpi", "res"),
                                    out_dtype=torch.float32, bias=a("lpi", "b"))
    return out


def test_nafnet_tlc_windows_match_reference():
    register_backend("oracle")(_OracleBackend)
    tiny, sd, t = load_nafnet_fixture()
    m = tiny_nafnet(Ops(["oracle"], torch.float32, torch.device("cpu"), log=lambda *a: None), tiny, sd)
    for tag in DT:
        want = [tuple(r) for r in t[f"tlc_{tag}"].tolist()]
        assert [m.tlc_kernel(lv) for lv in range(len(tiny["enc"]) + 1)] == want


@pytest.mark.parametrize("tag", ["fp32", "bf16"])
def test_oracle_nafnet_matches_reference(tag):
    register_backend("oracle")(_OracleBackend)
    tiny, sd, t = load_nafnet_fixture()
    ops = Ops(["oracle"], DT[tag], torch.device("cpu"), log=lambda *a: None)
    y = tiny_nafnet(ops, tiny, sd).forward(t["input"]).float()
    ref = t[f"out_{tag}"]
    assert y.shape == ref.shape == (1, 3, tiny["h"], tiny["w"])
    # same torch ops in the same order on the same CPU: the restatement is exact
    assert torch.equal(y, ref), (y - ref).abs().max().item()


@pytest.mark.parametrize("tag", ["fp32", "bf16"])
def test_oracle_combined_ops_match_reference(tag):
    t = load_ops_fixture()
    got = run_combined(TorchRef(DT[tag], "cpu"), t, tag, "cpu")
    for case, y in got.items():
        ref = t[f"{case}_{tag}.y"]
        assert y.dtype == ref.dtype and y.shape == ref.shape, case
        assert torch.equal(y, ref), (case, (y.float() - ref.float()).abs().max().item())


def test_oracle_linear_patch_filter_matches_reference():
    cases = load_freq_fixture()
    assert len(cases) == 8
    for key, (a, ln) in cases.items():
        tag = key.rsplit("_", 1)[1]
        y = run_linear_patch_filter(TorchRef(DT[tag], "cpu"), a, ln, "cpu")
        assert y.dtype == a["y"].dtype == DT[tag] and y.shape == a["y"].shape, key
        assert torch.equal(y, a["y"]), (key, (y.float() - a["y"].float()).abs().max().item())


class _RoundedIntermediate(TorchRef):
    """A planted mistake: the GEMM output rounded to the activation dtype before the filter."""

    def linear_patch_filter(self, x, w, bias, f, ln=False, ln_eps=1e-6, residual=None):
        y = self.linear(x, w, bias, ln=ln, ln_eps=ln_eps)
        return self.patch_filter(y, f, residual=residual)


def test_linear_patch_filter_fixture_catches_a_rounded_intermediate():
    cases = load_freq_fixture()
    wrong = 0
    for key, (a, ln) in cases.items():
        if key.endswith("_bf16"):
            y = run_linear_patch_filter(_RoundedIntermediate(torch.bfloat16, "cpu"), a, ln, "cpu")
            wrong += not torch.equal(y, a["y"])
    assert wrong == 4
