"""bench.py's printed line: one strict-JSON line that the driver's 8000-character stdout tail
holds whole, with the keys the measurement contract requires (CPU only)."""
import json
import math

import bench


def _rows(n, name_len):
    return [{"op": ("op %d " % i) + "x" * name_len, "us": 12.345 + i, "tflops": 100.0, "bound": "hbm",
             "frac": 0.5, "traffic_ratio": None if i % 3 else 1.02, "cpu_ms": 1.5, "gbs": 1e3,
             "kernel": "k" * 80, "timing": "cold (512 MB read before each rep), median"} for i in range(n)]


def _head():
    return {"metric": bench.METRIC, "value": 320.1, "unit": "TFLOP/s", "n_gpus": 1, "steps": 20, "warmup": 5,
            "ms_per_step": 0.354, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic", "config": {"workload": "w" * 150},
            "roofline": {"bound": "hbm", "achieved": 5750.0, "peak": 8000.0, "unit": "GB/s", "frac": 0.718,
                         "traffic": 3.6e8, "op": "c64 c->c+scale+res", "kernel": "k" * 60},
            "cpu_baseline": {"value": 0.28, "unit": "TFLOP/s", "cores": 16, "kind": "port", "sample": "s" * 200}}


def _e2e():
    served = {"linear": ["hip"], "up": ["hip"], "down": ["hip"]}
    return {"reference_block": {"ms": 7.98, "eager_ms": 8.08, "served": served},
            "fused_pairs": {"ms": 6.69, "eager_ms": 6.75, "served": served},
            "cpu": {"ms": 4315.0, "threads": 16}}


def test_line_fits_and_parses():
    text = bench.final_line(_head(), _rows(50, 40), _e2e(), "/x/gpurun_out/bench_per_op.json")
    assert "\n" not in text and len(text) <= bench.LINE_LIMIT < 8000
    d = json.loads(text)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d
    assert d["per_op_cols"] == bench.PER_OP_COLS and len(d["per_op"]) == 50
    assert d["per_op"][0][1] == 12.345 and d["per_op"][1][5] is None
    assert d["nafnet_e2e"]["ms"] == 7.98 and d["nafnet_e2e"]["fused_ops_ms"] == 6.69
    assert d["nafnet_e2e"]["all_hip"] is True


def test_line_shrinks_long_rows_and_drops_nonfinite():
    rows = _rows(90, 200)
    rows[0]["us"] = math.nan
    rows[1]["frac"] = math.inf
    text = bench.final_line(_head(), rows, None, None)
    assert len(text) <= bench.LINE_LIMIT
    d = json.loads(text)  # strict: a NaN would not parse as JSON elsewhere
    assert "NaN" not in text and "Infinity" not in text
    assert d["nafnet_e2e"] if "nafnet_e2e" in d else True
    assert d["per_op"] is None or all(len(r[0]) <= 60 for r in d["per_op"])
