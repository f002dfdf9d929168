"""Benchmark of the HIP GEMM-family hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-ops] [--no-e2e]

A step is one pass of BASELINE config 2 (NAFNet-w64 720p pointwise GEMMs, bf16 operands, fp32
accumulation): at each of the 5 UNet levels the expand c -> 2c + bias + SimpleGate and the
c -> c + bias, * beta, + residual GEMM, inputs resident in HBM. The step is captured in a HIP
graph (as clarus's worker captures its static-shape forward) and `value` is its algorithmic
TFLOP/s over K replays. Per-op times come from the same K steps launched eagerly behind a
bounded GPU spin (the host queues every launch before the GPU gets to them), each op bracketed
by HIP events on the stream it runs on (torch's current stream), so the per-op times and the
dominant kernel's roofline come from launches a rocprofv3 kernel trace of this command sees,
without host-side launch gaps.

Extra fields of the JSON line:
  roofline      dominant kernel of the step (largest share of the step time) against its bound
  cpu_baseline  the oracle (CPU restatement of the reference PyTorch backend) running the
                same config-2 step on this host's cores (fp32 math, bf16 storage)
  per_op        every config 1-5 op: time, TFLOP/s, GB/s, bound and fraction of the bound.
                Ops outside the step are timed cold: before each rep a read-only pass over
                512 MB (larger than the 256 MB MALL) evicts the caches without leaving dirty
                lines whose write-back would overlap the timed op.
  nafnet_e2e    NAFNet-w64 720p bf16 forward (HIP GEMMs, non-GEMM ops on torch) in ms

  python bench.py --summarize-trace DIR   per-(kernel, grid) durations from a rocprofv3
                                          kernel trace written under DIR
  python bench.py --summarize-e2e DIR     the same for the NAFNet forwards only, per forward

HBM traffic of the step's kernels (roofline.traffic), from two rocprofv3 counter passes of
`python bench.py --pmc-pass` (FETCH_SIZE, then WRITE_SIZE): that mode ends with one plain copy
kernel of known size (256 MiB read + 256 MiB written) followed by each step op once, and
`python bench.py --summarize-pmc FETCH_DIR WRITE_DIR` scales each op's counters by the copy's
(bytes per counted KiB) and writes profiles/pmc_traffic.json.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "per-op TFLOP/s + % MFMA/HBM roofline; NAFNet-w64 720p forward ms, 1 GPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def summarize_trace(directory: str) -> None:
    """Group a rocprofv3 kernel trace by (kernel, grid) and print mean durations in us."""
    files = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {directory}")
    groups: dict = {}
    for f in files:
        with open(f) as fh:
            for row in csv.DictReader(fh):
                name = row.get("Kernel_Name", "?")
                grid = (row.get("Grid_Size_X") or row.get("Grid_Size", "?"), row.get("Grid_Size_Y", ""),
                        row.get("Grid_Size_Z", ""))
                dur = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1000.0
                groups.setdefault((name, grid), []).append(dur)
    rows = sorted(groups.items(), key=lambda kv: -sum(kv[1]))
    print(f"{'calls':>6} {'mean_us':>9} {'median_us':>9} {'total_ms':>9}  grid  kernel")
    for (name, grid), d in rows[:60]:
        short = name if len(name) < 110 else name[:107] + "..."
        print(f"{len(d):6d} {statistics.mean(d):9.2f} {statistics.median(d):9.2f} {sum(d) / 1e3:9.3f}  "
              f"{'x'.join(g for g in grid if g)}  {short}")


def summarize_e2e(directory: str, top: int = 40) -> None:
    """Per-forward kernel time of the NAFNet e2e phase of a bench.py kernel trace: launches from
    the first intro kernel (intro_mfma_kernel / intro_kernel, the NAFNet stem) on, grouped by
    (kernel, grid), divided by the number of forwards in the trace (one intro kernel each)."""
    files = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {directory}")
    rows = []
    for f in files:
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    def is_intro(r):
        name = r.get("Kernel_Name", "")
        return "intro_kernel" in name or "intro_mfma_kernel" in name
    first = next((i for i, r in enumerate(rows) if is_intro(r)), None)
    if first is None:
        raise SystemExit("no NAFNet forward (intro kernel) in the trace")
    e2e = rows[first:]
    nfwd = sum(1 for r in e2e if is_intro(r))
    groups: dict = {}
    for r in e2e:
        name = r.get("Kernel_Name", "?").replace("(anonymous namespace)::", "")
        name = name.split("(")[0].replace("void ", "")
        grid = r.get("Grid_Size_X") or r.get("Grid_Size", "?")
        groups.setdefault((name, grid), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    total = sum(sum(v) for v in groups.values()) / nfwd
    print(f"forwards {nfwd}, launches per forward {len(e2e) / nfwd:.0f}, kernel time per forward {total:.0f} us")
    print(f"{'us/fwd':>8} {'calls':>6} {'mean_us':>8}  grid  kernel")
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]:
        print(f"{sum(d) / nfwd:8.1f} {len(d) / nfwd:6.1f} {statistics.mean(d):8.2f}  {grid}  {name[:100]}")


COPY_BYTES = 256 * 1024 * 1024  # the pmc pass's calibration copy: this many bytes read and written


def _pmc_dispatches(directory: str, counter: str) -> list:
    """(dispatch id, kernel name, counter value) of every dispatch in a rocprofv3 --pmc run."""
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {directory}")
    vals: dict = {}
    for f in files:
        with open(f) as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                key = int(row["Dispatch_Id"])
                name, v = row.get("Kernel_Name", "?"), float(row["Counter_Value"])
                prev = vals.get(key)
                vals[key] = (name, v + (prev[1] if prev else 0.0))
    return [(k, vals[k][0], vals[k][1]) for k in sorted(vals)]


def summarize_pmc(fetch_dir: str, write_dir: str) -> None:
    """Per-op HBM bytes of the step from the two counter passes of `--pmc-pass` (see above)."""
    from clarus_amd.workloads import config2_names
    names = config2_names()
    out = {"ops": {}, "copy_bytes": COPY_BYTES}
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        d = _pmc_dispatches(directory, counter)
        tail = d[-(len(names) + 1):]
        copy, ops = tail[0], tail[1:]
        if "clarus" in copy[1] or not all("clarus" in o[1] for o in ops):
            raise SystemExit(f"{counter}: the last dispatches are not the copy + step ops: {[t[1][:40] for t in tail]}")
        factor = COPY_BYTES / (copy[2] * 1024.0)  # bytes per counted KiB, from the known copy
        out[f"{counter.lower()}_copy_kib"] = copy[2]
        out[f"{counter.lower()}_factor"] = round(factor, 4)
        for nm, o in zip(names, ops):
            out["ops"].setdefault(nm, {})[counter.lower() + "_bytes"] = round(o[2] * 1024.0 * factor)
            out["ops"][nm]["kernel"] = o[1][:120]
    for nm, v in out["ops"].items():
        v["bytes_per_launch"] = v.get("fetch_size_bytes", 0) + v.get("write_size_bytes", 0)
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out, indent=1))


def cpu_baseline_config2(steps_cpu: int = 3) -> dict:
    """The oracle running the config-2 step on this host's cores (CPU leg only)."""
    import torch

    from clarus_amd.workloads import config2_cases
    from oracle.torch_ref import TorchRef
    threads = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "16") or 16))
    torch.set_num_threads(threads)
    ref = TorchRef(torch.bfloat16, "cpu")

    class _Shim:  # builds the config-2 inputs on the CPU through the oracle's linear
        def linear(self, *a, **k):
            return ref.linear(*a, **k)
    cases = config2_cases(_Shim(), "cpu")
    flops = sum(c.flops for c in cases)
    work = []
    for c in cases:
        d = c.cpu
        if "expand" in c.name:
            work.append(lambda d=d: ref.linear(d["x"], d["we"], d["be"], gate=True))
        else:
            u = ref.linear(d["x"], d["we"], d["be"], gate=True)
            work.append(lambda d=d, u=u: ref.linear(u, d["wc"], d["bc"], scale=d["beta"], residual=d["r"],
                                                     out_dtype=d["rdt"]))
    for fn in work:  # warm-up
        fn()
    times = []
    for _ in range(steps_cpu):
        t0 = time.perf_counter()
        for fn in work:
            fn()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            model = next((ln.split(":", 1)[1].strip() for ln in fh if ln.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "ms_per_step": round(t * 1e3, 1), "cpu_model": model,
            "sample": f"the full config-2 step (10 GEMMs, {flops / 1e9:.1f} GFLOP) on the oracle "
                      f"(fp32 math, bf16 storage), 1 warm-up + median of {steps_cpu} reps"}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=30, help="cold reps per op outside the step")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ops", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--summarize-trace", default=None)
    ap.add_argument("--summarize-e2e", default=None, help="per-forward kernel breakdown of the NAFNet e2e phase")
    ap.add_argument("--pmc-pass", action="store_true", help="one copy + each step op once (counter runs)")
    ap.add_argument("--summarize-pmc", nargs=2, default=None, metavar=("FETCH_DIR", "WRITE_DIR"))
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_e2e:
        summarize_e2e(args.summarize_e2e)
        return
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the path shards "
              f"data-parallel over images with no communication, so the per-GPU value is the N=1 value",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from clarus_amd import workloads as wl
    from clarus_amd.hip_ops import HipOps
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs the MI355X (no HIP device visible)")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    hip = HipOps(torch.bfloat16, dev)
    hip32 = HipOps(torch.float32, dev)
    stream = torch.cuda.current_stream(dev)

    # ------------------------------------------------------------ the timed config-2 step
    step = wl.config2_cases(hip, dev)
    flops_step = sum(c.flops for c in step)
    log(f"[bench] config-2 step: {len(step)} GEMMs, {flops_step / 1e9:.2f} GFLOP")
    if args.pmc_pass:  # the last dispatches of the process: the calibration copy, then each op once
        for c in step:
            c.run()
        src = torch.randn(COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        keep = []
        torch.cuda.synchronize()
        torch.mul(src, 1.0, out=dst)
        for c in step:
            keep.append(c.run())
        torch.cuda.synchronize()
        log(f"[bench] pmc pass: copy of {COPY_BYTES} B, then {[c.name for c in step]}")
        return
    # the step as one HIP graph (timed for `value`), captured on a side stream after an eager
    # warm-up: no host-side launch overhead enters the timed region
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for _ in range(max(args.warmup, 1)):
            for c in step:
                c.run()
    torch.cuda.synchronize()
    g_step = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_step, stream=side):
        for c in step:
            c.run()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        g_step.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        g_step.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    # per-op times: the same K steps launched eagerly behind a bounded GPU spin, so the host has
    # queued every timed launch before the GPU reaches them (kernels run back to back, no host
    # launch gaps inside the events)
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in step]
          for _ in range(args.steps)]
    torch.cuda._sleep(int(2.4e8))  # ~0.1 s of spinning
    for s in range(args.steps):
        for i, c in enumerate(step):
            ev[s][i][0].record(stream)
            c.run()
            ev[s][i][1].record(stream)
    torch.cuda.synchronize()
    per_step_op = []
    for i, c in enumerate(step):
        us = statistics.mean(ev[s][i][0].elapsed_time(ev[s][i][1]) * 1e3 for s in range(args.steps))
        per_step_op.append(us)
    value = flops_step / (ms_step / 1e3) / 1e12
    log(f"[bench] step {ms_step:.3f} ms -> {value:.1f} TFLOP/s (graph replays; eager ops sum {sum(per_step_op):.1f} us)")

    def op_row(c, us):
        tb, bound = c.t_bound()
        return {"op": c.name, "config": c.config, "dtype": c.dtype, "gflop": round(c.flops / 1e9, 3),
                "mb": round(c.nbytes / 1e6, 2), "us": round(us, 2), "tflops": round(c.flops / us / 1e6, 2),
                "gbs": round(c.nbytes / us / 1e3, 1), "bound": bound, "t_bound_us": round(tb * 1e6, 2),
                "frac": round(tb * 1e6 / us, 3)}
    rows = [op_row(c, us) for c, us in zip(step, per_step_op)]

    # dominant kernel of the step
    di = max(range(len(step)), key=lambda i: per_step_op[i])
    dc, dus = step[di], per_step_op[di]
    tb, bound = dc.t_bound()
    if bound == "hbm":
        ach, peak, unit = dc.nbytes / dus / 1e3, wl.PEAK_HBM / 1e9, "GB/s"
    else:
        ach, peak, unit = dc.flops / dus / 1e6, wl.PEAK_FLOPS[dc.dtype] / 1e12, "TFLOP/s"
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as fh:
            t = json.load(fh)
        traffic = t.get("ops", {}).get(dc.name, {}).get("bytes_per_launch")
    roofline = {"bound": bound, "achieved": round(ach, 1), "peak": peak, "unit": unit, "frac": round(ach / peak, 3),
                "traffic": traffic, "op": dc.name, "avg_us": round(dus, 2),
                "algorithmic_bytes": int(dc.nbytes), "algorithmic_flops": int(dc.flops)}

    # ------------------------------------------------------------ other configs, cold per op
    if not args.no_ops:
        flush = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)  # > MALL (256 MB)
        sink = torch.empty((), dtype=torch.float32, device=dev)
        others = (wl.config1_cases(hip32, dev) + wl.config3_cases(hip32, dev) + wl.config4_cases(hip, hip32, dev)
                  + wl.config5_cases(hip, dev))
        for c in others:
            for _ in range(3):
                c.run()
            ts = []
            for _ in range(args.reps):
                torch.sum(flush, dim=0, out=sink)  # reads 512 MB, writes 4 bytes
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                c.run()
                b.record(stream)
                ts.append((a, b))
            torch.cuda.synchronize()
            us = statistics.median(a.elapsed_time(b) * 1e3 for a, b in ts)
            rows.append(op_row(c, us))
        del flush, sink
    for r in rows:
        log(f"[op] cfg{r['config']} {r['op']:<44} {r['dtype']:>4} {r['us']:9.2f} us {r['tflops']:8.1f} TF/s "
            f"{r['gbs']:8.0f} GB/s  {r['bound']:>4} bound {r['t_bound_us']:8.2f} us  frac {r['frac']:.3f}")

    # ------------------------------------------------------------ NAFNet e2e
    e2e = None
    if not args.no_e2e:
        try:
            from clarus_amd import nafnet
            e2e = nafnet.bench_forward(dev, log=log)
        except ImportError:
            e2e = None

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle on the host cores) ...")
        cpu = cpu_baseline_config2()
        log(f"[bench] cpu baseline {cpu['value']} TFLOP/s on {cpu['cores']} threads ({cpu['ms_per_step']} ms/step)")

    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) activations, random-init weights)",
        "config": {"workload": "BASELINE config 2: NAFNet-w64 720p pointwise GEMMs (expand+gate and c->c+scale+res "
                               "at c=64..1024), bf16 operands, fp32 accumulate", "global_batch": 1,
                   "parallelism": "none (1 GPU)"},
        "roofline": roofline, "cpu_baseline": cpu, "per_op": rows, "nafnet_e2e": e2e,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
