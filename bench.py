"""Benchmark of the HIP GEMM-family hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--reps R] [--no-cpu] [--no-ops] [--no-e2e]

A step is one pass of BASELINE config 2 (NAFNet-w64 720p pointwise GEMMs, bf16 operands, fp32
accumulation): at each of the 5 UNet levels the expand c -> 2c + bias + SimpleGate and the
c -> c + bias, * beta, + residual GEMM, inputs resident in HBM. The step is captured in a HIP
graph (as clarus's worker captures its static-shape forward) and `value` is its algorithmic
TFLOP/s over K replays (default 50).

Extra fields of the JSON line:
  roofline      dominant kernel of the step (largest share of the step time) against its bound;
                its duration comes from HIP events on torch's current stream (where it launches)
  cpu_baseline  the oracle (CPU restatement of the reference PyTorch backend) running the same
                config-2 step on this host's cores (fp32 math, bf16 storage; threads = the CPUs
                this process may use, model from lscpu; 1 warm-up + median of 3)
  per_op        every config 1-5 op and the fused NAFNet level-3 pair: median of R (default 50)
                event-timed reps, TFLOP/s, GB/s, the bound and the fraction of it (plus the
                fraction of both the HBM and the MFMA ceiling), the kernel the library chose, the
                CPU time of the same op on the oracle, and (from profiles/pmc_ops.json) the HBM
                traffic over the algorithmic bytes and the MFMA busy fraction. The step's ops are
                timed eagerly behind a GPU spin (back to back, as in the step); the others cold:
                before each rep a read-only pass over 512 MB (more than the 256 MB MALL) evicts
                the caches without leaving dirty lines whose write-back would overlap the op.
  nafnet_e2e    NAFNet-w64 720p bf16 forward in ms (median of graph replays), with the fused ops
                (residual GEMM -> LayerNorm GEMM pairs at width 512, the feed-forward half as one op
                at the other widths) and with the reference's unchanged five-linear block, and the
                same forward on the oracle on the CPU

  python bench.py --summarize-trace DIR   per-(kernel, grid) durations from a rocprofv3 kernel trace
  python bench.py --summarize-e2e DIR     the same for the NAFNet forwards only, per forward

Counters: `python bench.py --pmc-pass` runs a calibration copy kernel of known size (256 MiB read
+ 256 MiB written) and then every benchmark op once, with marker kernels between them, and writes
the op list to --pmc-cases. Run it under separate rocprofv3 --pmc passes (FETCH_SIZE; WRITE_SIZE;
MfmaUtil GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_VALU_MFMA_MOPS_F32), then
`python bench.py --summarize-pmc DIR...` writes profiles/pmc_ops.json: per op the HBM bytes
(counters scaled by the copy's reading), their ratio to the algorithmic bytes, the MFMA busy
fraction and the counted MFMA flops over the algorithmic flops.
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
    """Per-forward kernel time of the NAFNet e2e phase of a bench.py kernel trace: the launches from
    the first intro kernel (intro_mfma_kernel / intro_kernel, the NAFNet stem) on, cut into forwards
    at each intro kernel, each forward classed by its call pattern (the fused ops when it launches
    a fused pair kernel, pair_kernel or gemm_rowln_kernel<true>, else the reference block),
    grouped by (kernel, grid) and
    divided by the number of forwards of that pattern."""
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
    starts = [i for i, r in enumerate(rows) if is_intro(r)]
    if not starts:
        raise SystemExit("no NAFNet forward (intro kernel) in the trace")
    forwards = [rows[a:b] for a, b in zip(starts, starts[1:] + [len(rows)])]
    # the last forward runs to the end of the trace: cut it after its ending conv (conv_halo_kernel<16, ...)
    last = forwards[-1]
    ends = [i for i, r in enumerate(last) if "conv_halo_kernel<16" in r.get("Kernel_Name", "")]
    if ends:
        forwards[-1] = last[:ends[-1] + 1]
    patterns = {"fused ops (linear_ln_linear, linear_gate_linear)": [], "reference block (five linear calls)": []}
    for fw in forwards:
        fused = any("gemm_rowln_kernel<true>" in r.get("Kernel_Name", "") or "pair_kernel" in r.get("Kernel_Name", "")
                    for r in fw)
        patterns["fused ops (linear_ln_linear, linear_gate_linear)" if fused else "reference block (five linear calls)"].append(fw)
    for pat, fws in patterns.items():
        if not fws:
            continue
        nfwd = len(fws)
        groups: dict = {}
        for fw in fws:
            for r in fw:
                name = r.get("Kernel_Name", "?").replace("(anonymous namespace)::", "")
                name = name.split("(")[0].replace("void ", "")
                grid = r.get("Grid_Size_X") or r.get("Grid_Size", "?")
                groups.setdefault((name, grid), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
        total = sum(sum(v) for v in groups.values()) / nfwd
        nl = sum(len(fw) for fw in fws) / nfwd
        print(f"== {pat}: forwards {nfwd}, launches per forward {nl:.0f}, kernel time per forward {total:.0f} us")
        print(f"{'us/fwd':>8} {'calls':>6} {'mean_us':>8}  grid  kernel")
        for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]:
            print(f"{sum(d) / nfwd:8.1f} {len(d) / nfwd:6.1f} {statistics.mean(d):8.2f}  {grid}  {name[:100]}")
        print()


COPY_BYTES = 256 * 1024 * 1024  # the pmc pass's calibration copy: this many bytes read and written
SIMD_PER_GPU = 256 * 4


def _pmc_rows(directory: str) -> list:
    """[(dispatch id, kernel name, {counter: value})] of every dispatch in a rocprofv3 --pmc run,
    in dispatch order."""
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {directory}")
    vals: dict = {}
    for f in files:
        with open(f) as fh:
            for row in csv.DictReader(fh):
                key = int(row["Dispatch_Id"])
                name = row.get("Kernel_Name", "?")
                entry = vals.setdefault(key, (name, {}))
                cn = row["Counter_Name"]
                entry[1][cn] = entry[1].get(cn, 0.0) + float(row["Counter_Value"])
    return [(k, vals[k][0], vals[k][1]) for k in sorted(vals)]


def _is_marker(name: str) -> bool:
    return "spin_kernel" in name


def _pmc_groups(rows: list, n_ops: int) -> tuple:
    """Splits the tail of a --pmc-pass run into the calibration copy and one dispatch group per
    op: the pass issues two marker kernels, the copy, then a marker before every op and one
    after the last."""
    start = None
    for i in range(len(rows) - 1, 0, -1):
        if _is_marker(rows[i][1]) and _is_marker(rows[i - 1][1]):
            start = i + 1
            break
    if start is None:
        raise SystemExit("no double marker (the --pmc-pass calibration start) in the counter run")
    tail = rows[start:]
    groups, cur = [], []
    for r in tail:
        if _is_marker(r[1]):
            groups.append(cur)
            cur = []
        else:
            cur.append(r)
    copy, ops = groups[0], groups[1:]
    if len(copy) != 1 or len(ops) != n_ops or any(not g for g in ops):
        raise SystemExit(f"counter run: expected the copy and {n_ops} ops, found {[len(g) for g in groups]}")
    return copy[0], ops


def summarize_pmc(dirs: list, cases_file: str) -> None:
    """Per-op HBM traffic and MFMA activity of every benchmark op, from the counter runs of
    `bench.py --pmc-pass` (any mix of FETCH_SIZE, WRITE_SIZE and MfmaUtil / GRBM_GUI_ACTIVE /
    SQ_INSTS_VALU_MFMA_MOPS_* passes; cases_file: the op list the pass wrote). FETCH_SIZE /
    WRITE_SIZE (KiB per dispatch) are scaled by what each counter reads for the pass's calibration
    copy of COPY_BYTES; writes profiles/pmc_ops.json."""
    with open(cases_file) as fh:
        meta = [tuple(m) for m in json.load(fh)]  # (name, config, flops, bytes) in dispatch order
    out = {"copy_bytes": COPY_BYTES, "simd_per_gpu": SIMD_PER_GPU, "ops": {}}
    for directory in dirs:
        rows = _pmc_rows(directory)
        copy, ops = _pmc_groups(rows, len(meta))
        counters = sorted(copy[2])
        out.setdefault("passes", []).append({"dir": os.path.basename(os.path.normpath(directory)),
                                             "counters": counters})
        for cn in ("FETCH_SIZE", "WRITE_SIZE"):
            if cn in copy[2]:
                out[f"{cn.lower()}_factor"] = round(COPY_BYTES / (copy[2][cn] * 1024.0), 4)
        for (name, _cfg, flops, nbytes), grp in zip(meta, ops):
            o = out["ops"].setdefault(name, {"algorithmic_bytes": nbytes, "algorithmic_flops": flops})
            o["kernels"] = sorted({g[1].replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")[:100]
                                   for g in grp})
            for cn in ("FETCH_SIZE", "WRITE_SIZE"):
                if cn in copy[2]:
                    o[f"{cn.lower()}_bytes"] = round(sum(g[2].get(cn, 0.0) for g in grp) * 1024.0
                                                     * out[f"{cn.lower()}_factor"])
            if "MfmaUtil" in copy[2]:
                gui = [g[2].get("GRBM_GUI_ACTIVE", 1.0) for g in grp]
                util = [g[2].get("MfmaUtil", 0.0) for g in grp]
                o["mfma_util"] = round(sum(u * w for u, w in zip(util, gui)) / max(sum(gui), 1.0) / 100.0, 4)
                mops = sum(g[2].get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) + g[2].get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0)
                           for g in grp)
                o["mfma_flops_counted"] = mops * 512.0
                o["mfma_flops_ratio"] = round(mops * 512.0 / flops, 3) if flops else None
    for o in out["ops"].values():
        if "fetch_size_bytes" in o and "write_size_bytes" in o:
            o["traffic_bytes"] = o["fetch_size_bytes"] + o["write_size_bytes"]
            o["traffic_ratio"] = round(o["traffic_bytes"] / o["algorithmic_bytes"], 3)
    path = os.path.join(ROOT, "profiles", "pmc_ops.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out, indent=1))


def host_cpu() -> tuple[int, str]:
    """(threads to use = the CPUs this process may run on, the lscpu model name)."""
    threads = len(os.sched_getaffinity(0))
    model = ""
    try:
        import subprocess
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((ln.split(":", 1)[1].strip() for ln in txt.splitlines() if ln.startswith("Model name")), "")
    except (OSError, subprocess.SubprocessError):
        pass
    return threads, model


def time_cpu(fn, reps: int = 3) -> float:
    """One warm-up, then the median of `reps` perf_counter timings, in seconds."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


class _CpuMetrics:
    """The float64 metric definitions on the host (the CPU leg of the metrics row)."""

    @staticmethod
    def metrics(pred, gt):
        from oracle import metrics_ref
        return metrics_ref.psnr(pred, gt), metrics_ref.ssim(pred, gt)


class _OracleBackend:
    """The oracle behind the op dispatch (CPU baseline legs only)."""

    def __init__(self, dtype, device):
        from oracle.torch_ref import TorchRef
        self.name = "oracle"
        self.dtype, self.device = dtype, device
        self._r = TorchRef(dtype, device)

    def __getattr__(self, op):
        if op.startswith("_") or op == "linear_ln_linear":
            raise AttributeError(op)
        return getattr(self._r, op)


def cpu_legs(step, others, e2e_reps: int, log=print) -> dict:
    """CPU times of the same ops on the oracle (the reference PyTorch backend's semantics) on
    this host's cores: every per-op row, the config-2 step (cpu_baseline) and the NAFNet-w64
    720p forward (the reference's five-linear block on the oracle's ops)."""
    import torch

    from clarus_amd.dispatch import register_backend
    from oracle.torch_ref import TorchRef
    threads, model = host_cpu()
    torch.set_num_threads(threads)
    refs = {d: TorchRef(d, "cpu") for d in (torch.bfloat16, torch.float32)}
    per_op = {}
    for c in step + others:
        if c.cpu_run is None:
            continue
        r = refs[torch.float32 if c.dtype == "fp32" else torch.bfloat16]
        if c.config == 4:
            r = refs[torch.float32 if c.name.endswith("fp32") else torch.bfloat16]
        if c.dtype == "fp64":
            r = _CpuMetrics()
        with torch.no_grad():
            t = time_cpu(lambda c=c, r=r: c.cpu_run(r)) * c.cpu_scale
        per_op[c.name] = (t * 1e3, c.cpu_sample)
        log(f"[cpu] {c.name:<48} {t * 1e3:10.2f} ms{'  (' + c.cpu_sample + ')' if c.cpu_sample else ''}")
    flops = sum(c.flops for c in step)
    r16 = refs[torch.bfloat16]
    with torch.no_grad():
        t_step = time_cpu(lambda: [c.cpu_run(r16) for c in step])
    base = {"value": round(flops / t_step / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "ms_per_step": round(t_step * 1e3, 1), "cpu_model": model,
            "sample": f"the full config-2 step (10 GEMMs, {flops / 1e9:.1f} GFLOP) on the oracle (fp32 math, bf16 "
                      f"storage), {threads} threads, 1 warm-up + median of 3 reps"}
    e2e = None
    if e2e_reps > 0:
        from clarus_amd.nafnet import NAFNet
        register_backend("bench_oracle")(_OracleBackend)
        from clarus_amd.dispatch import Ops
        ops = Ops(["bench_oracle"], torch.bfloat16, torch.device("cpu"), log=lambda *a: None)
        model_net = NAFNet(ops, fused_pairs=False)
        x = torch.rand(1, 3, 720, 1280, generator=torch.Generator().manual_seed(1))
        t = time_cpu(lambda: model_net.forward(x), reps=e2e_reps)
        e2e = {"ms": round(t * 1e3, 1), "reps": e2e_reps, "threads": threads, "cpu_model": model,
               "what": "NAFNet-w64 720p forward on the oracle (bf16 storage, fp32 math), the reference's block"}
        log(f"[cpu] NAFNet-w64 720p forward {t * 1e3:.0f} ms on {threads} threads")
    return {"baseline": base, "per_op_ms": per_op, "e2e": e2e}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=50, help="event-timed reps per op row")
    ap.add_argument("--e2e-reps", type=int, default=50, help="graph replays per NAFNet forward pattern")
    ap.add_argument("--cpu-e2e-reps", type=int, default=3, help="CPU NAFNet forwards after one warm-up (0: skip)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ops", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--summarize-trace", default=None)
    ap.add_argument("--summarize-e2e", default=None, help="per-forward kernel breakdown of the NAFNet e2e phase")
    ap.add_argument("--pmc-pass", action="store_true", help="calibration copy + every benchmark op once (counter runs)")
    ap.add_argument("--summarize-pmc", nargs="+", default=None, metavar="DIR")
    ap.add_argument("--pmc-cases", default=os.path.join(ROOT, "gpurun_out", "pmc_cases.json"),
                    help="the op list a --pmc-pass run writes and --summarize-pmc reads")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_e2e:
        summarize_e2e(args.summarize_e2e)
        return
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc, args.pmc_cases)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the path shards "
              f"data-parallel over images with no communication, so the per-GPU value is the N=1 value",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from clarus_amd import _lib
    from clarus_amd import workloads as wl
    from clarus_amd.hip_ops import HipOps
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs the MI355X (no HIP device visible)")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    hip = HipOps(torch.bfloat16, dev)
    hip32 = HipOps(torch.float32, dev)
    stream = torch.cuda.current_stream(dev)

    step = wl.config2_cases(hip, dev)
    flops_step = sum(c.flops for c in step)
    log(f"[bench] config-2 step: {len(step)} GEMMs, {flops_step / 1e9:.2f} GFLOP")
    others = [] if args.no_ops else (wl.config1_cases(hip32, dev) + wl.config3_cases(hip32, dev)
                                     + wl.config4_cases(hip, hip32, dev) + wl.config5_cases(hip, dev)
                                     + [wl.fftformer_dffn_case(hip, dev), wl.nafnet_pair_case(hip, dev),
                                        wl.nafnet_ffn_case(hip, dev), wl.nafnet_lndw_case(hip, dev),
                                        wl.nafnet_dw_case(hip, dev, 3), wl.nafnet_dw_case(hip, dev, 0),
                                        wl.evssm_scan_case(hip, dev), wl.metrics_case(dev)])
    if args.pmc_pass:  # the last dispatches: two markers, the copy, then a marker before each op and one after
        cases = wl.all_cases(hip, hip32, dev)
        os.makedirs(os.path.dirname(os.path.abspath(args.pmc_cases)), exist_ok=True)
        with open(args.pmc_cases, "w") as fh:
            json.dump([(c.name, c.config, c.flops, c.nbytes) for c in cases], fh)
        for c in cases:
            c.run()
        src = torch.randn(COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        keep = []
        torch.cuda.synchronize()
        torch.cuda._sleep(1000)
        torch.cuda._sleep(1000)
        torch.mul(src, 1.0, out=dst)
        for c in cases:
            torch.cuda._sleep(1000)
            keep.append(c.run())
        torch.cuda._sleep(1000)
        torch.cuda.synchronize()
        log(f"[bench] pmc pass: copy of {COPY_BYTES} B, then {len(cases)} ops")
        return

    # ------------------------------------------------------------ the timed config-2 step
    # captured once as a HIP graph on a side stream after an eager warm-up; `value` is its
    # algorithmic TFLOP/s over K replays (no host launch overhead inside the timed region)
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
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    value = flops_step / (ms_step / 1e3) / 1e12
    # per-op times of the step's ops: `reps` eager steps queued behind a bounded GPU spin, so the
    # kernels run back to back with no host launch gaps inside the events
    reps = args.reps
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in step]
          for _ in range(reps)]
    torch.cuda._sleep(int(2.4e8))  # ~0.1 s of spinning
    for s_ in range(reps):
        for i, c in enumerate(step):
            ev[s_][i][0].record(stream)
            c.run()
            ev[s_][i][1].record(stream)
    torch.cuda.synchronize()
    per_step_op = [statistics.median(ev[s_][i][0].elapsed_time(ev[s_][i][1]) * 1e3 for s_ in range(reps))
                   for i in range(len(step))]
    log(f"[bench] step {ms_step:.3f} ms -> {value:.1f} TFLOP/s (graph replays; eager ops sum {sum(per_step_op):.1f} us)")

    pmc = {}
    pfile = os.path.join(ROOT, "profiles", "pmc_ops.json")
    if os.path.exists(pfile):
        with open(pfile) as fh:
            pmc = json.load(fh).get("ops", {})

    def op_row(c, us, timing):
        tb, bound = c.t_bound()
        row = {"op": c.name, "config": c.config, "dtype": c.dtype, "gflop": round(c.flops / 1e9, 3),
               "mb": round(c.nbytes / 1e6, 2), "us": round(us, 2), "tflops": round(c.flops / us / 1e6, 2),
               "gbs": round(c.nbytes / us / 1e3, 1), "bound": bound, "t_bound_us": round(tb * 1e6, 2),
               "frac": round(tb * 1e6 / us, 3),
               "frac_hbm": round(c.nbytes / wl.PEAK_HBM * 1e6 / us, 3),
               "frac_mfma": round(c.flops / wl.PEAK_FLOPS[c.mfma or c.dtype] * 1e6 / us, 3),
               "frac_mfma_fp32": round(c.flops / wl.PEAK_FLOPS["fp32"] * 1e6 / us, 3) if c.dtype == "fp32" else None,
               "timing": timing, "reps": reps, "kernel": wl.kernel_of(c)}
        p = pmc.get(c.name)
        if p:
            row["traffic_ratio"] = p.get("traffic_ratio")
            row["mfma_util"] = p.get("mfma_util")
            row["mfma_flops_ratio"] = p.get("mfma_flops_ratio")
        return row
    rows = [op_row(c, us, "eager behind a spin, median") for c, us in zip(step, per_step_op)]

    # dominant kernel of the step
    di = max(range(len(step)), key=lambda i: per_step_op[i])
    dc, dus = step[di], per_step_op[di]
    tb, bound = dc.t_bound()
    if bound == "hbm":
        ach, peak, unit = dc.nbytes / dus / 1e3, wl.PEAK_HBM / 1e9, "GB/s"
    else:
        ach, peak, unit = dc.flops / dus / 1e6, wl.PEAK_FLOPS[dc.mfma or dc.dtype] / 1e12, "TFLOP/s"
    roofline = {"bound": bound, "achieved": round(ach, 1), "peak": peak, "unit": unit, "frac": round(ach / peak, 3),
                "traffic": pmc.get(dc.name, {}).get("traffic_bytes"), "op": dc.name, "avg_us": round(dus, 2),
                "kernel": rows[di]["kernel"], "algorithmic_bytes": int(dc.nbytes), "algorithmic_flops": int(dc.flops)}

    # ------------------------------------------------------------ other configs, cold per op
    if others:
        flush = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)  # > MALL (256 MB)
        sink = torch.empty((), dtype=torch.float32, device=dev)
        for c in others:
            for _ in range(3):
                c.run()
            ts = []
            for _ in range(reps):
                torch.sum(flush, dim=0, out=sink)  # reads 512 MB, writes 4 bytes
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                c.run()
                b.record(stream)
                ts.append((a, b))
            torch.cuda.synchronize()
            us = statistics.median(a.elapsed_time(b) * 1e3 for a, b in ts)
            rows.append(op_row(c, us, "cold (512 MB read before each rep), median"))
        del flush, sink
    for r in rows:
        log(f"[op] cfg{r['config']} {r['op']:<46} {r['dtype']:>4} {r['us']:9.2f} us {r['tflops']:8.1f} TF/s "
            f"{r['gbs']:8.0f} GB/s  {r['bound']:>4} {r['t_bound_us']:8.2f} us  frac {r['frac']:.3f}  {r['kernel']}")

    # ------------------------------------------------------------ NAFNet e2e
    e2e = None
    if not args.no_e2e:
        from clarus_amd import nafnet
        e2e = {"fused_pairs": nafnet.bench_forward(dev, reps=args.e2e_reps, fused_pairs=True, log=log),
               "reference_block": nafnet.bench_forward(dev, reps=args.e2e_reps, fused_pairs=False, log=log)}

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu legs (oracle on the host cores) ...")
        legs = cpu_legs(step, others, 0 if args.no_e2e else args.cpu_e2e_reps, log=log)
        cpu = legs["baseline"]
        for r in rows:
            got = legs["per_op_ms"].get(r["op"])
            if got is not None:
                ms, sample = got
                r["cpu_ms"] = round(ms, 2)
                r["cpu_over_gpu"] = round(ms * 1e3 / r["us"], 1)
                if sample:
                    r["cpu_sample"] = sample
        if e2e is not None and legs["e2e"] is not None:
            e2e["cpu"] = legs["e2e"]
        log(f"[bench] cpu baseline {cpu['value']} TFLOP/s on {cpu['cores']} threads ({cpu['ms_per_step']} ms/step)")

    head = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) activations, random-init weights)",
        "config": {"workload": "BASELINE config 2: NAFNet-w64 720p pointwise GEMMs (expand+gate and c->c+scale+res "
                               "at c=64..1024), bf16 operands, fp32 accumulate", "global_batch": 1,
                   "parallelism": "none (1 GPU)"},
        "roofline": roofline, "cpu_baseline": cpu,
    }
    detail = os.path.join(ROOT, "gpurun_out", "bench_per_op.json")
    try:
        os.makedirs(os.path.dirname(detail), exist_ok=True)
        with open(detail, "w") as fh:
            json.dump(_finite({**head, "per_op": rows, "nafnet_e2e": e2e}), fh, indent=1)
    except OSError as e:
        log(f"[bench] could not write {detail}: {e}")
        detail = None
    print(final_line(head, rows, e2e, detail), flush=True)


LINE_LIMIT = 7000  # the driver keeps the last 8000 characters of stdout; the line must fit whole
PER_OP_COLS = ["op", "us", "tflops", "bound", "frac", "traffic_ratio", "cpu_ms"]


def _finite(obj):
    """obj with every non-finite float replaced by None (strict JSON has no NaN / Infinity)."""
    if isinstance(obj, float):
        return obj if obj == obj and abs(obj) != float("inf") else None
    if isinstance(obj, dict):
        return {k: _finite(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return [_finite(v) for v in obj]
    return obj


def final_line(head: dict, rows: list, e2e: dict | None, detail: str | None) -> str:
    """The one JSON line bench.py prints: the required keys, roofline and cpu_baseline, the per-op
    rows as short tuples (PER_OP_COLS) and the NAFNet e2e figures, kept under LINE_LIMIT
    characters (op names are shortened first, then the per-op rows dropped, if it does not fit).
    The full rows go to `detail`."""
    line = dict(head)
    if e2e is not None:
        ref, fused, cpu = e2e.get("reference_block"), e2e.get("fused_pairs"), e2e.get("cpu")
        line["nafnet_e2e"] = {
            "ms": ref and ref["ms"], "eager_ms": ref and ref["eager_ms"],
            "block": "reference block (five linear calls), graph replay median",
            "fused_ops_ms": fused and fused["ms"], "cpu_ms": cpu and cpu["ms"],
            "cpu_threads": cpu and cpu["threads"],
            "all_hip": all(v == ["hip"] for p in (ref, fused) if p for k, v in p["served"].items()
                           if k not in ("pixel_shuffle", "pixel_unshuffle", "add_scaled")),
        }
    line["per_op_cols"] = PER_OP_COLS
    line["per_op_file"] = detail and os.path.relpath(detail, ROOT)
    for width in (60, 32, 0):
        line["per_op"] = [[r["op"][:width] if c == "op" else r.get(c) for c in PER_OP_COLS] for r in rows] \
            if width else None
        text = json.dumps(_finite(line), allow_nan=False, separators=(",", ":"))
        if len(text) <= LINE_LIMIT:
            return text
    raise RuntimeError(f"bench line of {len(text)} characters even without per-op rows")


if __name__ == "__main__":
    main()
