#!/usr/bin/env python3
"""
Benchmark of the tensor hot path on one MI355X.

Headline workload (`value`) = BASELINE.json configs[1] (cfg2), one step is
  bias-add      Y[8192,4096] = X + b[4096]                 (nn_layers.asm:472-539)
  row sum, mean, max, argmax over the last dim of Y        (math_kernels.asm:956-1264, main.asm:3245-3292)
  softmax and log-softmax rows of S[65536,1024]            (activations.asm:761-987, metrics_losses.c:47-64)
on synthetic fp32 inputs N(0,3) already resident in HBM.  The metric is the
achieved HBM bandwidth: algorithmic bytes (each input read once, each output
written once) divided by the step time (HIP events around K steps).

Every other BASELINE config is measured in the same run and reported in the
same JSON line under "configs" (cfg1 at the 64M-element headline size and at
its own 1M size, cfg3 in f32 and f64, cfg4, cfg5): per op the kernel time and
its % of 8 TB/s, per config the aggregate GB/s, a roofline object for its
dominant kernel and a CPU baseline timed on this host in this run.

Kernel times come from HIP event pairs that the library attaches to launches
(neural_hip_time_launches -> hipExtLaunchKernelGGL): a pair on one launch
brackets that kernel's own execution on its stream; a pair spanning every
launch of a multi-launch call (the library's launch counter gives how many)
brackets the whole op, gaps included.  Each figure is the median of 20 such
pairs.  Ops whose result returns to the host (neural_sum, neural_argmax, the
NaN/Inf/L2 scan) are also timed per call on the host clock (launch, kernels,
host wait, return).  A float4 streaming copy measured in the same run gives
the achievable 1:1 stream rate; every op also carries its % of it.  Outside
the step, an op whose footprint is below 1 GiB cycles over NROT copies of its
inputs and outputs from one timed call to the next, so that the 256 MB
memory-side cache cannot serve re-reads or absorb rewrites; the step keeps the
reference's one set of buffers, and the same step with its outputs rotating,
and with its inputs and outputs rotating, is reported beside it.

CPU baselines, one thread (the reference never dispatches to its thread pool):
  cfg2  the oracle's C restatement of the whole step (port);
  cfg1  the reference's AVX-256 ew_add / ew_mul / reduce_sum loops, node_relu's
        three passes and the scalar maxss max chain, restated in
        oracle/cpu_baseline.c (port); simd.asm's AVX-512 path separately;
  cfg3  the reference's own activations_c.c (compiled unchanged into
        oracle/_ref) on a sample;
  cfg4  the reference's quantize.c (oracle/_ref) on a sample widened to double;
  cfg5  the reference's optimizers_c.c AdamW (oracle/_ref) and the
        training_ops.asm scans (has_nan, has_inf: scalar; L2: SSE 4-lane) on a
        sample.
CPU GB/s use the same algorithmic bytes per element as the GPU op; each CPU
figure is the median of 5 runs after one warm-up run.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--detail FILE] [--suite]
"""

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "neural-assembly_amd"))

HBM_PEAK_GBS = 8000.0
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h
FP64_PEAK_TFLOPS = 78.6

ROWS, COLS = 8192, 4096
SROWS, SCOLS = 65536, 1024
N1 = 1 << 26                   # cfg1 headline size (64M)
N1_SMALL = 1 << 20             # cfg1 as specified (MALL-resident)
ACT_SHAPE = (64, 64, 128, 128)
ACTS = ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh"]
ACT_ALPHA = {"leaky_relu": 0.01, "elu": 1.0}
NQ = 268_435_456               # cfg4
NA = 100_000_000               # cfg5
REPS = 20                      # event-paired launches per op (median reported)
CPU_REPS = 5                   # timed CPU runs per leg after one warm-up (median reported)
VALU_CYCLES = 4                # cycles a wave64 VALU instruction occupies a 16-lane SIMD
CLOCK_GHZ = 2.4                # MI355X peak engine clock
N_SIMD = 256 * 4
# Untimed back-to-back calls of each op before its timed launches.  When the
# load switches (light f32 streams to FP64-heavy activations, say) the GPU's
# clocks take some milliseconds to settle: on one box f64 tanh ran 193-216 us
# per launch in the first ~10 ms of FP64 work and 171-175 us after it.
WARM_MS = 20.0
# Buffer sets an op cycles through from one timed call to the next.  The GPU's
# 256 MB memory-side cache (MALL) serves part of a re-read and absorbs
# rewrites of data touched by the previous call: a row sum of one 268 MB
# [16384,4096] input read it 9% faster than over four rotating inputs, and a
# bias add rewriting one output took 77 us against 88 us over four outputs.
# Every timed op whose footprint is below 1 GiB therefore rotates over NROT
# copies of its inputs and outputs, so that at least (NROT - 1) x its
# footprint of other traffic (>= 800 MB here) separates two uses of a buffer.
NROT = 4


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline legs")
    ap.add_argument("--no-configs", action="store_true", help="only the cfg2 step")
    ap.add_argument("--configs", default="cfg1,cfg3,cfg4,cfg5", help="comma-separated configs to run besides cfg2")
    ap.add_argument("--detail", default=None, help="write every per-op figure (JSON) to this file")
    ap.add_argument("--suite", action="store_true", help="also time the other kernel families (detail file)")
    return ap.parse_args()


def traffic_from_profile():
    """HBM bytes per launch ("<config>.<op>" -> bytes) from the committed
    rocprofv3 --pmc summary profiles/bench_pmc_traffic.txt (FETCH_SIZE +
    WRITE_SIZE, scaled by a 256 MiB copy measured in the same runs)."""
    p = ROOT / "profiles" / "bench_pmc_traffic.json"
    if not p.exists():
        return {}
    try:
        return {k: float(v) for k, v in json.loads(p.read_text())["traffic_bytes_per_launch"].items()}
    except Exception:
        return {}


TRAFFIC = traffic_from_profile()


def valu_from_profile():
    """Per-launch VALU instruction counts of the cfg3 f64 activations
    ("<op>" -> {"valu": wave instructions, "fp64_flops": FLOPs}) from the
    committed rocprofv3 --pmc summary profiles/cfg3_f64_valu_pmc.json."""
    p = ROOT / "profiles" / "cfg3_f64_valu_pmc.json"
    if not p.exists():
        return {}
    try:
        return json.loads(p.read_text())["per_launch"]
    except Exception:
        return {}


VALU = valu_from_profile()


class TimingEvent:
    """A HIP event used only for timing (hipEventDisableSystemFence), made
    through the HIP runtime that torch loaded."""

    _hip = None

    @classmethod
    def _lib(cls):
        if cls._hip is None:
            import torch
            p = Path(torch.__file__).parent / "lib" / "libamdhip64.so"
            hip = ctypes.CDLL(str(p) if p.exists() else "libamdhip64.so")
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            cls._hip = hip
        return cls._hip

    def __init__(self):
        self.ev = ctypes.c_void_p()
        rc = self._lib().hipEventCreateWithFlags(ctypes.byref(self.ev), HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed: {rc}")

    def record(self, stream):
        rc = self._lib().hipEventRecord(self.ev, ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed: {rc}")

    def elapsed_time(self, end) -> float:
        """Milliseconds from this event to `end` (both completed)."""
        ms = ctypes.c_float()
        rc = self._lib().hipEventElapsedTime(ctypes.byref(ms), self.ev, end.ev)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {rc}")
        return ms.value

    def __del__(self):
        if self._hip is not None and self.ev:
            self._hip.hipEventDestroy(self.ev)


class Clock:
    """Kernel, op and call timing on the library's launch stream."""

    def __init__(self, torch, lib, stream):
        self.torch, self.lib, self.stream = torch, lib, stream
        self.pairs = [(TimingEvent(), TimingEvent()) for _ in range(REPS)]

    def arm(self, pair, skip=0, count=1):
        rc = self.lib.neural_hip_time_launches(pair[0].ev, pair[1].ev, skip, count)
        if rc != 0:
            raise RuntimeError(f"neural_hip_time_launches failed: {rc}")

    def warm(self, fn, warm=3):
        """At least `warm` calls and WARM_MS of back-to-back calls."""
        t0, k = time.perf_counter(), 0
        while k < warm or (time.perf_counter() - t0) * 1e3 < WARM_MS:
            fn()
            k += 1
            if k % 8 == 0:
                self.torch.cuda.synchronize()
        self.torch.cuda.synchronize()

    def launches(self, fn):
        """Kernel launches one call of fn makes (after a first call, which
        may allocate and clear state)."""
        fn()
        c0 = self.lib.neural_hip_launch_count()
        fn()
        n = self.lib.neural_hip_launch_count() - c0
        self.torch.cuda.synchronize()
        return int(n)

    def kernel_us(self, fn, reps=REPS, skip=0, count=1, warm=3):
        """Median duration (us) over `reps` calls of fn, each with its own
        event pair on the launches skip .. skip + count - 1 of the call."""
        self.warm(fn, warm)
        for r in range(reps):
            self.arm(self.pairs[r], skip, count)
            fn()
        self.torch.cuda.synchronize()
        return 1e3 * statistics.median(a.elapsed_time(b) for a, b in self.pairs[:reps])

    def op(self, fn, reps=REPS):
        """(main kernel us, whole-op us, launches per call): the first launch,
        and the span over every launch of the call."""
        n = self.launches(fn)
        k = self.kernel_us(fn, reps)
        return k, (self.kernel_us(fn, reps, 0, n, warm=0) if n > 1 else k), n

    def host_call_us(self, fn, reps=REPS):
        """Median host-clock time (us) of one call of fn that returns its
        result to the host (the call waits for it)."""
        self.warm(fn)
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return 1e6 * statistics.median(ts)


def gbs(nbytes, us):
    return nbytes / us / 1e3


def pct(nbytes, us):
    return round(100.0 * gbs(nbytes, us) / HBM_PEAK_GBS, 1)


COPY = {}  # the same-run float4 copy: {"GBps": ..} (filled by measure_copy_peak)


class Rot:
    """A call that runs the next of several equivalent calls each time (the
    same op over NROT buffer sets, in turn)."""

    def __init__(self, fns):
        self.fns, self.k = list(fns), 0

    def __call__(self):
        f = self.fns[self.k]
        self.k = (self.k + 1) % len(self.fns)
        return f()


def copies(t, n=NROT):
    """t and n - 1 device copies of it."""
    return [t] + [t.clone() for _ in range(n - 1)]


def pct_copy(gbps):
    return round(100.0 * gbps / COPY["GBps"], 1) if COPY.get("GBps") else None


class Config:
    """Per-op GPU figures of one BASELINE config and its compact summary."""

    def __init__(self, name, workload):
        self.name, self.workload = name, workload
        self.ops = {}          # op -> dict(kernel, bytes, elems, kernel_us, op_us, launches, host_call_us, ...)

    def add(self, op, kernel, nbytes, elems, kernel_us, op_us=None, launches=1, host_call_us=None):
        """kernel_us: the op's main (first) launch; op_us: every launch of the
        call (default: kernel_us); host_call_us: the whole call on the host
        clock, for ops that return a result to the host."""
        op_us = kernel_us if op_us is None else op_us
        e = {"kernel": kernel, "bytes": nbytes, "elems": elems, "launches": launches,
             "kernel_us": round(kernel_us, 2), "op_us": round(op_us, 2),
             "GB/s": round(gbs(nbytes, op_us), 1), "pct_hbm": pct(nbytes, op_us),
             "pct_copy": pct_copy(gbs(nbytes, op_us)), "Gelem/s": round(elems / op_us / 1e3, 2)}
        if host_call_us is not None:
            e["host_call_us"] = round(host_call_us, 2)
            e["host_call_pct_hbm"] = pct(nbytes, host_call_us)
        self.ops[op] = e

    def aggregate_gbs(self):
        return sum(o["bytes"] for o in self.ops.values()) / sum(o["op_us"] for o in self.ops.values()) / 1e3

    def summary(self, cpu=None):
        """Compact form for the JSON line: ops as [op us, % of 8 TB/s] (op =
        every launch of the call); the main kernel alone where an op makes
        several launches; host-clock call times where a result returns to the
        host; the roofline of the dominant (longest) op, HBM-bound against
        8 TB/s: achieved = algorithmic bytes / median op us."""
        dom = max(self.ops, key=lambda k: self.ops[k]["op_us"])
        d = self.ops[dom]
        s = {
            "w": self.workload,
            "ops": {k: [o["op_us"], o["pct_hbm"]] for k, o in self.ops.items()},
            "GBps": round(self.aggregate_gbs(), 1),
            "pct_of_copy": round(100.0 * self.aggregate_gbs() / COPY["GBps"], 1) if COPY.get("GBps") else None,
            "roofline": {"kernel": dom, "us": d["op_us"], "bytes": d["bytes"], "achieved": d["GB/s"],
                         "frac": round(d["GB/s"] / HBM_PEAK_GBS, 4), "traffic": TRAFFIC.get(f"{self.name}.{dom}")},
        }
        multi = {k: {"launches": o["launches"], "first_kernel_us": o["kernel_us"]}
                 for k, o in self.ops.items() if o["launches"] > 1}
        if multi:
            s["multi_launch"] = multi
        host = {k: [o["host_call_us"], o["host_call_pct_hbm"]] for k, o in self.ops.items() if "host_call_us" in o}
        if host:
            s["host_call"] = host
        if cpu:
            c = {"GBps": cpu["value"], "kind": cpu["kind"], "cores": cpu["cores"]}
            if "avx512" in cpu:
                c["avx512_GBps"] = cpu["avx512"]["value"]
            c["speedup"] = round(s["GBps"] / cpu["value"], 1) if cpu.get("value") else None
            s["cpu"] = c
        return s

    def detail(self):
        return {"workload": self.workload, "ops": self.ops}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def _median_time(fn, reps=CPU_REPS, warm=1):
    """Median wall time (s) of `reps` runs of fn after `warm` untimed runs."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path would shard by rows / element ranges with one scalar all-reduce per global "
              "reduction", file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    import pyneural as pn
    from pyneural.core import _lib, _check_error

    pn.init()
    # A dedicated (non-null) torch stream: the library launches on it and the
    # HIP events are recorded on it.
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    pn.set_stream(stream.cuda_stream)
    dev = torch.device("cuda:0")
    clock = Clock(torch, _lib, stream)
    detail = {}
    measure_copy_peak(torch, _lib, clock, dev)

    # ---------------------------------------------------------------- cfg2 step
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    X = torch.randn(ROWS, COLS, device=dev, generator=g) * 3.0
    b = torch.randn(COLS, device=dev, generator=g) * 3.0
    g.manual_seed(3)
    S = torch.randn(SROWS, SCOLS, device=dev, generator=g) * 3.0
    Y = torch.empty_like(X)
    rsum = torch.empty(ROWS, device=dev)
    rmean = torch.empty(ROWS, device=dev)
    rmax = torch.empty(ROWS, device=dev)
    ridx = torch.empty(ROWS, dtype=torch.int64, device=dev)
    P = torch.empty_like(S)
    L = torch.empty_like(S)
    torch.cuda.synchronize()
    T = {k: pn.Tensor.from_torch(v) for k, v in
         dict(X=X, b=b, S=S, Y=Y, rsum=rsum, rmean=rmean, rmax=rmax, P=P, L=L).items()}

    n1, n2 = ROWS * COLS, SROWS * SCOLS
    step_ops = [
        ("bias_add", "k_rowbcast", 2 * n1 * 4 + COLS * 4, n1,
         lambda: _lib.neural_bias_add(T["Y"]._ptr, T["X"]._ptr, T["b"]._ptr)),
        ("row_sum", "k_reduce_rows", n1 * 4 + ROWS * 4, n1, lambda: _lib.neural_reduce_sum(T["Y"]._ptr, 1, T["rsum"]._ptr)),
        ("row_mean", "k_reduce_rows", n1 * 4 + ROWS * 4, n1,
         lambda: _lib.neural_reduce_mean(T["Y"]._ptr, 1, T["rmean"]._ptr)),
        ("row_max", "k_reduce_rows", n1 * 4 + ROWS * 4, n1, lambda: _lib.neural_reduce_max(T["Y"]._ptr, 1, T["rmax"]._ptr)),
        ("row_argmax", "k_reduce_rows", n1 * 4 + ROWS * 8, n1,
         lambda: _lib.neural_reduce_argmax(T["Y"]._ptr, 1, ctypes.c_void_p(ridx.data_ptr()))),
        ("softmax", "k_softmax_wave_f32<false>", 2 * n2 * 4, n2, lambda: _lib.neural_softmax(T["P"]._ptr, T["S"]._ptr)),
        ("log_softmax", "k_softmax_wave_f32<true>", 2 * n2 * 4, n2,
         lambda: _lib.neural_log_softmax(T["L"]._ptr, T["S"]._ptr)),
    ]
    step_bytes = sum(o[2] for o in step_ops)

    def step(instrument=None):
        for k, (name, _, _, _, fn) in enumerate(step_ops):
            if instrument is not None:
                clock.arm(instrument[k])
            rc = fn()
            if rc != 0:
                _check_error(rc, name)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # The same steps again with an event pair on every kernel: each kernel's
    # own duration inside the step sequence (cache state as in the step);
    # the mean over the steps (the roofline's average launch) and the median.
    inst = [[(TimingEvent(), TimingEvent()) for _ in step_ops] for _ in range(args.steps)]
    for s in range(args.steps):
        step(inst[s])
    torch.cuda.synchronize()
    cfg2 = Config("cfg2", "cfg2 step kernels, each timed inside the step sequence")
    mean_us = {}
    for k, (name, kern, nbytes, elems, _) in enumerate(step_ops):
        ts = [1e3 * inst[s][k][0].elapsed_time(inst[s][k][1]) for s in range(args.steps)]
        mean_us[name] = statistics.mean(ts)
        cfg2.add(name, kern, nbytes, elems, statistics.median(ts))
    kernel_sum_us = sum(mean_us.values())
    detail["cfg2_step"] = cfg2.detail()
    detail["cfg2_step"]["mean_us"] = {k: round(v, 2) for k, v in mean_us.items()}
    dom = max(mean_us, key=lambda k: mean_us[k])
    d = cfg2.ops[dom]
    frac_by_kernel = {k: round(cfg2.ops[k]["bytes"] / (v * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) for k, v in mean_us.items()}

    fused = fused_step(torch, _lib, clock, stream, T, ridx, step_ops, args, ms_per_step, n1)
    yres = y_residency(torch, pn, _lib, clock, Y, step_ops)
    rot_us = rotating_step(torch, pn, _lib, stream, T, ridx, args, X, S)

    cpu2 = None
    if not args.no_cpu:
        cpu2 = cpu_baseline_cfg2(X, b, S, step_bytes)

    line = {
        "metric": "achieved HBM GB/s (% of peak) at 64M fp32 elems; speedup vs host AVX path",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded torch generators, inputs resident in HBM (cfg2 N(0,3); others per BASELINE.json)",
        "config": {
            "workload": "cfg2: bias-add [8192,4096]+[4096]; row sum/mean/max/argmax; softmax + log-softmax rows [65536,1024]",
            "step_bytes": step_bytes,
            "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 1),
            "elements_per_s": round((5 * n1 + 2 * n2) / (ms_per_step * 1e-3), 0),
            "kernel_us_in_step": {k: round(v, 2) for k, v in mean_us.items()},
            "kernel_median_us_in_step": {k: o["kernel_us"] for k, o in cfg2.ops.items()},
            "kernel_sum_us": round(kernel_sum_us, 1),
            "fused_step": fused,
            "y_residency": yres,
            "step_outputs_rotating": {"us_per_step": round(rot_us[0], 1),
                                      "GBps": round(gbs(step_bytes, rot_us[0]), 1),
                                      "note": f"the same step with Y, P and L rotating over {NROT} buffers each"},
            "step_all_rotating": {"us_per_step": round(rot_us[1], 1),
                                  "GBps": round(gbs(step_bytes, rot_us[1]), 1),
                                  "note": f"the same step with X, S, Y, P and L rotating over {NROT} buffers each"},
            "copy_peak": COPY,
        },
        "roofline": {
            "kernel": f"{dom}: {d['kernel']} [65536,1024] f32" if "softmax" in dom else f"{dom}: {d['kernel']}",
            "bound": "hbm",
            "achieved": round(gbs(d["bytes"], mean_us[dom]), 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": frac_by_kernel[dom],
            "traffic": TRAFFIC.get(f"cfg2.{dom}"),
            "avg_launch_us": round(mean_us[dom], 2),
            "median_launch_us": d["kernel_us"],
            "algorithmic_bytes": d["bytes"],
            "frac_by_kernel": frac_by_kernel,
            "min_frac_in_step": min(frac_by_kernel.values()),
            "pct_of_copy": pct_copy(gbs(d["bytes"], mean_us[dom])),
        },
        "cpu_baseline": cpu2,
    }
    if cpu2:
        line["config"]["speedup_vs_cpu"] = round(value / cpu2["value"], 1)
    del T, X, Y, S, P, L
    torch.cuda.empty_cache()

    if not args.no_configs:
        line["configs"] = run_configs(torch, pn, _lib, clock, dev, args, detail)

    if args.suite:
        detail["suite"] = suite(torch, pn, clock, dev, cpu=not args.no_cpu)
    pn.set_stream(None)
    if args.detail:
        detail["host"] = {"cpu": _cpu_model(), "nproc": os.cpu_count()}
        detail["line"] = line
        Path(args.detail).parent.mkdir(parents=True, exist_ok=True)
        Path(args.detail).write_text(json.dumps(detail, indent=1))
    print(json.dumps(line, separators=(",", ":")), flush=True)


def measure_copy_peak(torch, lib, clock, dev):
    """The library's float4 streaming copy (neural_hip_stream_copy: the flat
    kernels' tiling, 16-byte non-temporal loads and stores) of 256 MiB (cfg1's
    64M f32, cfg2's softmax input) and of 1 GiB into a second buffer: the
    achievable rate of a 1:1 read/write stream in this run (the 256 MiB copy
    over NROT source / destination pairs, like the ops it is compared with).
    The faster of the two is the reference every op's pct_of_copy refers to."""
    res = {}
    for n, nrot in ((1 << 26, NROT), (1 << 28, 1)):
        srcs = copies(torch.empty(n, device=dev).uniform_(), nrot)
        dsts = [torch.empty_like(srcs[0]) for _ in range(nrot)]
        torch.cuda.synchronize()
        f = Rot([lambda d=d, s_=s_: lib.neural_hip_stream_copy(ctypes.c_void_p(d.data_ptr()),
                                                               ctypes.c_void_p(s_.data_ptr()), 4 * n)
                 for d, s_ in zip(dsts, srcs)])
        for _ in range(nrot):
            if f() != 0:
                raise RuntimeError("neural_hip_stream_copy failed")
        us = clock.kernel_us(f)
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(srcs, dsts)):
            raise RuntimeError("stream copy: destination differs from source")
        res[f"{4 * n >> 20}MiB"] = {"us": round(us, 2), "GBps": round(gbs(8 * n, us), 1), "pct_hbm": pct(8 * n, us)}
        del srcs, dsts, f
        torch.cuda.empty_cache()
    best = max(res.values(), key=lambda r: r["GBps"])
    COPY.update({"kernel": "k_map1_flat<float, FnCopy>, median of %d launches" % REPS, "sizes": res,
                 "GBps": best["GBps"], "pct_hbm": best["pct_hbm"]})


def y_residency(torch, pn, lib, clock, Y, step_ops, reps=REPS):
    """Where the step's row reductions read Y from.  A row sum of Y [8192,4096]
    timed: right after the bias add that wrote it (as in the step); after the
    bias add and then a 1 GiB read of another buffer (four times the 256 MB
    memory-side cache: Y cannot stay resident, and the read leaves no dirty
    lines behind); after the bias add and 1 GiB of writes (the timed read
    then also competes with their write-back); right after another row sum of
    Y.  Control: a row sum of a 64 MiB slice of Y right after a row sum of the
    same slice (the slice fits the cache), whose rate shows what a
    cache-served read looks like."""
    dev = torch.device("cuda:0")
    W = pn.Tensor.from_torch
    scrub = torch.empty(1 << 16, 1 << 12, device=dev)
    scrub_out = torch.empty(1 << 16, device=dev)
    ys, ys_out = Y[:4096], torch.empty(4096, device=dev)
    ts, tso, tys, tyso = W(scrub), W(scrub_out), W(ys), W(ys_out)
    bias = step_ops[0][4]
    rsum = step_ops[1][4]
    res = {}

    def read_scrub():
        lib.neural_reduce_sum(ts._ptr, 1, tso._ptr)

    def slice_sum():
        lib.neural_reduce_sum(tys._ptr, 1, tyso._ptr)

    phases = (("after_bias_add", lambda r: bias(), rsum),
              ("after_bias_add_then_1GiB_read", lambda r: (bias(), read_scrub()), rsum),
              ("after_bias_add_then_1GiB_write", lambda r: (bias(), scrub.fill_(float(r))), rsum),
              ("after_row_sum", lambda r: (bias(), rsum()), rsum),
              ("control_64MiB_slice_after_its_row_sum", lambda r: slice_sum(), slice_sum))
    for name, pre, timed in phases:
        for r in range(reps):
            pre(r)
            clock.arm(clock.pairs[r])
            timed()
        torch.cuda.synchronize()
        res[name] = round(1e3 * statistics.median(a.elapsed_time(b) for a, b in clock.pairs[:reps]), 2)
    ybytes = ROWS * COLS * 4
    res["GBps"] = {k: round(gbs(ybytes if not k.startswith("control") else ybytes // 2, v), 1)
                   for k, v in res.items()}
    res["kernel"] = "k_reduce_rows (row sum of Y [8192,4096] f32, %d MB), median of %d" % (ybytes // 10 ** 6, reps)
    del ts, tso, tys, tyso, scrub, scrub_out, ys_out
    torch.cuda.empty_cache()
    return res


def rotating_step(torch, pn, lib, stream, T, ridx, args, X, S):
    """Microseconds per cfg2 step (a) with its outputs Y, P and L rotating
    over NROT buffers each and (b) with its inputs X and S rotating as well
    (copies of the same values), against the timed steps' one set of buffers:
    whether the memory-side cache carries any buffer from one step to the next
    shows as a difference between them."""
    W = pn.Tensor.from_torch
    ys = [W(torch.empty(ROWS, COLS, device="cuda")) for _ in range(NROT)]
    ps = [W(torch.empty(SROWS, SCOLS, device="cuda")) for _ in range(NROT)]
    ls = [W(torch.empty(SROWS, SCOLS, device="cuda")) for _ in range(NROT)]
    xs = [W(X.clone()) for _ in range(NROT)]
    ss = [W(S.clone()) for _ in range(NROT)]
    torch.cuda.synchronize()

    def timed(inputs_rotate):
        def step(k):
            r = k % NROT
            y = ys[r]._ptr
            x, s_ = (xs[r], ss[r]) if inputs_rotate else (T["X"], T["S"])
            for rc in (lib.neural_bias_add(y, x._ptr, T["b"]._ptr), lib.neural_reduce_sum(y, 1, T["rsum"]._ptr),
                       lib.neural_reduce_mean(y, 1, T["rmean"]._ptr), lib.neural_reduce_max(y, 1, T["rmax"]._ptr),
                       lib.neural_reduce_argmax(y, 1, ctypes.c_void_p(ridx.data_ptr())),
                       lib.neural_softmax(ps[r]._ptr, s_._ptr), lib.neural_log_softmax(ls[r]._ptr, s_._ptr)):
                if rc != 0:
                    raise RuntimeError("rotating step: a call failed")

        for k in range(args.warmup):
            step(k)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for k in range(args.steps):
            step(k)
        t1.record(stream)
        torch.cuda.synchronize()
        return 1e3 * t0.elapsed_time(t1) / args.steps

    us = (timed(False), timed(True))
    del ys, ps, ls, xs, ss
    torch.cuda.empty_cache()
    return us


def fused_step(torch, lib, clock, stream, T, ridx, step_ops, args, ms_per_step, n1):
    """The same step with the library's NEW fused entry neural_bias_add_row_stats
    (no counterpart in the reference) in place of the bias add and the four
    row reductions: X read once, Y written once, no re-read of Y.  Reported
    beside the reference-shaped step, never as `value`; its outputs are checked
    bit for bit against the reference-shaped step's before it is timed."""
    keep = {k: T[k].numpy() for k in ("Y", "rsum", "rmean", "rmax")}
    keep_idx = ridx.clone()
    torch.cuda.synchronize()
    for k in ("Y", "rsum", "rmean", "rmax"):
        lib.neural_tensor_fill(T[k]._ptr, ctypes.c_double(float("nan")))
    ridx.fill_(-1)
    torch.cuda.synchronize()

    def fused_call():
        return lib.neural_bias_add_row_stats(T["Y"]._ptr, T["X"]._ptr, T["b"]._ptr, T["rsum"]._ptr,
                                             T["rmean"]._ptr, T["rmax"]._ptr, ctypes.c_void_p(ridx.data_ptr()))

    ops = [("bias_add_row_stats", fused_call)] + [(name, fn) for name, _, _, _, fn in step_ops[5:]]
    for name, fn in ops:
        if fn() != 0:
            raise RuntimeError(f"{name} failed")
    torch.cuda.synchronize()
    import numpy as np
    for k, want in keep.items():
        if not np.array_equal(T[k].numpy().view(np.uint32), want.view(np.uint32)):
            raise RuntimeError(f"fused step: {k} differs from the reference-shaped step")
    if not torch.equal(ridx, keep_idx):
        raise RuntimeError("fused step: argmax differs from the reference-shaped step")

    for _ in range(args.warmup):
        for _, fn in ops:
            fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        for _, fn in ops:
            fn()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    inst = [[(TimingEvent(), TimingEvent()) for _ in ops] for _ in range(args.steps)]
    for s in range(args.steps):
        for k, (_, fn) in enumerate(ops):
            clock.arm(inst[s][k])
            fn()
    torch.cuda.synchronize()
    kus = {name: round(1e3 * statistics.mean(inst[s][k][0].elapsed_time(inst[s][k][1]) for s in range(args.steps)), 2)
           for k, (name, _) in enumerate(ops)}
    rows = n1 // COLS
    fused_bytes = 2 * n1 * 4 + COLS * 4 + rows * (3 * 4 + 8)
    moved = fused_bytes + sum(o[2] for o in step_ops[5:])
    return {"entry": "neural_bias_add_row_stats (NEW, no reference counterpart) + softmax + log-softmax; "
                     "outputs bit-identical to the reference-shaped step (checked in this run)",
            "us_per_step": round(1e3 * ms, 1), "speedup_vs_step": round(ms_per_step / ms, 3),
            "hbm_bytes": moved, "pct_of_hbm_peak": round(100.0 * moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
            "kernel_us": kus,
            "fused_kernel_pct": round(100.0 * fused_bytes / (kus["bias_add_row_stats"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 1)}


# ------------------------------------------------------------------------------- configs

def run_configs(torch, pn, lib, clock, dev, args, detail):
    out = {}
    cpu_on = not args.no_cpu
    want = set(args.configs.split(","))
    g = torch.Generator(device=dev)
    if "cfg1" in want:
        _cfg1(torch, pn, lib, clock, dev, g, cpu_on, out, detail)
    if "cfg3" in want:
        _cfg3(torch, pn, lib, clock, dev, g, cpu_on, out, detail)
    if "cfg4" in want:
        _cfg4(torch, pn, lib, clock, dev, g, cpu_on, out, detail)
    if "cfg5" in want:
        _cfg5(torch, pn, lib, clock, dev, g, cpu_on, out, detail)
    return out


def _cfg1(torch, pn, lib, clock, dev, g, cpu_on, out, detail):
    """cfg1: a, b ~ U[-1,1] f32 (seed 0), 64M (the headline size) and 1M (as specified)."""
    W = pn.Tensor.from_torch
    g.manual_seed(0)
    a = torch.rand(N1, device=dev, generator=g) * 2 - 1
    bb = torch.rand(N1, device=dev, generator=g) * 2 - 1
    c = torch.empty_like(a)
    one = torch.empty(1, device=dev)
    one_i = torch.empty(1, dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    # the 64M arrays rotate over NROT copies (3.2 GB); the 1M case is the
    # cache-resident one and keeps one set
    a_s, b_s, c_s = copies(a), copies(bb), [c] + [torch.empty_like(c) for _ in range(NROT - 1)]
    torch.cuda.synchronize()
    for n, key in ((N1, "cfg1"), (N1_SMALL, "cfg1_1M")):
        nset = NROT if n == N1 else 1
        ta = [W(x[:n]) for x in a_s[:nset]]
        tb = [W(x[:n]) for x in b_s[:nset]]
        tc = [W(x[:n]) for x in c_s[:nset]]
        to = W(one)
        t1 = W(a[:1])
        cf = Config(key, f"cfg1: f32 add, mul, ReLU, full sum, max over {n:,} elements U[-1,1]"
                    + (" (256 MiB MALL holds it: cache-resident, reported not judged)" if n < N1
                       else f" ({NROT} rotating buffer sets)"))

        def rot(call):
            return Rot([lambda k=k: call(k) for k in range(nset)])

        ops = [("add", "k_map2_flat", 12 * n, rot(lambda k: lib.neural_add(tc[k]._ptr, ta[k]._ptr, tb[k]._ptr))),
               ("mul", "k_map2_flat", 12 * n, rot(lambda k: lib.neural_mul(tc[k]._ptr, ta[k]._ptr, tb[k]._ptr))),
               ("relu", "k_map1_flat", 8 * n, rot(lambda k: lib.neural_relu(tc[k]._ptr, ta[k]._ptr))),
               ("sum", "k_reduce_seg + k_reduce_combine", 4 * n,
                rot(lambda k: lib.neural_reduce_sum(ta[k]._ptr, -1, to._ptr))),
               ("max", "k_reduce_seg + k_reduce_combine", 4 * n,
                rot(lambda k: lib.neural_reduce_max(ta[k]._ptr, -1, to._ptr)))]
        for name, kern, nbytes, fn in ops:
            k, o, nl = clock.op(fn)
            cf.add(name, kern, nbytes, n, k, o, nl)
        if n == N1:
            # the reference's host-returning forms (neural_api.h:359,367): the
            # whole call on the host clock, result in host memory
            r = ctypes.c_double()
            idx = ctypes.c_int64()
            s_fn = rot(lambda k: lib.neural_sum(ta[k]._ptr, ctypes.byref(r)))
            a_fn = rot(lambda k: lib.neural_argmax(ta[k]._ptr, ctypes.byref(idx)))
            for name, fn in (("neural_sum", s_fn), ("neural_argmax", a_fn)):
                k, o, nl = clock.op(fn)
                cf.add(name, "k_reduce_seg + k_reduce_combine (result to the host)", 4 * n, n, k, o, nl,
                       host_call_us=clock.host_call_us(fn))
            # the floor of any host-returning call: one empty-work launch and
            # the host wait for its result (a 1-element sum)
            floor = clock.host_call_us(lambda: lib.neural_sum(t1._ptr, ctypes.byref(r)))
        cpu = cpu_cfg1(a[:n], bb[:n], n) if (cpu_on and n == N1) else None
        out[key] = cf.summary(cpu)
        if n < N1:
            out[key] = {"w": out[key]["w"], "ops_us": {k: o["op_us"] for k, o in cf.ops.items()}}
        detail[key] = cf.detail()
        if n == N1:
            out[key]["host_return_floor_us"] = round(floor, 2)
            if cpu:
                detail[key]["cpu"] = cpu
        del ta, tb, tc, to, t1
    del a, bb, c, one, one_i, a_s, b_s, c_s
    torch.cuda.empty_cache()


def _cfg3(torch, pn, lib, clock, dev, g, cpu_on, out, detail):
    """cfg3: the ten activations on [64,64,128,128], N(0,4) with 1% at +-30."""
    W = pn.Tensor.from_torch
    g.manual_seed(4)
    x4 = torch.randn(*ACT_SHAPE, device=dev, generator=g, dtype=torch.float64) * 4
    ne = x4.numel()
    sat = torch.randperm(ne, device=dev, generator=g)[: ne // 100]
    x4.view(-1)[sat] = 30.0 * (torch.randint(0, 2, (sat.numel(),), device=dev, generator=g).double() * 2 - 1)
    del sat
    for dt_name, tdt, bpe in (("f32", torch.float32, 8), ("f64", torch.float64, 16)):
        xx = x4.to(tdt).contiguous()
        xs = copies(xx)
        ys = [torch.empty_like(xx) for _ in range(NROT)]
        tx, ty = [W(t) for t in xs], [W(t) for t in ys]
        torch.cuda.synchronize()
        key = f"cfg3_{dt_name}"
        cf = Config(key, f"cfg3: ten activations on [64,64,128,128] {dt_name}, N(0,4) with 1% at +-30 "
                         f"({NROT} rotating buffer sets)")
        for nm in ACTS:
            fn_c = getattr(lib, "act_" + nm)
            if nm in ACT_ALPHA:
                f = Rot([lambda fn_c=fn_c, al=ACT_ALPHA[nm], k=k: fn_c(ty[k]._ptr, tx[k]._ptr, ctypes.c_double(al))
                         for k in range(NROT)])
            else:
                f = Rot([lambda fn_c=fn_c, k=k: fn_c(ty[k]._ptr, tx[k]._ptr) for k in range(NROT)])
            cf.add(nm, "k_map1_flat / k_map1_f32_tail" if dt_name == "f32" else "k_map1_flat", bpe * ne, ne,
                   clock.kernel_us(f))
        cpu = cpu_cfg3(xx, dt_name, bpe) if cpu_on else None
        out[key] = cf.summary(cpu)
        if dt_name == "f64":
            compute_bound(cf, out[key])
        detail[key] = cf.detail()
        if cpu:
            detail[key]["cpu"] = cpu
        del xx, xs, ys, tx, ty
    del x4
    torch.cuda.empty_cache()



def compute_bound(cf, summ):
    """FP64 and VALU-issue figures of the f64 activations beside their HBM
    figure, from the per-launch instruction counts of a rocprofv3 --pmc run
    (profiles/cfg3_f64_valu_pmc.json: SQ_INSTS_VALU, and FP64 FLOPs =
    64 (2 FMA + ADD + MUL) from SQ_INSTS_VALU_{FMA,ADD,MUL}_F64) and this
    run's launch times: FP64 TFLOP/s against 78.6 TFLOP/s, and the VALU issue
    fraction = wave instructions x 4 cycles / (1024 SIMDs x 2.4 GHz x launch
    time) (a wave64 VALU instruction, FP64 included, occupies a 16-lane SIMD
    for 4 cycles).  The roofline's `bound` is whichever fraction is larger."""
    per = {}
    for op, o in cf.ops.items():
        v = VALU.get(op)
        if not v:
            continue
        t = o["op_us"] * 1e-6
        per[op] = {"fp64_tflops": round(v["fp64_flops"] / t / 1e12, 2),
                   "fp64_frac": round(v["fp64_flops"] / t / 1e12 / FP64_PEAK_TFLOPS, 4),
                   "valu_issue_frac": round(v["valu"] * VALU_CYCLES / (N_SIMD * CLOCK_GHZ * 1e9 * t), 4),
                   "hbm_frac": round(o["pct_hbm"] / 100.0, 4)}
    if not per:
        return
    summ["compute"] = per
    rf = summ["roofline"]
    c = per.get(rf["kernel"])
    if c:
        rf["fp64_tflops"] = c["fp64_tflops"]
        rf["fp64_frac"] = c["fp64_frac"]
        rf["valu_issue_frac"] = c["valu_issue_frac"]
        rf["bound"] = "hbm" if rf["frac"] >= c["valu_issue_frac"] else "valu"
    summ["bound_by_op"] = {op: ("hbm" if c["hbm_frac"] >= c["valu_issue_frac"] else "valu") for op, c in per.items()}


def _cfg4(torch, pn, lib, clock, dev, g, cpu_on, out, detail):
    """cfg4: int8 quantization of 268M Laplace(0,1) f32, 0.1% outliers at +-50."""
    g.manual_seed(5)
    q_in = torch.empty(NQ, device=dev).exponential_(generator=g)
    q_in *= torch.randint(0, 2, (NQ,), device=dev, generator=g).float() * 2 - 1
    outl = torch.randperm(NQ, device=dev, generator=g)[: NQ // 1000]
    q_in[outl] = 50.0 * (torch.randint(0, 2, (outl.numel(),), device=dev, generator=g).float() * 2 - 1)
    q_in[outl[0]], q_in[outl[1]] = 50.0, -50.0
    del outl
    q8 = torch.empty(NQ, dtype=torch.int8, device=dev)
    dq = torch.empty(NQ, device=dev)
    dq64 = torch.empty(NQ, dtype=torch.float64, device=dev)
    psym = torch.zeros(5, dtype=torch.float64, device=dev)
    paff = torch.zeros(5, dtype=torch.float64, device=dev)
    torch.cuda.synchronize()
    cf = Config("cfg4", "cfg4: minmax calibration, symmetric and affine quantize, dequantize; 268,435,456 f32")
    cal = "k_reduce_seg + k_reduce_combine (params in device memory)"
    cf.add("calibrate_sym", cal, 4 * NQ, NQ,
           *clock.op(lambda: lib.calibrate_minmax_f32_dev(q_in.data_ptr(), NQ, 1, psym.data_ptr())))
    cf.add("calibrate_aff", cal, 4 * NQ, NQ,
           *clock.op(lambda: lib.calibrate_minmax_f32_dev(q_in.data_ptr(), NQ, 0, paff.data_ptr())))
    cf.add("quantize_sym", "k_quantize", 5 * NQ, NQ,
           *clock.op(lambda: lib.quantize_tensor_f32_dev(q_in.data_ptr(), q8.data_ptr(), NQ, psym.data_ptr())))
    cf.add("quantize_aff", "k_quantize", 5 * NQ, NQ,
           *clock.op(lambda: lib.quantize_tensor_f32_dev(q_in.data_ptr(), q8.data_ptr(), NQ, paff.data_ptr())))
    cf.add("dequantize_f32", "k_dequantize<float>", 5 * NQ, NQ,
           *clock.op(lambda: lib.dequantize_tensor_f32_dev(q8.data_ptr(), dq.data_ptr(), NQ, paff.data_ptr())))
    hp = pn.core.QuantParamsC()
    ctypes.memmove(ctypes.addressof(hp), paff.cpu().numpy().ctypes.data, 40)
    cf.add("dequantize_f64", "k_dequantize<double>", 9 * NQ, NQ,
           *clock.op(lambda: lib.dequantize_tensor(q8.data_ptr(), dq64.data_ptr(), NQ, ctypes.byref(hp))))
    cpu = cpu_cfg4(q_in) if cpu_on else None
    out["cfg4"] = cf.summary(cpu)
    detail["cfg4"] = cf.detail()
    if cpu:
        detail["cfg4"]["cpu"] = cpu
    del q8, dq, dq64, psym, paff
    torch.cuda.empty_cache()
    out["cfg4"]["host_e2e"] = host_e2e_cfg4(torch, pn, q_in)
    del q_in
    torch.cuda.empty_cache()



def _cfg5(torch, pn, lib, clock, dev, g, cpu_on, out, detail):
    """cfg5: NaN/Inf/L2 scan + AdamW over 100M f32 params (f64 moments)."""
    W = pn.Tensor.from_torch
    g.manual_seed(6)
    p = torch.randn(NA, device=dev, generator=g) * 0.02
    gr = torch.randn(NA, device=dev, generator=g) * 1e-3
    clean = gr.clone()
    inj = torch.randperm(NA, device=dev, generator=g)[:96]
    gr[inj[:32]] = float("nan")
    gr[inj[32:64]] = float("inf")
    gr[inj[64:]] = float("-inf")
    del inj
    tp, tg, tcl = W(p), W(gr), W(clean)
    # the scan (400 MB) rotates over three copies of the gradient; AdamW moves
    # 4.4 GB per call and keeps one set
    gs = copies(gr, 3)
    tgs = [tg] + [W(x) for x in gs[1:]]
    torch.cuda.synchronize()
    cf = Config("cfg5", "cfg5: fused NaN/Inf/L2 scan (3 rotating copies) + AdamW (lr 1e-3, wd 0.01) over 100M f32, "
                        "f64 m/v")
    hn, hi, ss = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
    scan = Rot([lambda t=t: lib.neural_tensor_scan(t._ptr, ctypes.byref(hn), ctypes.byref(hi), ctypes.byref(ss))
                for t in tgs])
    cf.add("scan", "k_reduce_seg + k_reduce_combine (flags + sum of squares to the host)", 4 * NA, NA,
           *clock.op(scan), host_call_us=clock.host_call_us(scan))
    flags = (hn.value, hi.value)
    opt = pn.AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01)
    cf.add("adamw", "k_adam_f32<AdamW>", 44 * NA, NA, *clock.op(lambda: opt.step([tp], [tg])))
    lib.neural_tensor_scan(tcl._ptr, ctypes.byref(hn), ctypes.byref(hi), ctypes.byref(ss))
    clean_norm = ss.value ** 0.5
    cpu = cpu_cfg5(p, clean, gr) if cpu_on else None
    out["cfg5"] = cf.summary(cpu)
    out["cfg5"]["check"] = {"nan_inf_flags": list(flags), "clean_l2": round(clean_norm, 6)}
    detail["cfg5"] = cf.detail()
    if cpu:
        detail["cfg5"]["cpu"] = cpu
    out["cfg5"]["host_e2e"] = host_e2e_cfg5(torch, pn, lib, tg)
    del p, gr, clean, tp, tg, tcl, opt, gs, tgs
    torch.cuda.empty_cache()


# ------------------------------------------------------------- host buffers, end to end

def _host_timed(fn, reps=CPU_REPS):
    """Median host-clock seconds of fn (one warm-up call first)."""
    return _median_time(fn, reps=reps, warm=1)


def host_e2e_cfg4(torch, pn, q_dev):
    """The reference's Quantizer calls on host arrays as its Python makes them
    (pyneural/quantize.py:76-151: float64 data, a fresh ctypes int8 / float64
    output array per call), through this library: host-clock time per call,
    PCIe copies (staged through HBM) and the output array's allocation
    included; rates over the same algorithmic bytes as the device ops (8 B
    read per value for the float64 API).  Reported beside the device-resident
    figures, never as them."""
    import numpy as np
    x = q_dev.cpu().numpy().astype(np.float64)
    n = x.size
    qz = pn.Quantizer(symmetric=True)
    qz.calibrate(x.ctypes.data, n)
    codes = qz.quantize(x.ctypes.data, n)
    t_cal = _host_timed(lambda: qz.calibrate(x.ctypes.data, n))
    t_q = _host_timed(lambda: qz.quantize(x.ctypes.data, n))
    t_dq = _host_timed(lambda: qz.dequantize(codes, n))
    out = {"w": f"Quantizer(symmetric=True) on {n:,} float64 values in host memory (the reference's API dtype)",
           "calibrate_ms": round(1e3 * t_cal, 2), "calibrate_GBps": round(8 * n / t_cal / 1e9, 2),
           "quantize_ms": round(1e3 * t_q, 2), "quantize_GBps": round(9 * n / t_q / 1e9, 2),
           "dequantize_ms": round(1e3 * t_dq, 2), "dequantize_GBps": round(9 * n / t_dq / 1e9, 2),
           "timing": f"host clock per call, median of {CPU_REPS} after one warm-up"}
    del x, codes
    return out


def host_e2e_cfg5(torch, pn, lib, tg):
    """NaN/Inf/L2 checks of the 100M-element gradient right after a kernel
    wrote it, as the reference's training.py:43-79 makes them (a host pointer
    from neural_tensor_data(), then the raw-pointer entry points; check() is
    has_nan then has_inf, each fetching the pointer again) and as this
    package's NaNDetector makes them (one device scan of the tensor).  Host
    clock per call, the rewrite of the gradient between calls excluded."""
    from pyneural.training import NaNDetector
    n = int(lib.neural_tensor_numel(tg._ptr))

    def dirty():  # g = g * 1 in place: the device copy is newer than the host mirror
        lib.neural_scalar_mul(tg._ptr, tg._ptr, ctypes.c_double(1.0))
        torch.cuda.synchronize()

    # the reference's tensors are library-owned (host mirror + device copy)
    own = pn.Tensor.create([n])
    pn.core._check_error(lib.neural_tensor_copy(own._ptr, tg._ptr), "copy")
    tg = own

    def ref_check():
        p = lib.neural_tensor_data(tg._ptr)
        lib.neural_tensor_has_nan(p, n)
        p = lib.neural_tensor_data(tg._ptr)
        lib.neural_tensor_has_inf(p, n)

    def ref_norm():
        lib.neural_tensor_grad_l2_norm(lib.neural_tensor_data(tg._ptr), n)

    det = NaNDetector(raise_on_detect=False)

    def timed(fn, reps=CPU_REPS):
        ts = []
        for r in range(reps + 1):
            dirty()
            t = time.perf_counter()
            fn()
            if r:
                ts.append(time.perf_counter() - t)
        return statistics.median(ts)

    t_ref, t_norm, t_dev = timed(ref_check), timed(ref_norm), timed(lambda: det.check(tg))
    return {"w": f"{n:,} f32 gradient resident on the device, rewritten by a kernel before each call",
            "reference_check_ms": round(1e3 * t_ref, 2),
            "reference_grad_l2_norm_ms": round(1e3 * t_norm, 2),
            "pyneural_check_ms": round(1e3 * t_dev, 3),
            "reference_check_GBps": round(4 * n / t_ref / 1e9, 2),
            "note": "reference shape: neural_tensor_data() downloads the tensor (PCIe); the raw-pointer scan "
                    "resolves the mirror to the tensor's device copy (one upload, no staging buffer, no re-upload "
                    "by the next kernel)",
            "timing": f"host clock per call, median of {CPU_REPS} after one warm-up"}


# ----------------------------------------------------------------------------- CPU legs

def _cpu_entry(ops, kind, sample, extra=None):
    """Aggregate GB/s over the ops ({op: (bytes, seconds)}), one thread."""
    tot_b = sum(b for b, _ in ops.values())
    tot_s = sum(s for _, s in ops.values())
    e = {"value": round(tot_b / tot_s / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": kind, "sample": sample,
         "_ops": {k: {"GB/s": round(b / s / 1e9, 3), "ms": round(1e3 * s, 2)} for k, (b, s) in ops.items()}}
    if extra:
        e.update(extra)
    return e


def cpu_baseline_cfg2(X, b, S, step_bytes):
    """The oracle's C restatement of the cfg2 step (reference loop orders,
    scalar libm exp/log, -O2, one thread), on the same data copied to host."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import ora
    x, bb, s = X.cpu().numpy(), b.cpu().numpy(), S.cpu().numpy()

    def run():
        y = ora.bias_add(x, bb)
        ora.rowsum_ref(y)
        ora.rowsum_ref(y) / np.float32(COLS)  # reduce_mean = row sum then divide
        ora.rowmax_chain(y)
        ora.rowargmax(y)
        ora.softmax_rows(s)
        ora.softmax_rows(s, log=True)
    sec = _median_time(run)
    return {
        "value": round(step_bytes / sec / 1e9, 2),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full cfg2 step on host (oracle/liboracle.so, gcc -O2 SSE2), median of {CPU_REPS} after one "
                  f"warm-up = {sec:.3f} s",
        "nproc": os.cpu_count(),
        "cpu_model": _cpu_model(),
        "threads": "1 (the reference never dispatches to its thread pool: pool size 1, unused)",
    }


def cpu_cfg1(a_dev, b_dev, n):
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import ora
    c = ora.cpu()
    a, b = a_dev.cpu().numpy(), b_dev.cpu().numpy()
    o = np.empty_like(a)
    ops = {}
    if c.cpu_has_avx():
        ops["add"] = (12 * n, _median_time(lambda: ora.cpu_binary("cpu_ew_add_avx", a, b, o)))
        ops["mul"] = (12 * n, _median_time(lambda: ora.cpu_binary("cpu_ew_mul_avx", a, b, o)))
    ops["relu"] = (8 * n, _median_time(lambda: ora.cpu_relu_node(a, o)))
    if c.cpu_has_avx():
        ops["sum"] = (4 * n, _median_time(lambda: ora.cpu_sum("cpu_reduce_sum_avx", a)))
    ops["max"] = (4 * n, _median_time(lambda: ora.max_chain(a)))
    e = _cpu_entry(ops, "port", "full 64M arrays: AVX-256 add/mul/sum (math_kernels.asm), node_relu 3 passes, "
                   "scalar maxss max; oracle/cpu_baseline.c -O2, median of 5 after one warm-up")
    if c.cpu_has_avx512f():
        ops5 = {"add": (12 * n, _median_time(lambda: ora.cpu_binary("cpu_simd_add_avx512", a, b, o))),
                "mul": (12 * n, _median_time(lambda: ora.cpu_binary("cpu_simd_mul_avx512", a, b, o))),
                "sum": (4 * n, _median_time(lambda: ora.cpu_sum("cpu_simd_sum_avx512", a)))}
        e5 = _cpu_entry(ops5, "port", "simd.asm AVX-512 path (exported, never called by the reference)")
        e["avx512"] = {"value": e5["value"], "kind": "port: simd.asm AVX-512 path, never called in the reference",
                       "_ops": e5["_ops"]}
    else:
        e["avx512"] = {"value": None, "kind": "host has no AVX-512F"}
    return e


class _TensorC(ctypes.Structure):
    """The 40-byte prefix of the reference descriptor (activations_c.c:36-43)."""
    _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int64), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("stride", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("flags", ctypes.c_int32)]


def _tensor_c(arr, keep):
    shape = (ctypes.c_int64 * arr.ndim)(*arr.shape)
    keep.append(shape)
    return _TensorC(arr.ctypes.data, arr.ndim, shape, None, 0 if arr.dtype.itemsize == 4 else 1, 0)


def _ref():
    sys.path.insert(0, str(ROOT / "oracle"))
    import ora
    return ora, ora.ref()


CPU_ACT_SAMPLE = 1 << 22


def cpu_cfg3(x_dev, dt_name, bpe):
    import numpy as np
    ora, ref = _ref()
    if ref is None:
        return None
    x = x_dev.reshape(-1)[:CPU_ACT_SAMPLE].cpu().numpy()
    y = np.empty_like(x)
    keep = []
    ti, to = _tensor_c(x, keep), _tensor_c(y, keep)
    ops = {}
    for nm in ACTS:
        fn = getattr(ref, "act_" + nm)
        if nm in ACT_ALPHA:
            fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_double]
            run = (lambda fn=fn, al=ACT_ALPHA[nm]: fn(ctypes.addressof(to), ctypes.addressof(ti), al))
        else:
            fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            run = (lambda fn=fn: fn(ctypes.addressof(to), ctypes.addressof(ti)))
        ops[nm] = (bpe * x.size, _median_time(run))
    return _cpu_entry(ops, "reference", f"activations_c.c compiled unchanged (oracle/_ref, -O2 SSE2, glibc libm), "
                      f"first {CPU_ACT_SAMPLE:,} elements of the same {dt_name} input")


CPU_Q_SAMPLE = 1 << 24


def cpu_cfg4(q_dev):
    import numpy as np
    ora, ref = _ref()
    if ref is None:
        return None
    x = q_dev[:CPU_Q_SAMPLE].cpu().numpy().astype(np.float64)  # the reference API is double-in (exact widening)
    n = x.size
    P = ctypes.c_void_p
    ref.calibrate_minmax.argtypes = [P, ctypes.c_int64, ctypes.c_int, P]
    ref.quantize_tensor.argtypes = [P, P, ctypes.c_int64, P]
    ref.dequantize_tensor.argtypes = [P, P, ctypes.c_int64, P]
    ps, pa = ora.QuantParams(), ora.QuantParams()
    q = np.empty(n, dtype=np.int8)
    d = np.empty(n)
    ops = {
        "calibrate_sym": (4 * n, _median_time(lambda: ref.calibrate_minmax(x.ctypes.data, n, 1, ctypes.byref(ps)))),
        "calibrate_aff": (4 * n, _median_time(lambda: ref.calibrate_minmax(x.ctypes.data, n, 0, ctypes.byref(pa)))),
        "quantize_sym": (5 * n, _median_time(lambda: ref.quantize_tensor(x.ctypes.data, q.ctypes.data, n,
                                                                        ctypes.byref(ps)))),
        "quantize_aff": (5 * n, _median_time(lambda: ref.quantize_tensor(x.ctypes.data, q.ctypes.data, n,
                                                                        ctypes.byref(pa)))),
        "dequantize_f64": (9 * n, _median_time(lambda: ref.dequantize_tensor(q.ctypes.data, d.ctypes.data, n,
                                                                            ctypes.byref(pa)))),
    }
    return _cpu_entry(ops, "reference", f"quantize.c compiled unchanged (oracle/_ref, -O2 SSE2) on the first "
                      f"{n:,} values widened to double; bytes as the GPU op's f32 stream")


CPU_A_SAMPLE = 1 << 22


def cpu_cfg5(p_dev, clean_dev, g_dev):
    import numpy as np
    ora, ref = _ref()
    if ref is None:
        return None
    n = CPU_A_SAMPLE
    p = p_dev[:n].cpu().numpy()
    gr = g_dev[:n].cpu().numpy()
    keep = []
    tp, tg = _tensor_c(p, keep), _tensor_c(gr, keep)
    h = ref.opt_adamw_create(1e-3, 0.9, 0.999, 1e-8, 0.01)
    pp = (ctypes.c_void_p * 1)(ctypes.addressof(tp))
    gp = (ctypes.c_void_p * 1)(ctypes.addressof(tg))
    ref.opt_step(h, pp, gp, 1)  # first step allocates the f64 moments
    adam_s = _median_time(lambda: ref.opt_step(h, pp, gp, 1))
    ref.opt_free(h)
    g16 = clean_dev[: 4 * n].cpu().numpy()
    scan_s = _median_time(lambda: (ora.has_nan(g16), ora.has_inf(g16), ora.cpu_l2(g16)))
    ops = {"scan": (4 * g16.size, scan_s), "adamw": (44 * n, adam_s)}
    return _cpu_entry(ops, "reference + port", f"AdamW: optimizers_c.c compiled unchanged (oracle/_ref) on "
                      f"{n:,} params; scan: training_ops.asm has_nan + has_inf (scalar) + SSE L2 "
                      f"(oracle ports) over {g16.size:,} grads, 3 passes as the reference runs them")


# ------------------------------------------------------------------------- other families

SUITE_CPU_SAMPLE = 1 << 22  # elements of each family's CPU leg


def suite(torch, pn, clock, dev, cpu=True):
    """Kernel families outside BASELINE's configs (detail file only): for each
    op the kernel time of its main launch (`k`, HIP event pair on that launch)
    and, where a call makes several launches or returns a result to the host,
    the call time (`call`: the event span over all of the call's launches and
    gaps, or, where the result returns to the host, the host-clock time of
    the whole call), in us, with the algorithmic bytes of the main kernel.  With `cpu`, each op also carries its CPU leg
    (`cpu`: one host thread, GB/s over the same bytes per element) on a bounded
    sample (SUITE_CPU_SAMPLE elements, rows of it for the row ops) of the same
    input: the reference's own C (oracle/_ref, kind "reference") where it
    compiles, else the oracle's restatement of the reference loop ("port");
    the oracle allocates each output, which those timings include.  Inputs and
    outputs of ops whose footprint is below 1 GiB rotate over copies (NROT, or
    2-3 for the larger ones) between timed calls."""
    import numpy as np
    from pyneural.core import _lib, QuantParamsC
    W = pn.Tensor.from_torch
    res = {}
    ora, ref = _ref() if cpu else (None, None)

    def put(name, nbytes, k=None, call=None, op=None):
        e = {"bytes": int(nbytes)}
        if k is not None:
            e["k_us"] = round(k, 2)
            e["k_pct"] = pct(nbytes, k)
        if call is not None:
            e["call_us"] = round(call, 2)
            e["call_pct"] = pct(nbytes, call)
        if op is not None:  # every launch of a call that leaves its result on the device
            e["op_us"] = round(op, 2)
            e["op_pct"] = pct(nbytes, op)
        res[name] = e

    def cpu_leg(name, nbytes, fn, kind, sample):
        if not cpu or (kind.startswith("reference") and ref is None):
            return
        sec = _median_time(fn)
        res[name]["cpu"] = {"GB/s": round(nbytes / sec / 1e9, 3), "ms": round(1e3 * sec, 2), "cores": 1,
                            "kind": kind, "sample": sample}

    g = torch.Generator(device=dev)
    g.manual_seed(7)
    # ---- bias add (>= 64M), fused bias + activation, row reductions at [16384,4096]
    R, C = 16384, 4096
    X = torch.randn(R, C, device=dev, generator=g) * 3
    bias = torch.randn(C, device=dev, generator=g) * 3
    Xs = copies(X)
    Ys = [torch.empty_like(X) for _ in range(NROT)]
    rs = torch.empty(R, device=dev)
    ri = torch.empty(R, dtype=torch.int64, device=dev)
    tX, tY, tb, trs = [W(t) for t in Xs], [W(t) for t in Ys], W(bias), W(rs)
    torch.cuda.synchronize()

    def rot(call, nset=NROT):
        return Rot([lambda k=k: call(k) for k in range(nset)])

    put("bias_add_f32_16384x4096", 8 * R * C,
        clock.kernel_us(rot(lambda k: _lib.neural_bias_add(tY[k]._ptr, tX[k]._ptr, tb._ptr))))
    for nm, act in (("relu", 1), ("gelu", 4)):
        put(f"bias_add_{nm}_f32_16384x4096", 8 * R * C, clock.kernel_us(rot(
            lambda k, act=act: _lib.neural_bias_add_act(tY[k]._ptr, tX[k]._ptr, tb._ptr, act, ctypes.c_double(0.0)))))
    put("row_sum_f32_16384x4096", 4 * R * C,
        clock.kernel_us(rot(lambda k: _lib.neural_reduce_sum(tY[k]._ptr, 1, trs._ptr))))
    put("row_max_f32_16384x4096", 4 * R * C,
        clock.kernel_us(rot(lambda k: _lib.neural_reduce_max(tY[k]._ptr, 1, trs._ptr))))
    put("row_argmax_f32_16384x4096", 4 * R * C,
        clock.kernel_us(rot(lambda k: _lib.neural_reduce_argmax(tY[k]._ptr, 1, ri.data_ptr()))))
    if cpu:
        rows = SUITE_CPU_SAMPLE // C
        Xh, bh = X[:rows].cpu().numpy(), bias.cpu().numpy()
        Yh = ora.bias_add(Xh, bh)
        smp = f"first {rows} rows"
        cpu_leg("bias_add_f32_16384x4096", 8 * Xh.size, lambda: ora.bias_add(Xh, bh), "port", smp)
        cpu_leg("bias_add_relu_f32_16384x4096", 8 * Xh.size, lambda: ora.relu(ora.bias_add(Xh, bh)), "port",
                smp + ": bias add, then ReLU, as the reference runs them")
        cpu_leg("bias_add_gelu_f32_16384x4096", 8 * Xh.size, lambda: ora.act("gelu", ora.bias_add(Xh, bh)), "port",
                smp + ": bias add, then GELU (activations_c.c formula)")
        cpu_leg("row_sum_f32_16384x4096", 4 * Yh.size, lambda: ora.rowsum_ref(Yh), "port", smp)
        cpu_leg("row_max_f32_16384x4096", 4 * Yh.size, lambda: ora.rowmax_chain(Yh), "port", smp)
        cpu_leg("row_argmax_f32_16384x4096", 4 * Yh.size, lambda: ora.rowargmax(Yh), "port", smp)
    del X, Xs, Ys, tX, tY, rs, ri, trs
    torch.cuda.empty_cache()

    # ---- dropout forward / backward, 64M f32, p = 0.5
    n = N1
    a = torch.rand(n, device=dev, generator=g) * 2 - 1
    a_s = copies(a)
    c_s = [torch.empty_like(a) for _ in range(NROT)]
    m_s = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(NROT)]
    torch.cuda.synchronize()
    # Repeated calls with one (n, p), as a training loop makes them: each call's
    # apply pass also makes the next call's keep bits, so a call is one launch.
    # A call whose (n, p) differs from the previous call's (here p alternates
    # between 0.5 and the next float up, a different threshold) runs the
    # keep-bit pass first, then the plain apply pass.
    fwd = rot(lambda k: _lib.neural_dropout_forward(a_s[k].data_ptr(), c_s[k].data_ptr(), m_s[k].data_ptr(), n,
                                                    ctypes.c_float(0.5)))
    alt_p = [0.5, float(np.nextafter(np.float32(0.5), np.float32(1)))]

    def alt_call(k):
        alt_p.reverse()
        return _lib.neural_dropout_forward(a_s[k].data_ptr(), c_s[k].data_ptr(), m_s[k].data_ptr(), n,
                                           ctypes.c_float(alt_p[0]))

    alt = rot(alt_call)
    clock.warm(fwd)
    k, o, nl = clock.op(fwd)
    put("dropout_fwd_f32_64M", 9 * n, k if nl == 1 else None, o)
    put("dropout_fwd_new_p_f32_64M", 9 * n, None, clock.op(alt)[1])
    put("dropout_fwd_keep_bits_f32_64M", 0, clock.kernel_us(alt, skip=0))
    put("dropout_fwd_apply_f32_64M", 9 * n, clock.kernel_us(alt, skip=1))
    put("dropout_bwd_f32_64M", 9 * n, clock.kernel_us(rot(
        lambda k: _lib.neural_dropout_backward(a_s[k].data_ptr(), c_s[k].data_ptr(), m_s[k].data_ptr(), n,
                                               ctypes.c_float(0.5)))))
    if cpu:
        xh = a[:SUITE_CPU_SAMPLE].cpu().numpy()
        _, _, mh = ora.dropout_forward(xh, 0.5)
        smp = f"first {xh.size:,} elements; glibc rand() per element"
        cpu_leg("dropout_fwd_f32_64M", 9 * xh.size, lambda: ora.dropout_forward(xh, 0.5), "port", smp)
        cpu_leg("dropout_bwd_f32_64M", 9 * xh.size, lambda: ora.dropout_backward(xh, mh, 0.5), "port",
                f"first {xh.size:,} elements")
    del a, a_s, c_s, m_s
    torch.cuda.empty_cache()

    # ---- cross-entropy [65536,1024]: label-smoothed forward / fused (f64, f32), tensor CE loss (f32)
    B, K = 65536, 1024
    tgt = torch.randint(0, K, (B,), device=dev, dtype=torch.int64, generator=g)
    lossv = ctypes.c_double()
    L64 = torch.randn(B, K, device=dev, dtype=torch.float64, generator=g) * 3
    G64 = torch.empty_like(L64)
    L64s = copies(L64, 2)  # the forward reads 537 MB per call: two copies
    torch.cuda.synchronize()
    f = rot(lambda k: _lib.label_smoothing_ce_forward(L64s[k].data_ptr(), tgt.data_ptr(), B, K, 0.1,
                                                      ctypes.byref(lossv)), 2)
    put("ls_ce_forward_f64_65536x1024", 8 * B * K, clock.kernel_us(f), clock.host_call_us(f))
    # the NEW form that leaves the loss in device memory: no host wait
    dloss = torch.zeros(1, dtype=torch.float64, device=dev)
    f = rot(lambda k: _lib.label_smoothing_ce_forward_dev(L64s[k].data_ptr(), tgt.data_ptr(), B, K, 0.1,
                                                          dloss.data_ptr()), 2)
    kk, op, _ = clock.op(f)
    put("ls_ce_forward_dev_f64_65536x1024", 8 * B * K, kk, op=op)
    f = lambda: _lib.label_smoothing_ce_fused(L64.data_ptr(), tgt.data_ptr(), B, K, 0.1, ctypes.byref(lossv),
                                              G64.data_ptr())
    put("ls_ce_fused_f64_65536x1024", 16 * B * K, clock.kernel_us(f), clock.host_call_us(f))
    if cpu:
        rows = SUITE_CPU_SAMPLE // K
        Lh, th = L64[:rows].cpu().numpy(), tgt[:rows].cpu().numpy()
        smp = f"first {rows} rows; metrics_losses.c compiled unchanged"
        cpu_leg("ls_ce_forward_f64_65536x1024", 8 * Lh.size, lambda: ora.ls_ce_forward(Lh, th, 0.1, use_ref=True),
                "reference", smp)
        cpu_leg("ls_ce_fused_f64_65536x1024", 16 * Lh.size,
                lambda: (ora.ls_ce_forward(Lh, th, 0.1, use_ref=True), ora.ls_ce_backward(Lh, th, 0.1, use_ref=True)),
                "reference", smp + ": forward, then backward")
    del L64, G64, L64s
    L32 = torch.randn(B, K, device=dev, generator=g) * 3
    L32s = copies(L32)
    G32s = [torch.empty_like(L32) for _ in range(NROT)]
    torch.cuda.synchronize()
    f = rot(lambda k: _lib.label_smoothing_ce_fused_f32(L32s[k].data_ptr(), tgt.data_ptr(), B, K, 0.1,
                                                        ctypes.byref(lossv), G32s[k].data_ptr()))
    put("ls_ce_fused_f32_65536x1024", 8 * B * K, clock.kernel_us(f), clock.host_call_us(f))
    f = rot(lambda k: _lib.label_smoothing_ce_fused_f32_dev(L32s[k].data_ptr(), tgt.data_ptr(), B, K, 0.1,
                                                            dloss.data_ptr(), G32s[k].data_ptr()))
    kk, op, _ = clock.op(f)
    put("ls_ce_fused_f32_dev_65536x1024", 8 * B * K, kk, op=op)
    tv = W(tgt.float())
    tL = [W(t) for t in L32s]
    f = rot(lambda k: _lib.neural_cross_entropy_loss(tL[k]._ptr, tv._ptr, ctypes.byref(lossv)))
    put("ce_loss_f32_65536x1024", 4 * B * K, clock.kernel_us(f), clock.host_call_us(f))
    if cpu:
        rows = SUITE_CPU_SAMPLE // K
        Lh, th = L32[:rows].cpu().numpy(), tgt[:rows].cpu().numpy()
        Lw = Lh.astype("float64")
        cpu_leg("ls_ce_fused_f32_65536x1024", 8 * Lh.size,
                lambda: (ora.ls_ce_forward(Lw, th, 0.1, use_ref=True), ora.ls_ce_backward(Lw, th, 0.1, use_ref=True)),
                "reference", f"first {rows} rows widened to double (the reference API is double-only); "
                             "metrics_losses.c forward, then backward")
        tvh = th.astype("float32")
        cpu_leg("ce_loss_f32_65536x1024", 4 * Lh.size, lambda: ora.ce_loss(Lh, tvh), "port", f"first {rows} rows")
    del L32, L32s, G32s, tL, tv, tgt
    torch.cuda.empty_cache()

    # ---- gradient clipping over one 100M f32 gradient (norm: sum of squares,
    # decide, scale; each timed call clips by 0.999, so every call scales)
    # three rotating copies (400 MB each): every copy is clipped in turn with
    # a max_norm that keeps falling, so every timed call scales
    na = NA
    gr = torch.randn(na, device=dev, generator=g) * 1e-3
    grs = copies(gr, 3)
    tgs = [W(t) for t in grs]
    glists = [(ctypes.c_void_p * 1)(t._ptr) for t in tgs]
    tot = ctypes.c_double()
    torch.cuda.synchronize()
    _lib.neural_clip_grad_norm_list(glists[0], 1, ctypes.c_double(1e30), ctypes.byref(tot))
    state = {"m": tot.value}

    def clip_scaling(k):
        state["m"] *= 0.999
        return _lib.neural_clip_grad_norm_list(glists[k], 1, ctypes.c_double(state["m"]), ctypes.byref(tot))

    put("clip_grad_norm_clipping_f32_100M", 12 * na, None, clock.host_call_us(rot(clip_scaling, 3)))
    put("clip_grad_norm_below_f32_100M", 4 * na, None, clock.host_call_us(rot(
        lambda k: _lib.neural_clip_grad_norm_list(glists[k], 1, ctypes.c_double(1e30), ctypes.byref(tot)), 3)))
    f = rot(lambda k: _lib.neural_clip_grad_value_list(glists[k], 1, ctypes.c_double(-1e-3), ctypes.c_double(1e-3)),
            3)
    put("clip_grad_value_f32_100M", 8 * na, clock.kernel_us(f), clock.op(f)[1])
    if cpu:
        gh = gr[:SUITE_CPU_SAMPLE].cpu().numpy()
        nh = ora.clip_grad_norm([gh], 1e30)[0]
        smp = f"first {gh.size:,} elements; the port clips a copy, which the timing includes"
        cpu_leg("clip_grad_norm_clipping_f32_100M", 12 * gh.size, lambda: ora.clip_grad_norm([gh], 0.5 * nh), "port",
                smp)
        cpu_leg("clip_grad_norm_below_f32_100M", 4 * gh.size, lambda: ora.clip_grad_norm([gh], 1e30), "port", smp)
        cpu_leg("clip_grad_value_f32_100M", 8 * gh.size, lambda: ora.clip_grad_value([gh], -1e-3, 1e-3), "port", smp)
    del gr, grs, tgs, glists
    torch.cuda.empty_cache()

    # ---- per-feature transforms, [1M, 64] f64, device pointers
    TB, TF = 1 << 20, 64
    D = torch.randn(TB, TF, device=dev, dtype=torch.float64, generator=g) * 2 + 1
    Ds = copies(D, 2)  # the statistics read 537 MB per call: two copies
    O = torch.empty_like(D)
    st = [torch.empty(TF, device=dev, dtype=torch.float64) for _ in range(4)]
    torch.cuda.synchronize()
    f = rot(lambda k: _lib.transform_compute_stats(Ds[k].data_ptr(), TB, TF, *[t.data_ptr() for t in st]), 2)
    put("transform_compute_stats_f64_1Mx64", 8 * TB * TF, clock.kernel_us(f), clock.op(f)[1])
    f = lambda: _lib.transform_normalize(D.data_ptr(), O.data_ptr(), TB, TF, st[0].data_ptr(), st[1].data_ptr(),
                                         ctypes.c_double(1e-8))
    put("transform_normalize_f64_1Mx64", 16 * TB * TF, clock.kernel_us(f), clock.op(f)[1])
    if cpu:
        Dh = D[:SUITE_CPU_SAMPLE // TF].cpu().numpy()
        _, mu, sd, _, _ = ora.transform_stats(Dh, use_ref=True)
        smp = f"first {Dh.shape[0]:,} rows; transforms.c compiled unchanged"
        cpu_leg("transform_compute_stats_f64_1Mx64", 8 * Dh.size, lambda: ora.transform_stats(Dh, use_ref=True),
                "reference", smp)
        cpu_leg("transform_normalize_f64_1Mx64", 16 * Dh.size,
                lambda: ora.transform_apply(0, Dh, mu, sd, 1e-8, use_ref=True), "reference", smp)
    del D, Ds, O, st
    torch.cuda.empty_cache()

    # ---- the rest of the quantization API: percentile calibration (64M f64)
    # and the int8 product (4096^3, device pointers)
    P = torch.randn(1 << 26, device=dev, dtype=torch.float64, generator=g)
    Ps = copies(P, 2)
    qp = QuantParamsC()
    torch.cuda.synchronize()
    put("calibrate_percentile_f64_64M", 8 * P.numel(), None, clock.host_call_us(rot(
        lambda k: _lib.calibrate_percentile(Ps[k].data_ptr(), P.numel(), ctypes.c_double(0.01), 1,
                                            ctypes.byref(qp)), 2)))
    if cpu:
        Ph = P[:SUITE_CPU_SAMPLE].cpu().numpy()
        cpu_leg("calibrate_percentile_f64_64M", 8 * Ph.size,
                lambda: ora.calibrate_percentile(Ph, 0.01, True, use_ref=True), "reference",
                f"first {Ph.size:,} values; quantize.c (qsort) compiled unchanged")
    del P, Ps
    m = 4096
    A8 = torch.randint(-128, 128, (m, m), dtype=torch.int8, device=dev, generator=g)
    B8 = torch.randint(-128, 128, (m, m), dtype=torch.int8, device=dev, generator=g)
    C8 = torch.empty(m, m, dtype=torch.float64, device=dev)
    pa, pb = QuantParamsC(), QuantParamsC()
    pa.scale, pa.zero_point, pb.scale, pb.zero_point = 0.013, -7, 0.37, 11
    torch.cuda.synchronize()
    us = clock.op(lambda: _lib.quantized_matmul(A8.data_ptr(), B8.data_ptr(), C8.data_ptr(), m, m, m,
                                                     ctypes.byref(pa), ctypes.byref(pb)))[1]
    res["quantized_matmul_4096^3"] = {"call_us": round(us, 2), "int8_TOPS": round(2.0 * m ** 3 / us / 1e6, 1)}
    if cpu and ref is not None:
        mc = 256
        Ah, Bh = A8[:mc, :mc].cpu().numpy(), B8[:mc, :mc].cpu().numpy()
        qa, qb = ora.QuantParams(), ora.QuantParams()
        qa.scale, qa.zero_point, qb.scale, qb.zero_point = 0.013, -7, 0.37, 11
        sec = _median_time(lambda: ora.quantized_matmul(Ah, Bh, mc, mc, mc, qa, qb, use_ref=True))
        res["quantized_matmul_4096^3"]["cpu"] = {
            "int8_TOPS": round(2.0 * mc ** 3 / sec / 1e12, 4), "ms": round(1e3 * sec, 2), "cores": 1,
            "kind": "reference", "sample": f"{mc}^3 corner of the same operands; quantize.c compiled unchanged"}
    del A8, B8, C8
    torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    main()
