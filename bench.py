#!/usr/bin/env python3
"""
Benchmark of the tensor hot path on one MI355X.

Default workload = BASELINE.json configs[1] (cfg2): one step is
  bias-add      Y[8192,4096] = X + b[4096]                 (nn_layers.asm:472-539)
  row sum, mean, max, argmax over the last dim of Y        (math_kernels.asm:956-1264, main.asm:3245-3292)
  softmax and log-softmax rows of S[65536,1024]            (activations.asm:761-987, metrics_losses.c:47-64)
on synthetic fp32 inputs N(0,3) already resident in HBM.  The metric is the
achieved HBM bandwidth: algorithmic bytes (each input read once, each output
written once) divided by the step time.

Prints ONE JSON line (the driver contract) with a roofline object for the
dominant kernel (row softmax on [65536,1024]: each launch inside the timed
steps carries a pair of HIP events -- created with hipEventDisableSystemFence
and handed to the library by neural_hip_time_next_softmax, which launches the
kernel with hipExtLaunchKernelGGL -- so each pair times that kernel's own
execution on its stream; a back-to-back figure after the timed region is
reported beside it) and a cpu_baseline object (the oracle's C restatement of the same step,
single-threaded, on this host).

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--suite]   (--suite: per-kernel table on stderr)
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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--suite", action="store_true", help="also time every kernel family (stderr table)")
    ap.add_argument("--suite-json", default=None, help="write the per-kernel table to this file")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--calib", action="store_true",
                    help="also run a plain 256 MiB device copy (the PMC byte-counter calibration kernel)")
    return ap.parse_args()


def traffic_from_profile():
    """HBM bytes per softmax launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration factor)."""
    p = ROOT / "profiles" / "softmax_f32_65536x1024_pmc.json"
    if not p.exists():
        return None
    try:
        return float(json.loads(p.read_text())["traffic_bytes_per_launch"])
    except Exception:
        return None


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


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path would shard by rows / element ranges with one scalar all-reduce per global "
              "reduction", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    import pyneural as pn
    from pyneural.core import _lib, _check_error

    pn.init()
    # A dedicated (non-null) torch stream: the library launches on it and the
    # HIP events below are recorded on it.
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    pn.set_stream(stream.cuda_stream)
    dev = torch.device("cuda:0")

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

    sm_times = []

    def step(record):
        _check_error(_lib.neural_bias_add(T["Y"]._ptr, T["X"]._ptr, T["b"]._ptr), "bias_add")
        _check_error(_lib.neural_reduce_sum(T["Y"]._ptr, 1, T["rsum"]._ptr), "row sum")
        _check_error(_lib.neural_reduce_mean(T["Y"]._ptr, 1, T["rmean"]._ptr), "row mean")
        _check_error(_lib.neural_reduce_max(T["Y"]._ptr, 1, T["rmax"]._ptr), "row max")
        _check_error(_lib.neural_reduce_argmax(T["Y"]._ptr, 1, ctypes.c_void_p(ridx.data_ptr())), "row argmax")
        if record:
            # the events ride on the softmax kernel's own launch (hipExtLaunchKernelGGL)
            e0, e1 = ev_pairs[len(sm_times)]
            _check_error(_lib.neural_hip_time_next_softmax(e0.ev, e1.ev), "time_next_softmax")
        _check_error(_lib.neural_softmax(T["P"]._ptr, T["S"]._ptr), "softmax")
        if record:
            sm_times.append((e0, e1))
        _check_error(_lib.neural_log_softmax(T["L"]._ptr, T["S"]._ptr), "log_softmax")

    # Event pairs for the roofline kernel, created before the timed region.
    ev_pairs = [(TimingEvent(), TimingEvent()) for _ in range(args.steps)]
    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        step(True)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    sm_ms = statistics.mean(a.elapsed_time(c) for a, c in sm_times)
    # The same kernel launched back to back after the timed steps (its input
    # and output then partly in the last-level cache from the previous launch):
    # reported beside the in-step figure.
    b0, b1 = TimingEvent(), TimingEvent()
    b0.record(stream)
    for _ in range(args.steps):
        _check_error(_lib.neural_softmax(T["P"]._ptr, T["S"]._ptr), "softmax")
    b1.record(stream)
    torch.cuda.synchronize()
    sm_b2b_ms = b0.elapsed_time(b1) / args.steps

    n1, n2 = ROWS * COLS, SROWS * SCOLS
    step_bytes = (2 * n1 * 4 + COLS * 4) + 3 * (n1 * 4 + ROWS * 4) + (n1 * 4 + ROWS * 8) + 2 * (2 * n2 * 4)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    sm_bytes = 2 * n2 * 4
    sm_gbs = sm_bytes / (sm_ms * 1e-3) / 1e9

    cpu = None if args.no_cpu else cpu_baseline(X, b, S, step_bytes)

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
        "data": "synthetic: torch N(0,3) fp32, seeds 2 (X, b) and 3 (S), resident in HBM",
        "config": {
            "workload": "cfg2: bias-add [8192,4096]+[4096]; row sum/mean/max/argmax; softmax + log-softmax rows [65536,1024]",
            "step_bytes": step_bytes,
            "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 1),
            # elements through the step's ops: bias add and four row reductions
            # over [8192,4096], softmax and log-softmax over [65536,1024]
            "elements_per_s": round((5 * n1 + 2 * n2) / (ms_per_step * 1e-3), 0),
        },
        "roofline": {
            "kernel": "k_softmax_wave_f32<false,4,true,1> (neural_softmax [65536,1024] f32)",
            "bound": "hbm",
            "achieved": round(sm_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(sm_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profile(),
            "avg_launch_us": round(sm_ms * 1e3, 2),
            "algorithmic_bytes": sm_bytes,
            "backtoback_us": round(sm_b2b_ms * 1e3, 2),
            "achieved_backtoback": round(sm_bytes / (sm_b2b_ms * 1e-3) / 1e9, 1),
        },
        "cpu_baseline": cpu,
    }
    if cpu:
        line["config"]["speedup_vs_cpu"] = round(value / cpu["value"], 1)

    if args.calib:
        # Known-size copy: FETCH_SIZE / WRITE_SIZE of this dispatch calibrate the
        # byte counters (256 MiB read + 256 MiB written).
        src = torch.empty(64 << 20, device=dev).uniform_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()

    if args.suite:
        rows = suite(torch, pn, stream)
        if args.suite_json:
            Path(args.suite_json).write_text(json.dumps(rows, indent=1))
        for r in rows:
            print(json.dumps(r), file=sys.stderr, flush=True)
    pn.set_stream(None)
    print(json.dumps(line), flush=True)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_baseline(X, b, S, step_bytes):
    """The oracle's C restatement of the same step (reference loop orders,
    scalar libm exp/log, -O2, one thread), on the same data copied to host."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import ora
    x, bb, s = X.cpu().numpy(), b.cpu().numpy(), S.cpu().numpy()
    times = []
    for _ in range(3):
        t = time.perf_counter()
        y = ora.bias_add(x, bb)
        ora.rowsum_ref(y)
        ora.rowsum_ref(y) / np.float32(COLS)  # reduce_mean = row sum then divide
        ora.rowmax_chain(y)
        ora.rowargmax(y)
        ora.softmax_rows(s)
        ora.softmax_rows(s, log=True)
        times.append(time.perf_counter() - t)
    sec = statistics.median(times)
    return {
        "value": round(step_bytes / sec / 1e9, 2),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full cfg2 step on host (oracle/liboracle.so, gcc -O2 SSE2), median of 3 = {sec:.3f} s; "
                  f"host {_cpu_model()}, {os.cpu_count()} logical CPUs, 1 used (the reference never dispatches "
                  f"to its thread pool: pool size 1, unused)",
    }


def suite(torch, pn, stream):
    """Per-kernel timing on the BASELINE configs (HIP events, 3 warm + 10 timed)."""
    import numpy as np
    from pyneural.core import _lib, _check_error, QuantParamsC
    dev = torch.device("cuda:0")
    out = []

    def timeit(name, fn, nbytes, reps=10, flops=None, elems=None, int8_ops=None):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        r = {"kernel": name, "us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1),
             "pct_hbm": round(100 * nbytes / us / 1e3 / HBM_PEAK_GBS, 1), "bytes": nbytes}
        if elems:
            r["Gelem/s"] = round(elems / us / 1e3, 2)
        if copy_peak:
            r["x_rocm_copy"] = round(nbytes / us / 1e3 / copy_peak[0], 3)
        if flops:
            r["fp64_TFLOPs"] = round(flops / us / 1e6, 2)
        if int8_ops:
            r["int8_TOPS"] = round(int8_ops / us / 1e6, 1)
        out.append(r)
        print(json.dumps(r), file=sys.stderr, flush=True)

    W = pn.Tensor.from_torch
    n = 1 << 26
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    a = torch.rand(n, device=dev, generator=g) * 2 - 1
    b2 = torch.rand(n, device=dev, generator=g) * 2 - 1
    c = torch.empty_like(a)
    ta, tb, tc = W(a), W(b2), W(c)
    torch.cuda.synchronize()
    # every row is also quoted against a measured copy: torch's copy_ of the
    # same 64M-element vector, i.e. the ROCm runtime's device-to-device copy
    # kernel (x_rocm_copy = the row's GB/s over that copy's)
    copy_peak = []
    timeit("copy f32 64M (torch copy_ = ROCm runtime D2D copy kernel)", lambda: c.copy_(a), 8 * n, elems=n)
    copy_peak.append(out[-1]["GB/s"])
    out[-1]["x_rocm_copy"] = 1.0
    timeit("add f32 64M", lambda: _check_error(_lib.neural_add(tc._ptr, ta._ptr, tb._ptr), "add"), 12 * n, elems=n)
    timeit("mul f32 64M", lambda: _check_error(_lib.neural_mul(tc._ptr, ta._ptr, tb._ptr), "mul"), 12 * n, elems=n)
    timeit("relu f32 64M", lambda: _check_error(_lib.neural_relu(tc._ptr, ta._ptr), "relu"), 8 * n, elems=n)
    r = ctypes.c_double()
    one = torch.empty(1, device=dev)
    tone = W(one)
    timeit("sum f32 64M (device result)", lambda: _lib.neural_reduce_sum(ta._ptr, -1, tone._ptr), 4 * n, elems=n)
    timeit("max f32 64M (device result)", lambda: _lib.neural_reduce_max(ta._ptr, -1, tone._ptr), 4 * n, elems=n)
    one_i = torch.empty(1, dtype=torch.int64, device=dev)
    timeit("argmax f32 64M (device result)",
           lambda: _lib.neural_reduce_argmax(ta._ptr, -1, ctypes.c_void_p(one_i.data_ptr())), 4 * n, elems=n)
    timeit("sum f32 64M (host API, result on the host)", lambda: _lib.neural_sum(ta._ptr, ctypes.byref(r)), 4 * n, elems=n)
    X = torch.randn(16384, 4096, device=dev)
    bias = torch.randn(4096, device=dev)
    Y = torch.empty_like(X)
    tX, tbias, tY = W(X), W(bias), W(Y)
    torch.cuda.synchronize()
    timeit("bias_add f32 [16384,4096]", lambda: _lib.neural_bias_add(tY._ptr, tX._ptr, tbias._ptr), 8 * X.numel(), elems=X.numel())
    timeit("bias_add+relu fused f32 [16384,4096]",
           lambda: _lib.neural_bias_add_act(tY._ptr, tX._ptr, tbias._ptr, 1, ctypes.c_double(0.0)), 8 * X.numel(), elems=X.numel())
    timeit("bias_add+gelu fused f32 [16384,4096]",
           lambda: _lib.neural_bias_add_act(tY._ptr, tX._ptr, tbias._ptr, 4, ctypes.c_double(0.0)), 8 * X.numel(), elems=X.numel())
    # dropout over the 64M cfg1 vector: 4 B in + 4 B out + 1 B mask per element
    dmask = torch.empty(n, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    timeit("dropout fwd f32 64M (p=0.5, draws + apply)",
           lambda: _lib.neural_dropout_forward(a.data_ptr(), c.data_ptr(), dmask.data_ptr(), n, ctypes.c_float(0.5)), 9 * n, elems=n)
    timeit("dropout bwd f32 64M", lambda: _lib.neural_dropout_backward(a.data_ptr(), c.data_ptr(), dmask.data_ptr(), n,
                                                                       ctypes.c_float(0.5)), 9 * n, elems=n)
    del dmask
    rs = torch.empty(16384, device=dev)
    trs = W(rs)
    timeit("row sum f32 [16384,4096]", lambda: _lib.neural_reduce_sum(tX._ptr, 1, trs._ptr), 4 * X.numel(), elems=X.numel())
    timeit("row max f32 [16384,4096]", lambda: _lib.neural_reduce_max(tX._ptr, 1, trs._ptr), 4 * X.numel(), elems=X.numel())
    idx = torch.empty(16384, dtype=torch.int64, device=dev)
    timeit("row argmax f32 [16384,4096]",
           lambda: _lib.neural_reduce_argmax(tX._ptr, 1, ctypes.c_void_p(idx.data_ptr())), 4 * X.numel(), elems=X.numel())
    del X, Y, tX, tY
    S = torch.randn(65536, 1024, device=dev) * 3
    P = torch.empty_like(S)
    tS, tP = W(S), W(P)
    timeit("softmax f32 [65536,1024]", lambda: _lib.neural_softmax(tP._ptr, tS._ptr), 8 * S.numel(), elems=S.numel())
    timeit("log_softmax f32 [65536,1024]", lambda: _lib.neural_log_softmax(tP._ptr, tS._ptr), 8 * S.numel(), elems=S.numel())
    # cross-entropy on the same [65536,1024] logits (the label-smoothed and tensor CE entry points):
    # label-smoothed forward + backward in one pass (f32 and f64 logits, int64
    # targets), and the tensor cross_entropy_loss (reads the logits once)
    tgt = torch.randint(0, 1024, (65536,), device=dev, dtype=torch.int64)
    tgt_f = tgt.to(torch.float32)
    ttf = W(tgt_f)
    lossv = ctypes.c_double()
    timeit("ls_ce fused fwd+bwd f32 [65536,1024]",
           lambda: _lib.label_smoothing_ce_fused_f32(S.data_ptr(), tgt.data_ptr(), 65536, 1024, 0.1,
                                                     ctypes.byref(lossv), P.data_ptr()), 8 * S.numel(), elems=S.numel())
    timeit("cross_entropy_loss f32 [65536,1024] (result on the host)",
           lambda: _lib.neural_cross_entropy_loss(tS._ptr, ttf._ptr, ctypes.byref(lossv)), 4 * S.numel(), elems=S.numel())
    del P, tP
    S64 = S.double()
    G64 = torch.empty_like(S64)
    torch.cuda.synchronize()
    timeit("ls_ce fused fwd+bwd f64 [65536,1024]",
           lambda: _lib.label_smoothing_ce_fused(S64.data_ptr(), tgt.data_ptr(), 65536, 1024, 0.1,
                                                 ctypes.byref(lossv), G64.data_ptr()), 16 * S.numel(), elems=S.numel())
    timeit("ls_ce forward f64 [65536,1024] (result on the host)",
           lambda: _lib.label_smoothing_ce_forward(S64.data_ptr(), tgt.data_ptr(), 65536, 1024, 0.1,
                                                   ctypes.byref(lossv)), 8 * S.numel(), elems=S.numel())
    del S, tS, S64, G64
    # cfg3 activations: normal(0,4) with 1% of the values set to +-30 (saturation)
    x4 = torch.randn(64, 64, 128, 128, device=dev) * 4
    sat = torch.randperm(x4.numel(), device=dev)[: x4.numel() // 100]
    x4.view(-1)[sat] = 30.0 * (torch.randint(0, 2, (sat.numel(),), device=dev).float() * 2 - 1)
    del sat
    y4 = torch.empty_like(x4)
    tx4, ty4 = W(x4), W(y4)
    ne = x4.numel()
    acts = ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh"]
    for dt_name, xx, yy in (("f32", tx4, ty4), ("f64", None, None)):
        if dt_name == "f64":
            x8 = x4.double()
            y8 = torch.empty_like(x8)
            xx, yy = W(x8), W(y8)
            torch.cuda.synchronize()
        bpe = 8 if dt_name == "f32" else 16
        for nm in acts:
            fn = getattr(_lib, "act_" + nm)
            if nm in ("leaky_relu", "elu"):
                f = (lambda fn=fn: fn(yy._ptr, xx._ptr, ctypes.c_double(0.01 if nm == "leaky_relu" else 1.0)))
            else:
                f = (lambda fn=fn: fn(yy._ptr, xx._ptr))
            timeit(f"act_{nm} {dt_name} [64,64,128,128]", f, bpe * ne, elems=ne)
        if dt_name == "f64":
            del x8, y8
    del x4, y4
    # cfg4 quantization
    nq = 268435456
    q_in = torch.empty(nq, device=dev).exponential_() * (torch.randint(0, 2, (nq,), device=dev) * 2 - 1)
    q8 = torch.empty(nq, dtype=torch.int8, device=dev)
    dq = torch.empty(nq, device=dev)
    pbuf = torch.zeros(5, dtype=torch.float64, device=dev)
    torch.cuda.synchronize()
    timeit("calibrate_minmax f32 268M (device params)",
           lambda: _lib.calibrate_minmax_f32_dev(q_in.data_ptr(), nq, 0, pbuf.data_ptr()), 4 * nq, elems=nq)
    timeit("quantize f32->i8 268M", lambda: _lib.quantize_tensor_f32_dev(q_in.data_ptr(), q8.data_ptr(), nq,
                                                                       pbuf.data_ptr()), 5 * nq, elems=nq)
    timeit("dequantize i8->f32 268M", lambda: _lib.dequantize_tensor_f32_dev(q8.data_ptr(), dq.data_ptr(), nq,
                                                                           pbuf.data_ptr()), 5 * nq, elems=nq)
    del q_in, q8, dq
    # percentile calibration: exact radix select of two order statistics, 8 passes
    # over the data with a host read of the histograms between passes; bytes
    # counted as ONE read of the input (the algorithmic minimum)
    npc = 1 << 26
    pc_in = torch.randn(npc, device=dev, dtype=torch.float64)
    qp = pn.core.QuantParamsC()
    torch.cuda.synchronize()
    timeit("calibrate_percentile f64 64M p=0.01 (result on the host)",
           lambda: _lib.calibrate_percentile(pc_in.data_ptr(), npc, ctypes.c_double(0.01), 0, ctypes.byref(qp)),
           8 * npc, reps=5, elems=npc)
    del pc_in
    # int8 product C[M,N] f64 = dequant(A) dequant(B) on the matrix cores; bytes:
    # A + B read once, C written once (the algorithmic minimum)
    mq = kq = nq2 = 4096
    qa = torch.randint(-128, 128, (mq, kq), dtype=torch.int8, device=dev)
    qb = torch.randint(-128, 128, (kq, nq2), dtype=torch.int8, device=dev)
    qc = torch.empty(mq, nq2, dtype=torch.float64, device=dev)
    qpa, qpb = pn.core.QuantParamsC(), pn.core.QuantParamsC()
    qpa.scale, qpa.zero_point, qpb.scale, qpb.zero_point = 0.02, -3, 0.5, 5
    torch.cuda.synchronize()
    timeit("quantized_matmul int8 4096^3 -> f64 (device pointers)",
           lambda: _lib.quantized_matmul(qa.data_ptr(), qb.data_ptr(), qc.data_ptr(), mq, kq, nq2, ctypes.byref(qpa),
                                         ctypes.byref(qpb)), mq * kq + kq * nq2 + 8 * mq * nq2, reps=5,
           int8_ops=2 * mq * kq * nq2)
    del qa, qb, qc
    # cfg5 AdamW + scan
    na = 100_000_000
    p = torch.randn(na, device=dev) * 0.02
    gr = torch.randn(na, device=dev) * 1e-3
    tp, tg = W(p), W(gr)
    torch.cuda.synchronize()
    opt = pn.AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01)
    timeit("adamw f32 params, f64 m/v, 100M", lambda: opt.step([tp], [tg]), 44 * na, elems=na)
    hn, hi, ss = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
    timeit("nan/inf/l2 scan f32 100M (result on the host)",
           lambda: _lib.neural_tensor_scan(tg._ptr, ctypes.byref(hn), ctypes.byref(hi), ctypes.byref(ss)), 4 * na, elems=na)
    # per-feature transforms on [1M, 64] f64 (512 MB), device pointers
    tb_rows, tb_f = 1 << 20, 64
    tdat = torch.randn(tb_rows, tb_f, device=dev, dtype=torch.float64) * 3 + 1
    tout = torch.empty_like(tdat)
    tstat = [torch.empty(tb_f, device=dev, dtype=torch.float64) for _ in range(4)]
    torch.cuda.synchronize()
    timeit("transform_compute_stats f64 [1M,64] (mean/std/min/max)",
           lambda: _lib.transform_compute_stats(tdat.data_ptr(), tb_rows, tb_f, *[s.data_ptr() for s in tstat]), 8 * tdat.numel(), elems=tdat.numel())
    timeit("transform_normalize f64 [1M,64]",
           lambda: _lib.transform_normalize(tdat.data_ptr(), tout.data_ptr(), tb_rows, tb_f, tstat[0].data_ptr(),
                                            tstat[1].data_ptr(), ctypes.c_double(1e-8)), 16 * tdat.numel(), elems=tdat.numel())
    del tdat, tout
    # gradient clipping over the same 100M gradients (no host readback).  A
    # negative max_norm clips on every call (scale -|max|/norm, magnitudes kept).
    glist = (ctypes.c_void_p * 1)(tg._ptr)
    norm0 = float(ss.value) ** 0.5
    timeit("clip_grad_norm f32 100M, clipping (sumsq + scale)",
           lambda: _lib.neural_clip_grad_norm_list(glist, 1, ctypes.c_double(-norm0), None), 12 * na, elems=na)
    timeit("clip_grad_norm f32 100M, below threshold (sumsq only)",
           lambda: _lib.neural_clip_grad_norm_list(glist, 1, ctypes.c_double(1e300), None), 4 * na, elems=na)
    timeit("clip_grad_value f32 100M",
           lambda: _lib.neural_clip_grad_value_list(glist, 1, ctypes.c_double(-1e-3), ctypes.c_double(1e-3)), 8 * na, elems=na)
    return out


if __name__ == "__main__":
    main()
