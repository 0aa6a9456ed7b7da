"""Host-CPU baselines for the benchmark (test infrastructure: only the
benchmark's CPU-baseline leg uses this module).

Every row times the reference's own compiled kernels (``_ref/libqa_ref.so``,
OpenMP) when they were built, else the C restatement, on the host's
physical cores (counted from ``lscpu``; threads bound with
``OMP_PROC_BIND=close`` and ``OMP_PLACES=cores``, which the caller sets
before the OpenMP runtime starts) and on one thread. Each figure is the
median of at least ten timed runs after three untimed ones. The work is the
call sequence the reference makes (``quant_layers.py:320-341``,
``:384-402``, ``:470-472``): int32 activations centred by the zero point, the
integer conv / GEMM, a separate requantize, then the lookup table; whole
passes run the oracle pipeline over the same kernels."""

import os
import statistics
import subprocess
import time

import numpy as np

from oracle import abi
from oracle.pipeline import OraclePipeline

WARMUP, RUNS = 3, 10


_CORES = []


def physical_cores():
    """Distinct (core, socket) pairs that ``lscpu -p`` lists, limited to the
    CPUs this process may run on. Counted once: call it before the OpenMP
    runtime starts, since binding pins the calling thread to one CPU and
    narrows its affinity mask."""
    if not _CORES:
        _CORES.append(_count_cores())
    return _CORES[0]


def _count_cores():
    allowed = os.sched_getaffinity(0)
    try:
        out = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"],
                             capture_output=True, text=True, check=True)
        cores = set()
        for line in out.stdout.splitlines():
            if line.startswith("#") or not line.strip():
                continue
            cpu, core, sock = (int(v) for v in line.split(",")[:3])
            if cpu in allowed:
                cores.add((core, sock))
        if cores:
            return len(cores)
    except (OSError, ValueError, subprocess.CalledProcessError):
        pass
    return len(allowed)


def median_time(fn, runs=RUNS, warmup=WARMUP):
    """``(median seconds, runs)`` of ``fn()`` after ``warmup`` calls."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), runs


def _library():
    kind = "reference" if abi.ref_available() else "port"
    return abi.load("ref" if kind == "reference" else "oracle"), kind


def _row(workload, value, unit, threads, kind, sample, med, runs):
    return {"workload": workload, "value": round(value, 3), "unit": unit,
            "cores": threads, "kind": kind, "sample": sample,
            "median_s": round(med, 6), "runs": runs,
            "warmup": WARMUP}


def gemm_rows(spec, thread_counts):
    """The standalone GEMM + requantize at the ABI level (GOP/s)."""
    lib, kind = _library()
    a = (spec["a"].astype(np.int32) - spec["zp_in"]).astype(np.int16)
    w = spec["w"].astype(np.int16)
    m, k, n = spec["M"], spec["K"], spec["N"]
    ops = 2 * m * n * k

    def run():
        acc = lib.gemm_int(a, w, False)
        lib.requantize(acc, m, n, 1, spec["mult"], spec["shift"],
                       spec["zp_out"], spec["qmin"], spec["qmax"],
                       pre_bias=spec["bias"])

    rows = []
    for t in thread_counts:
        lib.set_num_threads(t)
        med, runs = median_time(run)
        rows.append(_row(f"qgemm M={m} K={k} N={n} + requantize (ABI)",
                         ops / med / 1e9, "GOP/s", t, kind,
                         "the full shape, int16 x int16 -> int32 then "
                         "qa_requantize_i32", med, runs))
    return rows


def conv_rows(spec, thread_counts):
    """The standalone conv + requantize + table at the ABI level (GOP/s)."""
    lib, kind = _library()
    x = spec["x"].astype(np.int32) - spec["zp_in"]
    w = spec["w"].astype(np.int32)
    n, cin, h, wd = x.shape
    cout, _, kh, kw = w.shape
    p, s = spec["pad"], spec["stride"]
    oh = (h + 2 * p - kh) // s + 1
    ow = (wd + 2 * p - kw) // s + 1
    ops = 2 * n * cout * oh * ow * cin * kh * kw

    def run():
        acc = lib.conv2d_int(x, w, (s, s), (p, p, p, p), (1, 1), 1, wide=False)
        rq = lib.requantize(acc, n, cout, oh * ow, spec["mult"],
                            spec["shift"], spec["zp_out"], spec["qmin"],
                            spec["qmax"], pre_bias=spec["bias"])
        lib.lut(rq, spec["lut"], spec["lut_offset"])

    rows = []
    for t in thread_counts:
        lib.set_num_threads(t)
        med, runs = median_time(run)
        rows.append(_row(
            f"qconv b{n} {cin}->{cout} {kh}x{kw} {h}x{wd} + requantize + "
            "SiLU table (ABI)", ops / med / 1e9, "GOP/s", t, kind,
            "the full shape: qa_conv_i32_i16_i32, qa_requantize_i32, qa_lut",
            med, runs))
    return rows


def pipeline_rows(name, graph, qjson, x, thread_counts):
    """A whole integer pass of ``graph`` over the batch ``x`` (images/s)."""
    lib, kind = _library()
    pipe = OraclePipeline(graph, qjson, lib="ref" if kind == "reference"
                          else "oracle")
    rows = []
    for t in thread_counts:
        lib.set_num_threads(t)
        med, runs = median_time(lambda: pipe.run(x))
        rows.append(_row(name, len(x) / med, "images/s", t, kind,
                         f"integer passes over {len(x)} image(s)", med,
                         runs))
    return rows
