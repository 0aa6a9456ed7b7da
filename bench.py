"""Benchmark: int8 YOLOv8n-cls integer-only inference, batch 64, one MI355X.

One step = one integer-only inference pass over a batch of 64 224x224 images
already resident in HBM: input quantization, 26 fused conv kernels (int8
MFMA, bias + requantize + SiLU table + residual Add in the epilogue), C2f
concatenations, GlobalAveragePool, the 1280->1000 Gemm, the Softmax float
fallback and output dequantization, replayed as one captured HIP graph.
By default two batches are in flight (``--in-flight``): two executors, each
with its own input, buffers and full pass, captured as two parallel branches
of one graph, so one replay runs two steps and the GPU overlaps one batch's
launches with the other's launch gaps and idle CUs; K steps are K / 2 such
replays. ``single_batch`` in the line is the same K steps one pass a replay.
Weights are random from a seed (2.72 M parameters); the model is calibrated
on 32 seeded N(0,1) images; inputs are seeded N(0,1) images (synthetic data).

Before timing, the run passes a correctness gate: the logits (pre-Softmax)
of the first images must equal, bit for bit, the reference kernels' result
on the CPU (oracle pipeline over the compiled reference library, same graph
and q.json), and the Softmax output must agree within one step.

The JSON line also carries
* ``roofline`` for the kernel with the largest average duration, timed with
  HIP events on the launch stream;
* ``kernels``: the standalone fused qGEMM (M=4096 K=576 N=64) and qconv
  (b32 64->64 3x3 56x56) launches with their int8 TOPS vs MFMA peak;
* ``cpu_baseline``: the same pass on the host's physical cores with the
  reference's own compiled kernels (OpenMP, threads bound to cores), the
  median of ten timed passes after three untimed ones; ``cpu_baselines``
  adds the standalone GEMM and conv at the ABI level, the int16 and ViT-S
  passes on samples, and single-thread rows;
* the standalone requantize and SiLU-table kernels over the conv's 6.42 M
  outputs, in HBM GB/s;
* ``h2d_d2h``: the same pass with the float batch copied in from pinned
  host memory and the float outputs copied back inside every step, serial
  and with the next batch's copy overlapping the current pass (reported
  beside ``value``, which is the device-resident rate).

Tile codes of the convolutions come from the committed
``profiles/yolov8n_cls_b64_int8_tiles.json`` (the set the committed counter
profile measured) unless ``--retune`` times them again.
"""

import argparse
import json
import os
import sys
import time

# CPU baseline threads: bound to the physical cores (read by the OpenMP
# runtime when it starts, so set before anything loads it)
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

import numpy as np  # noqa: E402

PEAK_I8_TOPS = 5000.0  # MI355X dense int8 MFMA, TOP/s
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, GB/s
ROOT = os.path.dirname(os.path.abspath(__file__))
TILES = os.path.join(ROOT, "profiles", "yolov8n_cls_b64_int8_tiles.json")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--batch", type=int, default=64)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--profile-only", action="store_true",
                   help="skip the CPU baseline and the correctness gate")
    p.add_argument("--eager", action="store_true",
                   help="time eager launches instead of graph replays (for "
                        "per-dispatch counter collection)")
    p.add_argument("--no-tune", action="store_true",
                   help="keep the library's own conv tiling (no plan-time "
                        "timing of the tile variants)")
    p.add_argument("--tiles", metavar="JSON", default=TILES,
                   help="fixed tile codes instead of timing them: a bench "
                        "line's \"tiles\" object, or that object alone "
                        "(default: the committed set, when present)")
    p.add_argument("--retune", action="store_true",
                   help="time the tile variants of every convolution "
                        "instead of using the committed set (alone, then "
                        "with the batches in flight)")
    p.add_argument("--no-extra", action="store_true",
                   help="skip the ViT-S and int16 YOLOv8n-cls passes")
    p.add_argument("--only", choices=("vit", "int16", "gemm", "kernels"),
                   help="time only that pass (ViT-S/16 int8 b32, "
                        "YOLOv8n-cls int16, the ViT-S weight GEMMs, or the "
                        "standalone GEMM / conv / requantize / table "
                        "kernels) and print its records, e.g. under a "
                        "profiler")
    p.add_argument("--in-flight", type=int, default=2, metavar="N",
                   help="batches in flight: N executors (own inputs and "
                        "buffers) as parallel branches of one HIP graph; "
                        "1: one pass a replay")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="finish with one device copy of MIB MiB (a plain "
                        "copy kernel that calibrates byte counters)")
    return p.parse_args()


def layer_work(layer, x_shape, in_bytes=1):
    """Algorithmic ops and HBM bytes of one fused conv launch (int8; the
    input is float32, ``in_bytes`` 4, when its quantization is fused in)."""
    if layer.kind == "conv":
        n, cin, h, w = x_shape
        cout, cg, kh, kw = layer.w_centered.shape
        strides, pads, dil, _ = layer.geometry(x_shape)
        oh = (h + pads[0] + pads[2] - dil[0] * (kh - 1) - 1) // strides[0] + 1
        ow = (w + pads[1] + pads[3] - dil[1] * (kw - 1) - 1) // strides[1] + 1
        ops = 2 * n * cout * oh * ow * cg * kh * kw
        byts = n * cin * h * w * in_bytes + cout * cg * kh * kw + \
            n * cout * oh * ow
    else:
        m = int(np.prod(x_shape[:-1]))
        k, ncol = layer.w_centered.shape
        ops = 2 * m * k * ncol
        byts = m * k + k * ncol + m * ncol
    return ops, byts


def time_launch(fn, reps, torch, per_graph=20):
    """Average duration (ms) of one launch of `fn`: ``per_graph`` launches
    captured back to back in one HIP graph, replayed so that about ``reps``
    launches run, timed with HIP events on the stream the graph replays on
    (Python's own launch cost, several microseconds a call, would otherwise
    be timed for kernels shorter than it)."""
    fn(torch.cuda.current_stream().cuda_stream)  # warm-up, outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream().cuda_stream
        for _ in range(per_graph):
            fn(s)
    g.replay()
    torch.cuda.synchronize()
    n = max(1, reps // per_graph)
    e0, e1 = torch.cuda.Event(enable_timing=True), \
        torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        g.replay()
    e1.record()
    e1.synchronize()
    del g
    return e0.elapsed_time(e1) / (n * per_graph)


def roofline(ops, byts, ms):
    ai = ops / byts
    if ai >= PEAK_I8_TOPS * 1e12 / (PEAK_HBM_GBS * 1e9):
        ach = ops / (ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(ach, 2),
                "peak": PEAK_I8_TOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_I8_TOPS, 4), "traffic": None}
    ach = byts / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4),
            "traffic": None}


def pcie_inclusive(ex, x, steps, torch):
    """Images/s with the float batch copied from pinned host memory and the
    float outputs copied back to pinned host memory inside every step
    (the device-resident rate excludes both). ``serial``: copy in, pass,
    copy out, one after the other on one stream. ``overlapped``: the next
    batch's host-to-device copy runs on a second stream into one of two
    staging buffers while the current pass runs; a device copy moves it
    into the captured graph's input before its pass."""
    inp = ex.inputs_f32["images"]
    outs = list(ex.outputs_f32.values())
    host_in = torch.empty(x.shape, dtype=torch.float32, pin_memory=True)
    host_in.copy_(torch.from_numpy(np.ascontiguousarray(x, np.float32)))
    host_out = [torch.empty(o.shape, dtype=o.dtype, pin_memory=True)
                for o in outs]
    main = torch.cuda.current_stream()

    def serial_step():
        inp.copy_(host_in, non_blocking=True)
        ex.replay()
        for o, h in zip(outs, host_out):
            h.copy_(o, non_blocking=True)

    stage = [torch.empty_like(inp) for _ in range(2)]
    copier = torch.cuda.Stream()  # default priority
    ready = [torch.cuda.Event() for _ in range(2)]
    free = [torch.cuda.Event() for _ in range(2)]

    def upload(i):
        with torch.cuda.stream(copier):
            copier.wait_event(free[i % 2])  # its last reader has copied it
            stage[i % 2].copy_(host_in, non_blocking=True)
            ready[i % 2].record(copier)

    def overlapped(n):
        upload(0)
        for i in range(n):
            main.wait_event(ready[i % 2])
            inp.copy_(stage[i % 2], non_blocking=True)
            free[i % 2].record(main)
            if i + 1 < n:
                upload(i + 1)
            ex.replay()
            for o, h in zip(outs, host_out):
                h.copy_(o, non_blocking=True)

    rec = {"h2d_bytes_per_step": int(inp.numel() * inp.element_size()),
           "d2h_bytes_per_step": int(sum(o.numel() * o.element_size()
                                         for o in outs)),
           "steps": steps}
    for label, run in (("serial", lambda n: [serial_step()
                                            for _ in range(n)]),
                       ("overlapped", overlapped)):
        run(3)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run(steps)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        rec[label] = {"images_per_s": round(x.shape[0] / dt, 1),
                      "ms_per_step": round(dt * 1e3, 4)}
    return rec


def in_flight(c, ex, x, out_name, nf, torch):
    """``nf`` batches in flight: ``ex`` and nf - 1 more executors of
    container ``c`` (own buffers, ``ex``'s tiles), batch k holding ``x``
    rolled by k B / nf images, as one graph of parallel branches
    (``executor.InFlight``). Returns it and whether every extra batch's
    output ``out_name`` equals ``ex``'s (which holds its pass over ``x``),
    rolled the same way, bit for bit."""
    from quantanything_amd.executor import DeviceExecutor, InFlight

    B = x.shape[0]
    exs = [ex]
    first = ex.tensors[out_name].to_host()
    same = True
    for k in range(1, nf):
        shift = k * B // nf
        e = DeviceExecutor(c, {"images": x.shape})
        e.inputs_f32["images"].copy_(
            torch.from_numpy(np.ascontiguousarray(np.roll(x, shift, 0))))
        for (n0, d0, _, _), (n1, d1, _, _) in zip(ex.tunables, e.tunables):
            if n0 != n1:
                raise RuntimeError("executors planned differently")
            d1.tile = d0.tile
        e.launch()
        torch.cuda.synchronize()
        same &= bool(np.array_equal(e.tensors[out_name].to_host(),
                                    np.roll(first, shift, 0)))
        exs.append(e)
    return InFlight(exs), same


def measure_pass(name, g, quant_type, batch, steps, tune, torch, nf=1):
    """Images/s of one captured integer pass of graph ``g`` (calibrated on
    32 seeded N(0, 1) images, tiles tuned as for the headline pass)."""
    from quantanything_amd.container import QuantContainer
    from quantanything_amd.synth import Stream

    c = QuantContainer(g, quant_type, per_channel=True)
    calib = Stream(4).normal((32, 3, 224, 224)).astype(np.float32)
    c.calibrate([calib[:batch] if batch < 32 else calib])
    x = Stream(5).normal((batch, 3, 224, 224)).astype(np.float32)
    ex = c.executor({"images": x.shape})
    ex.inputs_f32["images"].copy_(torch.from_numpy(x))
    ex.launch()
    torch.cuda.synchronize()
    if tune:
        ex.tune()
    ex.launch()
    torch.cuda.synchronize()
    ex.capture()

    def timed(step, k):
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(k):
            step()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    dt = timed(ex.replay, steps) / steps
    rec = {"workload": name, "quant_type": quant_type, "global_batch": batch,
           "images_per_s": round(batch / dt, 1),
           "ms_per_step": round(dt * 1e3, 4), "steps": steps,
           "launches_per_step": len(ex.launches),
           "params": g.num_params()}
    if nf > 1:  # the same steps with nf batches in flight
        fl, same = in_flight(c, ex, x, g.outputs[0], nf, torch)
        reps = max(1, steps // nf)
        dtf = timed(fl.replay, reps) / (reps * nf)
        rec["in_flight"] = {"batches": nf, "outputs_equal": same,
                            "images_per_s": round(batch / dtf, 1),
                            "ms_per_step": round(dtf * 1e3, 4)}
    return rec, c


def kernel_rows(tune, torch, steps=50):
    """The standalone GEMM + requantize and conv + requantize + SiLU table
    workloads (int8 TOPS) and the element-wise requantize / table kernels
    (HBM GB/s), each timed over ``steps`` launches."""
    from quantanything_amd.workloads import (
        ConvWorkload,
        GemmWorkload,
        LutWorkload,
        RequantizeWorkload,
    )

    kernels = []
    for wl in (GemmWorkload(), ConvWorkload()):
        code = 0
        if tune:  # the same plan-time tile timing as the pass
            from quantanything_amd.executor import DeviceExecutor

            wl.launch()
            times = {}
            for _ in range(2):  # two rounds: the first also warms clocks
                for c_ in DeviceExecutor.tile_candidates(wl.d):
                    wl.d.tile = c_
                    t = time_launch(wl.launch, 40, torch)
                    times[c_] = min(times.get(c_, t), t)
            code = min(times, key=times.get)
            wl.d.tile = code
        kms = time_launch(wl.launch, steps, torch)
        r = roofline(wl.ops, wl.bytes, kms)
        tops = wl.ops / (kms * 1e-3) / 1e12
        kernels.append({"workload": wl.name, "tile": hex(code),
                        "avg_ms": round(kms, 5),
                        "int8_tops": round(tops, 2),
                        "frac_of_mfma_peak": round(tops / PEAK_I8_TOPS, 4),
                        "roofline": r})

    for wl in (RequantizeWorkload(), LutWorkload()):
        kms = time_launch(wl.launch, steps, torch)
        gbs = wl.bytes / (kms * 1e-3) / 1e9
        kernels.append({"workload": wl.name, "avg_ms": round(kms, 5),
                        "bytes_per_launch": wl.bytes,
                        "roofline": {"bound": "hbm", "achieved": round(gbs, 1),
                                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                     "frac": round(gbs / PEAK_HBM_GBS, 4),
                                     "traffic": None}})
    return kernels


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): this "
              "build measures the single-GPU path; the multi-GPU sharding is "
              "a design note.", file=sys.stderr)
        return 2
    if not (args.no_cpu or args.profile_only):
        from oracle import cpu_baseline

        # counted before an OpenMP runtime pins this thread to one core
        cpu_baseline.physical_cores()
    import torch

    from quantanything_amd import graph as G
    from quantanything_amd import native
    from quantanything_amd.container import QuantContainer
    from quantanything_amd.synth import Stream
    from quantanything_amd import synth
    from quantanything_amd.workloads import GemmWorkload

    native.require()
    B = args.batch
    if args.only == "kernels":  # the standalone kernel workloads alone
        for row in kernel_rows(not args.no_tune, torch, args.steps):
            print(json.dumps(row), flush=True)
        return 0
    if args.only == "gemm":  # the weight GEMM shapes of a ViT-S block
        from quantanything_amd.workloads import vit_gemm_shapes

        for name, m, k, n in vit_gemm_shapes():
            wl = GemmWorkload(seed=7, M=m, K=k, N=n)
            kms = time_launch(wl.launch, args.steps, torch)
            tops = wl.ops / (kms * 1e-3) / 1e12
            print(json.dumps({"workload": f"vit {name} {m}x{k}x{n}",
                              "tile": hex(wl.d.tile), "avg_ms": round(kms, 5),
                              "int8_tops": round(tops, 1),
                              "frac_of_mfma_peak": round(tops / PEAK_I8_TOPS,
                                                         4)}), flush=True)
        return 0
    if args.only:
        if args.only == "vit":
            rec, _ = measure_pass("ViT-S/16 (12 blocks, 197 tokens) int8",
                                  G.vit(seed=5, batch=32), "int8", 32,
                                  args.steps, not args.no_tune, torch,
                                  max(1, args.in_flight))
        else:
            rec, _ = measure_pass("YOLOv8n-cls int16 (wide accumulation)",
                                  G.yolov8n_cls(seed=3), "int16", B,
                                  args.steps, not args.no_tune, torch)
        print(json.dumps(rec))
        return 0
    g = G.yolov8n_cls(seed=3)
    c = QuantContainer(g, "int8", per_channel=True)
    calib = Stream(4).normal((32, 3, 224, 224)).astype(np.float32)
    QuantContainer(g, "int8", per_channel=True).calibrate([calib[:2]])
    t0 = time.perf_counter()
    c.calibrate([calib])  # float pass (GPU conv / GEMM), ranges, parameters
    calib_s = time.perf_counter() - t0
    x = Stream(5).normal((B, 3, 224, 224)).astype(np.float32)
    ex = c.executor({"images": x.shape})
    ex.inputs_f32["images"].copy_(torch.from_numpy(x))
    ex.launch()
    torch.cuda.synchronize()
    tiles = {}
    if args.retune:
        args.tiles = None
    if args.tiles and os.path.exists(args.tiles):  # a recorded choice
        with open(args.tiles) as f:
            fixed = json.load(f)
        fixed = fixed.get("tiles", fixed)
        for name, d, codes, _ in ex.tunables:
            if name in fixed:
                d.tile = int(fixed[name][0], 16)
                tiles[name] = (d.tile, float("nan"), float("nan"))
        ex.launch()
        torch.cuda.synchronize()
    elif not args.no_tune:  # plan time: per-layer tile variants, fastest kept
        tiles = ex.tune()
        ex.launch()
        torch.cuda.synchronize()

    # ---- correctness gate + CPU baseline (reference kernels on the host) --
    cpu = None
    cpu_rows = []
    gate = None
    qdir = None
    if not args.profile_only:
        import tempfile

        from oracle import cpu_baseline
        from oracle.pipeline import OraclePipeline

        cores = cpu_baseline.physical_cores()
        soft = g.nodes[-1]
        logits_name = soft.inputs[0]
        qdir = tempfile.TemporaryDirectory()
        qpath = os.path.join(qdir.name, "q.json")
        c.save(qpath)
        lib_kind = "ref" if cpu_baseline.abi.ref_available() else "oracle"
        cpu_baseline.abi.load(lib_kind).set_num_threads(cores)
        gl = G.yolov8n_cls(seed=3, softmax=False)
        n_gate = min(4, B)
        ints, _ = OraclePipeline(gl, qpath, lib=lib_kind).run(x[:n_gate])
        dev_logits = ex.tensors[logits_name].to_host()[:n_gate]
        exact = bool(np.array_equal(dev_logits, ints[gl.outputs[0]]))
        ref_out, _ = OraclePipeline(g, qpath, lib=lib_kind).run(x)
        dev_out = ex.tensors[g.outputs[0]].to_host()
        soft_diff = int(np.abs(dev_out.astype(np.int64)
                               - ref_out[g.outputs[0]]).max())
        gate = {"logits_bit_exact": exact, "images_checked": n_gate,
                "softmax_max_step_diff": soft_diff}
        if not exact or soft_diff > 1:
            print(json.dumps({"error": "correctness gate failed",
                              "gate": gate}))
            return 1
        if not args.no_cpu:
            name = f"YOLOv8n-cls int8 b{B} (integer pass)"
            head = cpu_baseline.pipeline_rows(name, g, qpath, x, [cores])[0]
            cpu = {k: head[k] for k in ("value", "unit", "cores", "kind")}
            cpu["sample"] = (f"{head['runs']} timed passes over the batch-{B} "
                             "input after 3 untimed, median; the reference's "
                             "compiled kernels, OpenMP threads bound to the "
                             "physical cores")
            cpu_rows.append(head)
            cpu_rows += cpu_baseline.pipeline_rows(
                "YOLOv8n-cls int8 (integer pass)", g, qpath, x[:4], [1])
            cpu_rows += cpu_baseline.gemm_rows(synth.gemm_workload(),
                                               [cores, 1])
            cpu_rows += cpu_baseline.conv_rows(synth.conv_workload(),
                                               [cores, 1])

    # ---- further batches in flight: their own executors, inputs and
    # buffers; each must give the first one's outputs for the same images
    nf = 1 if args.eager else max(1, args.in_flight)
    flight = None
    if nf > 1:
        flight, same = in_flight(c, ex, x, g.outputs[0], nf, torch)
        if args.retune:  # the codes again, with the batches in flight
            from quantanything_amd.executor import InFlight, tune_in_flight

            # the launch slowest alone keeps its fastest code alone (the
            # roofline kernel)
            slowest = max(tiles, key=lambda n: tiles[n][1]) if tiles else None
            chosen = tune_in_flight(flight.executors,
                                    keep=() if slowest is None else (slowest,))
            for n, code in chosen.items():
                if n in tiles and code != tiles[n][0]:
                    tiles[n] = (code, float("nan"), tiles[n][2])
            ex.launch()
            torch.cuda.synchronize()
            flight = InFlight(flight.executors)
        if gate is not None:
            gate["in_flight_batches_equal"] = same
        if not same:
            print(json.dumps({"error": "a batch in flight differs from the "
                                       "first executor's pass"}))
            return 1

    # ---- timed region: captured graph replays ----------------------------
    step = ex.launch if args.eager else ex.replay
    if not args.eager:
        ex.capture()

    def timed(inflight):
        if inflight is None:
            for _ in range(args.warmup):
                step()
        else:
            for _ in range(max(1, args.warmup // nf)):
                inflight.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if inflight is None:
            for _ in range(args.steps):
                step()
        else:  # K steps: K // N replays of N batches, the rest one by one
            reps, rest = divmod(args.steps, nf)
            for _ in range(reps):
                inflight.replay()
            for _ in range(rest):
                step()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    dt = timed(flight)
    ms = dt * 1e3 / args.steps
    value = B * args.steps / dt
    single = None
    if flight is not None:
        dt1 = timed(None)
        single = {"images_per_s": round(B * args.steps / dt1, 1),
                  "ms_per_step": round(dt1 * 1e3 / args.steps, 4)}
    # the same pass with its float input and output crossing PCIe
    pcie = None if args.eager else pcie_inclusive(
        ex, x, max(5, min(args.steps, 50)), torch)

    # ---- per-launch durations (HIP events on the launch stream) ----------
    per = []
    shapes = {"images": x.shape}
    for name, t in ex.tensors.items():
        shapes[name] = t.shape
    for name, fn in ex.launches:
        per.append((time_launch(fn, 40, torch), name, fn))
    layers = {l.name: l for l in c.layers}
    # a conv's fused residual Add reads, and its Concat copy writes, one
    # more output-sized tensor
    descs = {ln[5:]: d for d, _, _, ln in ex.mfma_descs}

    def fused_io(lname, out_shape):
        d = descs.get(lname)
        if d is None:
            return 0
        return int(np.prod(out_shape)) * ((1 if d.res else 0) +
                                          (1 if d.y2 else 0))

    def conv_out_shape(layer, xs):
        n, _, h, w = xs
        cout, _, kh, kw = layer.w_centered.shape
        strides, pads, dil, _ = layer.geometry(xs)
        return (n, cout,
                (h + pads[0] + pads[2] - dil[0] * (kh - 1) - 1) // strides[0]
                + 1,
                (w + pads[1] + pads[3] - dil[1] * (kw - 1) - 1) // strides[1]
                + 1)

    def work(name):
        """(layer, ops, bytes) of a conv launch ("qconv:": float input;
        "pair:" / "chain:": two convs, the intermediate not in HBM;
        "pairtail:": a pair and the 1x1 conv reading the Concat it ends,
        whose last channels come from LDS)."""
        kind, _, lname = name.partition(":")
        if kind == "pairtail":
            a, b, t = lname.split("+")
            if a not in layers or b not in layers or t not in layers:
                return None
            la, lb, lt = layers[a], layers[b], layers[t]
            xs = shapes[la.data_inputs[0]]
            mid = conv_out_shape(la, xs)
            oa, ba = layer_work(la, xs)
            ob, bb = layer_work(lb, mid)
            ot, bt = layer_work(lt, shapes[lt.data_inputs[0]])
            return (lt, oa + ob + ot,
                    ba + bb + bt - 3 * int(np.prod(mid)) + fused_io(b, mid))
        if kind in ("pair", "chain"):
            a, _, b = lname.partition("+")
            if a not in layers or b not in layers:
                return None
            la, lb = layers[a], layers[b]
            xs = shapes[la.data_inputs[0]]
            mid = conv_out_shape(la, xs)
            oa, ba = layer_work(la, xs)
            ob, bb = layer_work(lb, mid)
            return lb, oa + ob, (ba + bb - 2 * int(np.prod(mid)) +
                                 fused_io(b, conv_out_shape(lb, mid)))
        if kind not in ("conv", "qconv", "convpool") or lname not in layers:
            return None
        layer = layers[lname]
        xs = shapes[layer.data_inputs[0]]
        ops, byts = layer_work(layer, xs, 4 if kind == "qconv" else 1)
        if kind == "convpool":  # the pooled output replaces the conv output
            cout = layer.w_centered.shape[0]
            byts -= ops // (2 * layer.w_centered[0].size) - xs[0] * cout
        elif layer.kind == "conv":
            byts += fused_io(lname, conv_out_shape(layer, xs))
        return layer, ops, byts

    in_order = []
    for t, n, _ in per:
        row = [n, round(t, 5)]
        w = work(n)
        if w is not None:  # algorithmic ops and bytes of a fused conv launch
            row += [w[1], w[2]]
        in_order.append(row)
    per.sort(reverse=True, key=lambda r: r[0])
    top_ms, top_name, _ = per[0]
    w = work(top_name)
    if w is not None:
        top, ops, byts = w
        roof = roofline(ops, byts, top_ms)
        roof["kernel"] = (f"fused conv {top_name.partition(':')[2]} (int8 "
                          "MFMA" + (", float input quantized in" if
                                    top_name.startswith("qconv:") else "")
                          + ")")
        roof["ops_per_launch"] = ops
        roof["bytes_per_launch"] = byts
    else:
        roof = {"bound": "hbm", "achieved": None, "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": None, "traffic": None,
                "kernel": top_name}
    roof["avg_ms"] = round(top_ms, 5)
    # HBM bytes of that launch from the committed counter profile (rocprofv3
    # FETCH_SIZE + WRITE_SIZE, calibrated on a copy kernel), when it has it
    prof = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "yolov8n_cls_b64_int8_traffic.json")
    if os.path.exists(prof):
        with open(prof) as f:
            measured = json.load(f).get("traffic", {})
        if top_name in measured:
            roof["traffic"] = measured[top_name]

    kernels = kernel_rows(not args.no_tune, torch)

    # ---- the other end-to-end configurations (parity: tests/) ------------
    extra = []
    if not args.no_extra and not args.profile_only:
        steps = max(5, min(args.steps, 50))
        rec, cv = measure_pass("ViT-S/16 (12 blocks, 197 tokens) int8",
                               G.vit(seed=5, batch=32), "int8", 32, steps,
                               not args.no_tune, torch, nf)
        extra.append(rec)
        rec, c16 = measure_pass("YOLOv8n-cls int16 (wide accumulation)",
                                G.yolov8n_cls(seed=3), "int16", B, steps,
                                not args.no_tune, torch)
        extra.append(rec)
        if qdir is not None and not args.no_cpu:
            from oracle import cpu_baseline

            cores = cpu_baseline.physical_cores()
            p16 = os.path.join(qdir.name, "q16.json")
            c16.save(p16)
            cpu_rows += cpu_baseline.pipeline_rows(
                "YOLOv8n-cls int16 (integer pass, int64 accumulation)", g,
                p16, x[:8], [cores])
            pv = os.path.join(qdir.name, "qvit.json")
            cv.save(pv)
            xv = Stream(5).normal((2, 3, 224, 224)).astype(np.float32)
            cpu_rows += cpu_baseline.pipeline_rows(
                "ViT-S/16 int8 (integer pass, float fallbacks)",
                G.vit(seed=5, batch=2), pv, xv, [cores])

    line = {
        "metric": "int8 YOLOv8n-cls images/s (b=64) + qGEMM TOPS as % of "
                  "i8 MFMA peak",
        "value": round(value, 1),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) images, random-init weights)",
        "config": {"workload": "YOLOv8n-cls int8 integer-only inference",
                   "global_batch": B, "image": 224, "quant_type": "int8",
                   "per_channel": True, "params": g.num_params(),
                   "parallelism": "single GPU", "batches_in_flight": nf},
        "single_batch": single,
        "roofline": roof,
        "cpu_baseline": cpu,
        "cpu_baselines": cpu_rows,
        "kernels": kernels,
        "other_configs": extra,
        "gate": gate,
        "h2d_d2h": pcie,
        "calibration_s": round(calib_s, 3),
        "launches_per_step": len(ex.launches),
        "top_launches_ms": [[n, round(t, 5)] for t, n, _ in per[:6]],
        "launches_ms": in_order,
        "tiles": {n: [hex(code), None if best != best else round(best, 5),
                      None if lib != lib else round(lib, 5)]
                  for n, (code, best, lib) in tiles.items()},
    }
    if args.copy_probe > 0:
        src = torch.empty(args.copy_probe << 20, dtype=torch.uint8,
                          device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
