"""Benchmark of the MI355X matmul / attention dispatch path.

Default run (the driver's contract): one JSON line for BASELINE.json's metric
on configs[1], the int8 x int8 -> i32 matmul M=N=K=4096 (A row-major, B
column-major), one step = one dispatch over inputs resident in HBM. The line
also carries the other two figures the metric names (fp16 4096^3 TFLOP/s and
M=1 GEMV HBM GB/s), the roofline of the dominant kernel measured with HIP
events on the stream it runs on, and the CPU baseline (the C oracle on the
host cores, labelled "port": IREE is not installable here).

The default line also times C3 M=2048 with row-major weights, C4 attention
and C5 W8A16 (M=1, 512), and measures this box's ceilings with the
calibration kernels: a register-only MFMA loop on random operands (the
`ceiling` next to `peak`) and a pure HBM stream read of the GEMV's bytes.

--suite prints one JSON line per BASELINE config (C1..C5 and the C3 sweep),
each with the C oracle timed beside it on this host.
--only <workload> runs one workload for profiler passes; --only stream and
--only mfma_ceiling print the calibration ceilings alone.
--tune times every compiled MFMA macro-tile on the 4096^3 shapes;
--tune --tune-counters profiles each one under rocprofv3 (SQ counters per
wave: MFMA busy fraction, waits, LDS and VALU instructions).
--tune --tune-skinny sweeps tiles x split counts on the skinny shapes; with
--tune-counters it profiles the planner's pick and the fastest candidates of
each shape under rocprofv3 (SQ counters and HBM bytes).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_I8_TOPS = 5000.0      # dense int8 MFMA, MI355X published
PEAK_F16_TFLOPS = 2500.0   # dense fp16 MFMA, MI355X published
PEAK_HBM_GBS = 8000.0      # HBM3E, MI355X published
ROTATE_BYTES = 600 << 20   # > 2 x 256 MiB Infinity Cache


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # The defaults time the GPU at its sustained clock: on random operands
    # the shader clock settles over the first ~30 ms of MFMA load (measured
    # 1.5 -> 2.0 GHz), so 1000 warmup dispatches (~70 ms) precede the
    # 500 timed ones (~35 ms) of the headline workload.
    p.add_argument("--steps", type=int, default=500)
    p.add_argument("--warmup", type=int, default=1000)
    p.add_argument("--suite", action="store_true")
    p.add_argument("--tune", action="store_true")
    p.add_argument("--tune-skinny", action="store_true",
                   help="with --tune: sweep tiles x split counts on the "
                        "skinny C3 / C5 shapes")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--resources", action="store_true",
                   help="print every compiled kernel's registers, LDS, "
                        "scratch and occupancy (one JSON line each)")
    p.add_argument("--no-graph", action="store_true",
                   help="time eager launches instead of one captured graph")
    p.add_argument("--only", choices=["i8", "f16", "f16nn", "gemv", "attn",
                                      "w8a16", "w8a16_gemm", "w8a16_nk",
                                      "runtime", "stream", "mfma_ceiling",
                                      "config"],
                   help="run one workload (for rocprof passes) and exit")
    p.add_argument("--config", default=None,
                   help="with --only config: the MFMA configuration to run")
    p.add_argument("--shape", default="4096,4096,4096",
                   help="with --only config: M,N,K")
    p.add_argument("--splits", type=int, default=0,
                   help="with --only config: K splits of a split-K tile "
                        "(0: the planner's; -1: stream-K)")
    p.add_argument("--rotate", action="store_true",
                   help="with --only config: rotate copies of B past the "
                        "Infinity Cache, as the skinny sweep does")
    p.add_argument("--tune-counters", action="store_true",
                   help="with --tune: profile every candidate on the 4096^3 "
                        "shapes under rocprofv3 (SQ counters per wave)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="with --only: first copy 256 MiB device-to-device "
                        "once, the known-size reference for FETCH_SIZE / "
                        "WRITE_SIZE counter scaling")
    return p.parse_args()


USE_GRAPH = True
SPIN_CYCLES = 5_000_000  # a few ms of GPU clock


def profiled_traffic(kernel):
    """HBM bytes per launch of `kernel` (a config name) as measured by the
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes summarised under profiles/, or
    None. Each summary holds a line `traffic[<config>] = <bytes> bytes`."""
    import glob
    import re
    pat = re.compile(r"^traffic\[(\S+)\] = (\d+) bytes", re.M)
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        with open(path) as f:
            for name, nbytes in pat.findall(f.read()):
                if name == kernel:
                    return int(nbytes)
    return None


def timed(fn, steps, warmup):
    """Average ms per step of fn() over exactly `steps` steps.

    `warmup` eager steps first (they also size the wrapper's workspace of
    the capture stream, so the timed steps allocate nothing). The `steps`
    launches are then captured into
    one HIP graph (no memset nodes: the kernels re-arm their own counters) and
    replayed once untimed and once between HIP events recorded on the capture
    stream, with a device synchronize on both sides. Without the graph a
    5-microsecond GEMV would measure the Python launch path, not the kernel.
    """
    import torch
    stream = capture_stream()
    # Warm up on the stream the graph is captured on: the library keeps one
    # workspace per stream and never allocates under capture.
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn()
    torch.cuda.synchronize()
    if not USE_GRAPH:
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            start.record(stream)
            for _ in range(steps):
                fn()
            stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(steps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        # A bounded spin first, so the host has submitted the graph before
        # the start event fires: the timed region is the K dispatches, not
        # the host's graph submission.
        torch.cuda._sleep(SPIN_CYCLES)
        start.record(stream)
        graph.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


_CAPTURE_STREAM = None


def capture_stream():
    """The one side stream every timed workload runs and is captured on."""
    import torch
    global _CAPTURE_STREAM
    if _CAPTURE_STREAM is None:
        _CAPTURE_STREAM = torch.cuda.Stream()
    return _CAPTURE_STREAM


_CAL = None


def calibration():
    """The benchmark's ceiling kernels (lib/libiree_mi355x_calibrate.so):
    a pure HBM stream read and a register-only MFMA loop."""
    import ctypes
    global _CAL
    if _CAL is None:
        path = os.path.join(ROOT, "iree-hexagon-plugins_amd", "lib",
                            "libiree_mi355x_calibrate.so")
        if not os.path.exists(path):
            raise ImportError(f"{path} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(path)
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.iree_mi355x_calibrate_stream_read.argtypes = [p, i64, p,
                                                          ctypes.c_int, p]
        lib.iree_mi355x_calibrate_mfma_loop.argtypes = [
            ctypes.c_int, p, ctypes.c_int, p, ctypes.c_int, p]
        _CAL = lib
    return _CAL


def stream_ceiling(dev, nbytes, steps, warmup):
    """GB/s of a pure read of `nbytes`, rotating copies past the 256 MiB
    Infinity Cache; the best over four grid sizes."""
    import torch
    lib = calibration()
    copies = max(2, ROTATE_BYTES // nbytes + 1)
    bufs = [torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,),
                          dtype=torch.int32, device=dev) for _ in range(copies)]
    best = None
    for wgs in (512, 1024, 2048, 4096):
        sink = torch.empty(wgs, dtype=torch.int32, device=dev)
        it = [0]

        def fn():
            st = lib.iree_mi355x_calibrate_stream_read(
                bufs[it[0] % copies].data_ptr(), nbytes, sink.data_ptr(), wgs,
                torch.cuda.current_stream().cuda_stream)
            assert st == 0
            it[0] += 1
        ms = timed(fn, max(steps, 4 * copies), warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        if best is None or gbs > best[0]:
            best = (gbs, wgs, ms)
    del bufs
    return {"gbs": round(best[0], 1), "us": round(best[2] * 1e3, 2),
            "workgroups": best[1], "bytes": nbytes, "rotating_copies": copies}


def mfma_ceiling(dev, kind, random_operands, steps=50, warmup=100,
                 iters=4096, shape=32):
    """Dense TOPS (kind "i8") or TFLOP/s ("f16") of MFMAs on operands held
    in registers (no memory traffic), 256 workgroups of 8 waves: the MFMA
    pipe at the clock the operand data lets the chip hold. `shape` 32:
    the 32x32 MFMAs the GEMM kernels issue; 16: the 16x16 ones."""
    import torch
    lib = calibration()
    g = torch.Generator().manual_seed(5)
    n = 64 * 256 * 16
    per_lane_k = 32 if kind == "i8" else 16  # K of the 32x32 shape
    if kind == "i8":
        src = (torch.randint(-128, 128, (n,), generator=g, dtype=torch.int8)
               if random_operands else torch.ones(n, dtype=torch.int8))
    else:
        src = (torch.randn(n // 2, generator=g).half() if random_operands
               else torch.ones(n // 2, dtype=torch.float16))
    if shape == 32:
        ops_per_mfma = 2 * 32 * 32 * per_lane_k
    else:
        ops_per_mfma = 2 * 16 * 16 * 2 * per_lane_k
        iters *= 2  # half the products per instruction
    src = src.to(dev)
    wgs = 256
    sink = torch.empty(wgs * 512, dtype=torch.int32, device=dev)

    code = (0 if kind == "i8" else 1) + (2 if shape == 16 else 0)

    def fn():
        st = lib.iree_mi355x_calibrate_mfma_loop(
            code, src.data_ptr(), iters, sink.data_ptr(),
            wgs, torch.cuda.current_stream().cuda_stream)
        assert st == 0
    ms = timed(fn, steps, warmup)
    return ops_per_mfma * 4 * iters * wgs * 8 / (ms * 1e-3) / 1e12


def cpu_info():
    """nproc and the CPU model of this host (BASELINE's CPU baseline asks
    for both next to the threads used)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def cpu_threads():
    """Host threads for the CPU baseline: this box's share (OMP_NUM_THREADS,
    16 per GPU here), whatever nproc reports."""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "16")))
    except ValueError:
        return 16


def cpu_time(fn, budget_s=2.0, max_runs=100):
    """Seconds per run of fn() on the host, repeated to about `budget_s`:
    (seconds per run, runs)."""
    runs, t0 = 0, time.perf_counter()
    while runs < max_runs and (runs == 0 or
                               time.perf_counter() - t0 < budget_s):
        fn()
        runs += 1
    return (time.perf_counter() - t0) / runs, runs


def rotating(make, count):
    """`count` independent copies of a device tensor, to rotate through."""
    return [make() for _ in range(count)]


def cpu_baseline_i8(a, bt, threads, budget_s=12.0, max_runs=400):
    """The C oracle on the host cores over the full C2 workload, repeated
    until about `budget_s` of CPU work: (TOPS, runs, seconds)."""
    import oracle
    m, k = a.shape
    n = bt.shape[0]
    runs, t0 = 0, time.perf_counter()
    while runs < max_runs and (runs == 0 or
                               time.perf_counter() - t0 < budget_s):
        oracle.matmul_i8(a, bt, b_transposed=True, threads=threads)
        runs += 1
    dt = time.perf_counter() - t0
    return 2.0 * m * n * k * runs / dt / 1e12, runs, dt


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every GPU box "
                          "here has one, and the path shards without exchange "
                          "(see the design notes); run with --gpus 1"}))
        sys.exit(2)
    import torch
    import __graft_entry__ as entry
    pkg = entry.load_package()
    from importlib import import_module
    inputs = import_module(entry.PKG_NAME + ".inputs")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    global USE_GRAPH
    USE_GRAPH = not args.no_graph
    if args.only:
        return only(pkg, inputs, dev, args)
    if args.tune:
        return tune(pkg, inputs, dev, args)
    if args.suite:
        return suite(pkg, inputs, dev, args)
    if args.resources:
        for rec in pkg.kernel_resources():
            print(json.dumps(rec), flush=True)
        return

    # ---- headline: C2 int8 4096^3 ----
    m = n = k = 4096
    a, bt = inputs.c2_matmul_i8(m, n, k)
    a_d, bt_d = a.to(dev), bt.to(dev)
    c_d = torch.empty(m, n, dtype=torch.int32, device=dev)
    plan = pkg.plan(pkg.make_desc(pkg.ELEM_I8, pkg.ELEM_I8, pkg.ELEM_I32, m, n,
                                  k, pkg.B_TRANSPOSED))
    step = lambda: pkg.matmul(a_d, bt_d, c_d, b_transposed=True)  # noqa: E731
    ms = timed(step, args.steps, args.warmup)
    ops = 2.0 * m * n * k
    tops = ops / (ms * 1e-3) / 1e12

    # ---- fp16 4096^3 (B transposed: the TN MFMA path) ----
    g = torch.Generator().manual_seed(0)
    x16_h = (torch.randn(m, k, generator=g) * 0.02).half()
    w16_h = (torch.randn(n, k, generator=g) * 0.02).half()
    x16, w16 = x16_h.to(dev), w16_h.to(dev)
    y16 = torch.empty(m, n, dtype=torch.float16, device=dev)
    plan16 = pkg.plan(pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_F16, pkg.ELEM_F16,
                                    m, n, k, pkg.B_TRANSPOSED))
    ms16 = timed(lambda: pkg.matmul(x16, w16, y16, b_transposed=True),
                 args.steps, args.warmup)
    tflops16 = ops / (ms16 * 1e-3) / 1e12

    # ---- GEMV M=1, N=K=4096 f16, rotating weights past the MALL ----
    wbytes = 4096 * 4096 * 2
    copies = max(2, ROTATE_BYTES // wbytes + 1)
    ws = rotating(lambda: (torch.randn(4096, 4096, device=dev) * 0.02).half(),
                  copies)
    xv = torch.randn(1, 4096, device=dev).half()
    yv = torch.empty(1, 4096, dtype=torch.float16, device=dev)
    it = [0]

    def gemv_step():
        pkg.matmul(xv, ws[it[0] % copies], yv)
        it[0] += 1
    msv = timed(gemv_step, max(args.steps, 4 * copies), args.warmup)
    gemv_bytes = wbytes + 4096 * 2 * 2
    gemv_gbs = gemv_bytes / (msv * 1e-3) / 1e9
    del ws

    # ---- the other BASELINE configs the metric's kernels run on ----
    # C3 M=2048 N=K=4096 with row-major weights (linalg.matmul's map, NN)
    c3_h = inputs.c3_linear_f16(2048, 4096, 4096)
    x, wn = (t.to(dev) for t in c3_h)
    yn = torch.empty(2048, 4096, dtype=torch.float16, device=dev)
    ms_nn = timed(lambda: pkg.matmul(x, wn, yn), args.steps, args.warmup)
    nn_tflops = 2.0 * 2048 * 4096 * 4096 / (ms_nn * 1e-3) / 1e12
    del x, wn, yn
    # C4 attention
    q, kk, v = (t.to(dev) for t in inputs.c4_attention_f16())
    o = torch.empty_like(q)
    ms_att = timed(lambda: pkg.attention(q, kk, v, o, causal=True),
                   min(args.steps, 200), min(args.warmup, 200))
    att_flops = 4.0 * 32 * 2048 * 2048 * 128 / 2
    att_tflops = att_flops / (ms_att * 1e-3) / 1e12
    del q, kk, v, o
    # C5 W8A16, M=1 (rotating int8 weights) and M=512
    c5 = {}
    for mm in (1, 512):
        xq, wq, sq = inputs.c5_w8a16(mm)
        cp = max(1, min(24, ROTATE_BYTES // wq.numel() + 1)) if mm == 1 else 1
        wqs = [wq.to(dev)] + [wq.to(dev).clone() for _ in range(cp - 1)]
        xq, sq = xq.to(dev), sq.to(dev)
        yq = torch.empty(mm, wq.shape[1], dtype=torch.float16, device=dev)
        itq = [0]

        def w8_step():
            pkg.quantized_matmul(xq, wqs[itq[0] % cp], sq, yq)
            itq[0] += 1
        c5[mm] = timed(w8_step, max(args.steps, 4 * cp), args.warmup)
        del wqs
    c5_m1_bytes = 4096 * 11008 + 2 * 11008 + 2 * 4096 + 2 * 11008
    c5_m1_gbs = c5_m1_bytes / (c5[1] * 1e-3) / 1e9
    c5_512_tflops = 2.0 * 512 * 11008 * 4096 / (c5[512] * 1e-3) / 1e12

    # ---- ceilings measured on this box (calibration kernels) ----
    # The register-only loop issues the MFMA shape the timed kernel issues:
    # the _m16 tiles run 16x16 MFMAs, which sustain more products per
    # second on random operands than the 32x32 ones.
    def mfma_shape(cfg):
        return 16 if cfg.endswith("_m16") else 32
    shape_i8 = mfma_shape(plan.config_name.decode())
    shape_f16 = mfma_shape(plan16.config_name.decode())
    ceil_i8 = mfma_ceiling(dev, "i8", True, shape=shape_i8)
    ceil_f16 = mfma_ceiling(dev, "f16", True, shape=shape_f16)
    stream32 = stream_ceiling(dev, 4096 * 4096 * 2, args.steps, args.warmup)

    out = {
        "metric": "int8/fp16 matmul TOPS/TFLOPS + % MFMA peak at 4096^3; "
                  "GEMV HBM GB/s",
        "value": round(tops, 1),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic (seeded torch generators, BASELINE configs[1])",
        "config": {"workload": "C2 int8 matmul M=N=K=4096, A row-major, "
                               "B column-major, i32 out",
                   "kernel": plan.config_name.decode()},
        "roofline": {"bound": "mfma", "achieved": round(tops, 1),
                     "peak": PEAK_I8_TOPS, "unit": "TOPS",
                     "frac": round(tops / PEAK_I8_TOPS, 4),
                     "traffic": profiled_traffic(plan.config_name.decode()),
                     "ceiling": round(ceil_i8, 1),
                     "ceiling_frac": round(tops / ceil_i8, 4),
                     "ceiling_kind": f"register-only int8 {shape_i8}x"
                                     f"{shape_i8} MFMA loop (the shape the "
                                     "kernel issues) on random operands, "
                                     "measured in this run"},
        "extra": {
            "fp16_4096_tflops": round(tflops16, 1),
            "fp16_4096_frac_peak": round(tflops16 / PEAK_F16_TFLOPS, 4),
            "fp16_4096_layout": "B [N,K] (transposed), f32 acc, f16 out",
            "fp16_4096_kernel": plan16.config_name.decode(),
            "fp16_mfma_ceiling_tflops": round(ceil_f16, 1),
            "fp16_mfma_ceiling_shape": f"{shape_f16}x{shape_f16}",
            "fp16_4096_frac_ceiling": round(tflops16 / ceil_f16, 4),
            "c3_m2048_n4096_k4096_nn_tflops": round(nn_tflops, 1),
            "c3_m2048_n4096_k4096_nn_frac_peak":
                round(nn_tflops / PEAK_F16_TFLOPS, 4),
            "gemv_m1_4096_gbs": round(gemv_gbs, 1),
            "gemv_m1_4096_frac_hbm": round(gemv_gbs / PEAK_HBM_GBS, 4),
            "gemv_rotating_copies": copies,
            "hbm_stream_read_32mib_gbs": stream32["gbs"],
            "gemv_m1_4096_frac_stream": round(gemv_gbs / stream32["gbs"], 4),
            "c4_attention_tflops": round(att_tflops, 1),
            "c4_attention_us": round(ms_att * 1e3, 2),
            "c4_attention_frac_peak": round(att_tflops / PEAK_F16_TFLOPS, 4),
            "c5_w8a16_m1_gbs": round(c5_m1_gbs, 1),
            "c5_w8a16_m1_us": round(c5[1] * 1e3, 2),
            "c5_w8a16_m1_frac_hbm": round(c5_m1_gbs / PEAK_HBM_GBS, 4),
            "c5_w8a16_m512_tflops": round(c5_512_tflops, 1),
            "c5_w8a16_m512_frac_peak": round(c5_512_tflops / PEAK_F16_TFLOPS, 4),
        },
    }
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        out["extra"]["cpu_baselines"] = cpu_baselines_extra(
            inputs, threads, x16_h, w16_h, c3_h)
        cpu_tops, runs, dt = cpu_baseline_i8(a.numpy(), bt.numpy(), threads)
        out["cpu_baseline"] = {
            "value": round(cpu_tops, 4), "unit": "TOPS", "cores": threads,
            "kind": "port", **cpu_info(),
            "sample": f"the full C2 4096^3 int8 matmul, {runs} runs in "
                      f"{dt:.1f} s, by the C oracle (OpenMP, -O3 AVX2, "
                      f"{threads} threads: this box's share) on the same "
                      "inputs; IREE llvm-cpu is not installable without "
                      "network"}
    print(json.dumps(out), flush=True)


def cpu_baselines_extra(inputs, threads, x16, w16, c3, budget_s=1.5):
    """The C oracle on the host cores beside each extra workload of the
    default line: a bounded sample of the same inputs (rows of the output,
    or one attention head), each repeated to about `budget_s`, reported in
    the workload's own unit and labelled with the sample."""
    import oracle
    import numpy as np
    res = {}

    def rec(name, value, unit, sample):
        res[name] = {"value": round(value, 4), "unit": unit, "cores": threads,
                     "kind": "port", "sample": sample}

    rows = 256
    xs, wt = x16.numpy()[:rows], w16.numpy()
    sec, runs = cpu_time(lambda: oracle.matmul_f16(
        xs, wt, b_transposed=True, threads=threads), budget_s)
    rec("fp16_4096", 2.0 * rows * 4096 * 4096 / sec / 1e12, "TFLOP/s",
        f"{rows} of the 4096 output rows of the fp16 4096^3 TN matmul, "
        f"{runs} runs")
    xs, wn = c3[0].numpy()[:rows], c3[1].numpy()
    sec, runs = cpu_time(lambda: oracle.matmul_f16(xs, wn, threads=threads),
                         budget_s)
    rec("c3_m2048_n4096_k4096_nn", 2.0 * rows * 4096 * 4096 / sec / 1e12,
        "TFLOP/s", f"{rows} of the 2048 output rows of C3 M=2048 N=K=4096 NN, "
        f"{runs} runs")
    xv, wv = c3[0].numpy()[:1], c3[1].numpy()
    sec, runs = cpu_time(lambda: oracle.matmul_f16(xv, wv, threads=threads),
                         budget_s)
    rec("gemv_m1_4096", (4096 * 4096 * 2 + 4 * 4096) / sec / 1e9, "GB/s",
        f"the whole C3 M=1 N=K=4096 GEMV, {runs} runs")
    q, k, v = (t.numpy()[:, :1] for t in inputs.c4_attention_f16())
    sec, runs = cpu_time(lambda: oracle.attention_f16(
        q, k, v, causal=True, threads=threads), budget_s)
    rec("c4_attention", 4.0 * 2048 * 2048 * 128 / 2 / sec / 1e12, "TFLOP/s",
        f"1 of the 32 heads of C4 (causal, S=2048, D=128), {runs} runs")
    for mm, sample_rows in ((1, 1), (512, 64)):
        xq, wq, sq = (t.numpy() for t in inputs.c5_w8a16(mm))
        xq = np.ascontiguousarray(xq[:sample_rows])
        sec, runs = cpu_time(lambda: oracle.w8a16(xq, wq, sq,
                                                  threads=threads), budget_s)
        if mm == 1:
            rec("c5_w8a16_m1",
                (4096 * 11008 + 2 * 11008 + 4 * 4096) / sec / 1e9, "GB/s",
                f"the whole C5 M=1 W8A16 GEMV, {runs} runs")
        else:
            rec("c5_w8a16_m512",
                2.0 * sample_rows * 11008 * 4096 / sec / 1e12, "TFLOP/s",
                f"{sample_rows} of the 512 output rows of C5 M=512, "
                f"{runs} runs")
    return res


def suite(pkg, inputs, dev, args):
    import torch
    import oracle
    steps, warm = args.steps, args.warmup
    threads = cpu_threads()
    host = cpu_info()

    def emit(name, ms, flops, nbytes, bound, extra=None, cpu=None):
        """One line per config; `cpu` = (fn, sample text, fraction of the
        config's work one fn() call does) times the C oracle beside it."""
        rec = {"config": name, "ms": round(ms, 5),
               "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
               "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "bound": bound}
        peak = PEAK_HBM_GBS if bound == "hbm" else (
            PEAK_I8_TOPS if "i8" in name else PEAK_F16_TFLOPS)
        rec["frac"] = round((rec["gbs"] if bound == "hbm" else rec["tflops"])
                            / peak, 4)
        if extra:
            rec.update(extra)
        if cpu is not None and not args.no_cpu_baseline:
            fn, sample, share = cpu
            sec, runs = cpu_time(fn)
            full = sec / share  # seconds for the whole config
            rec["cpu_baseline"] = {
                "ms": round(full * 1e3, 3),
                "tflops": round(flops / full / 1e12, 4),
                "gbs": round(nbytes / full / 1e9, 2),
                "gpu_speedup": round(full * 1e3 / ms, 1),
                "cores": threads, "kind": "port", **host,
                "sample": f"{sample}, {runs} run(s), C oracle on {threads} "
                          "threads"}
        print(json.dumps(rec), flush=True)

    ah, bh = inputs.c1_matmul_f16()
    a, b = ah.to(dev), bh.to(dev)
    c = torch.empty(128, 512, dtype=torch.float16, device=dev)
    ms = timed(lambda: pkg.matmul(a, b, c), steps, warm)
    an, bn = ah.numpy(), bh.numpy()
    emit("C1 f16 128x512x256", ms, 2 * 128 * 512 * 256, 458752, "latency",
         cpu=(lambda: oracle.matmul_f16(an, bn, threads=threads),
              "the full C1 matmul", 1.0))

    ah, bh = inputs.c2_matmul_i8()
    a, bt = ah.to(dev), bh.to(dev)
    c = torch.empty(4096, 4096, dtype=torch.int32, device=dev)
    ms = timed(lambda: pkg.matmul(a, bt, c, b_transposed=True), steps, warm)
    an, bn = ah.numpy(), bh.numpy()
    emit("C2 i8 4096^3", ms, 2 * 4096 ** 3, 100663296, "mfma",
         cpu=(lambda: oracle.matmul_i8(an, bn, b_transposed=True,
                                       threads=threads),
              "the full C2 matmul", 1.0))
    del a, bt, c

    for m in (1, 16, 128, 2048):
        for n, k in ((4096, 4096), (11008, 4096), (4096, 11008)):
            x, w = inputs.c3_linear_f16(m, n, k)
            wbytes = n * k * 2
            copies = max(1, min(24, ROTATE_BYTES // wbytes + 1)) if m <= 16 else 1
            ws = [w.to(dev)] + [w.to(dev).clone() for _ in range(copies - 1)]
            x = x.to(dev)
            y = torch.empty(m, n, dtype=torch.float16, device=dev)
            it = [0]

            def step():
                pkg.matmul(x, ws[it[0] % copies], y)
                it[0] += 1
            ms = timed(step, max(steps, 3 * copies), warm)
            fam = pkg.plan(pkg.make_desc(0, 0, 0, m, n, k, 0)).config_name.decode()
            rows = min(m, 256)  # the oracle on a row sample of the big M
            xn, wn = x[:rows].cpu().numpy(), w.numpy()
            emit(f"C3 f16 M={m} N={n} K={k}", ms, 2 * m * n * k,
                 2 * (m * k + k * n + m * n), "hbm" if m <= 16 else "mfma",
                 {"kernel": fam, "rotating_copies": copies},
                 cpu=(lambda: oracle.matmul_f16(xn, wn, threads=threads),
                      f"{rows} of {m} rows, scaled by {m / rows:g}",
                      rows / m))
            del ws

    qh, kh, vh = inputs.c4_attention_f16()
    q, k_, v = qh.to(dev), kh.to(dev), vh.to(dev)
    o = torch.empty_like(q)
    ms = timed(lambda: pkg.attention(q, k_, v, o, causal=True), steps, warm)
    # the oracle on 4 of the 32 heads (every head costs the same)
    q4, k4, v4 = (t[:, :4].contiguous().numpy() for t in (qh, kh, vh))
    emit("C4 attention causal B1 H32 S2048 D128", ms,
         4 * 32 * 2048 * 2048 * 128 / 2, 4 * q.numel() * 2, "mfma",
         cpu=(lambda: oracle.attention_f16(q4, k4, v4, causal=True,
                                           threads=threads),
              "4 of the 32 heads, scaled by 8", 4 / 32))
    # The same shape through the general form (not BASELINE configs): an
    # additive [S, S] mask shared by every head (the MFMA kernel's mask
    # instance), an f32 result, and head dim 96 (the 128-wide layout
    # reading 96 columns). The oracle on 4 heads beside each.
    g = torch.Generator().manual_seed(5)
    mh = (2 * torch.randn(2048, 2048, generator=g)).half()
    md = mh.to(dev)
    o32 = torch.empty(q.shape, dtype=torch.float32, device=dev)
    for name, fn, oracle_fn, nbytes in (
            ("C4 shape, additive mask [S, S], causal",
             lambda: pkg.attention(q, k_, v, o, causal=True, mask=md),
             lambda: oracle.attention(q4, k4, v4, causal=True, mask=mh.numpy(),
                                      threads=threads),
             4 * q.numel() * 2 + md.numel() * 2),
            ("C4 shape, f32 result, causal",
             lambda: pkg.attention(q, k_, v, o32, causal=True),
             lambda: oracle.attention(q4, k4, v4, causal=True, out_f32=True,
                                      threads=threads),
             3 * q.numel() * 2 + o32.numel() * 4)):
        ms = timed(fn, steps, warm)
        emit(name, ms, 4 * 32 * 2048 * 2048 * 128 / 2, nbytes, "mfma",
             cpu=(oracle_fn, "4 of the 32 heads, scaled by 8", 4 / 32))
    q96, k96, v96 = (t[..., :96].contiguous() for t in (qh, kh, vh))
    q96d, k96d, v96d = q96.to(dev), k96.to(dev), v96.to(dev)
    o96 = torch.empty_like(q96d)
    ms = timed(lambda: pkg.attention(q96d, k96d, v96d, o96, causal=True),
               steps, warm)
    q4, k4, v4 = (t[:, :4].contiguous().numpy() for t in (q96, k96, v96))
    emit("C4 shape, head dim 96, causal", ms, 4 * 32 * 2048 * 2048 * 96 / 2,
         4 * q96d.numel() * 2, "mfma",
         cpu=(lambda: oracle.attention(q4, k4, v4, causal=True,
                                       threads=threads),
              "4 of the 32 heads, scaled by 8", 4 / 32))
    del q, k_, v, o, md, o32, q96d, k96d, v96d, o96

    for m in (1, 512):
        x, w, s = inputs.c5_w8a16(m)
        wbytes = w.numel()
        copies = max(1, min(24, ROTATE_BYTES // wbytes + 1)) if m == 1 else 1
        ws = [w.to(dev)] + [w.to(dev).clone() for _ in range(copies - 1)]
        x, s = x.to(dev), s.to(dev)
        y = torch.empty(m, w.shape[1], dtype=torch.float16, device=dev)
        it = [0]

        def step():
            pkg.quantized_matmul(x, ws[it[0] % copies], s, y)
            it[0] += 1
        ms = timed(step, max(steps, 3 * copies), warm)
        n, k = w.shape[1], w.shape[0]
        rows = min(m, 128)
        xn, wn, sn = x[:rows].cpu().numpy(), w.numpy(), s.cpu().numpy()
        emit(f"C5 w8a16 M={m} N={n} K={k}", ms, 2 * m * n * k,
             n * k + 2 * n + 2 * m * k + 2 * m * n, "hbm" if m == 1 else "mfma",
             {"rotating_copies": copies},
             cpu=(lambda: oracle.w8a16(xn, wn, sn, threads=threads),
                  f"{rows} of {m} rows, scaled by {m / rows:g}", rows / m))
        del ws

    runtime_suite(pkg, inputs, dev, emit, steps)


def timed_queued(fn, steps, warmup):
    """Average ms per step of fn() for work that cannot be graph-captured
    (concurrent lane streams): `warmup` steps, then `steps` steps enqueued
    behind a spin kernel long enough that the host has queued them all before
    the GPU starts, timed between events on the current stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(SPIN_CYCLES * 16)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def runtime_suite(pkg, inputs, dev, emit, steps):
    """The runtime's concurrency (the reference's max concurrent dispatches):
    one command buffer of 8 independent dispatches, submitted with 1, 2, 4
    and 8 lanes, for C1-size f16 matmuls (4 workgroups each), C3 M=16 skinny
    ones (split-K over every CU, one workspace slice per lane) and long int8
    matmuls of 2 workgroups each (K = 8192, no split-K for int8)."""
    import torch
    cases = (("C1 f16 128x512x256", "matmul_f16", (128, 512, 256)),
             ("C3 f16 M=16 N=4096 K=4096", "matmul_f16", (16, 4096, 4096)),
             ("i8 256x512x8192", "matmul_i8", (256, 512, 8192)))
    for label, export, (m, n, k) in cases:
        g = torch.Generator().manual_seed(1)
        i8 = export == "matmul_i8"
        if i8:
            xs = [torch.randint(-128, 128, (m, k), generator=g).to(torch.int8).to(dev)
                  for _ in range(8)]
            w = torch.randint(-128, 128, (n, k), generator=g).to(torch.int8).to(dev)
            ys = [torch.empty(m, n, dtype=torch.int32, device=dev) for _ in range(8)]
            consts = pkg.matmul_constants(m, n, k, k, k, n, pkg.B_TRANSPOSED)
        else:
            xs = [torch.randn(m, k, generator=g).half().to(dev) for _ in range(8)]
            w = torch.randn(k, n, generator=g).half().to(dev)
            ys = [torch.empty(m, n, dtype=torch.float16, device=dev) for _ in range(8)]
            consts = pkg.matmul_constants(m, n, k, k, n, n, 0)
        cb = pkg.CommandBuffer()
        for i in range(8):
            cb.dispatch(export, consts, [pkg.slot(i), pkg.slot(8), pkg.slot(9 + i)])
        cb.end()
        table = xs + [w] + ys
        for lanes in (1, 2, 4, 8):
            steps_q = max(20, min(steps, 100))
            ms = timed_queued(lambda: cb.submit(table, max_concurrent=lanes),
                              steps_q, 20)
            emit(f"runtime 8 x {label}, {lanes} lane{'s' if lanes > 1 else ''}",
                 ms, 8 * 2 * m * n * k, 8 * 2 * (m * k + k * n + m * n),
                 "latency", {"dispatches": 8, "lanes": lanes})


def only(pkg, inputs, dev, args):
    """One workload, for profiler passes: prints ms per step."""
    import torch
    w = args.only
    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if w == "stream":
        # the GEMV's 32 MiB, the C5 int8 weights (45 MB) and the 11008 x
        # 4096 f16 weights (90 MB)
        for nbytes in (4096 * 4096 * 2, 4096 * 11008, 11008 * 4096 * 2):
            rec = stream_ceiling(dev, nbytes, args.steps, args.warmup)
            rec["frac_hbm"] = round(rec["gbs"] / PEAK_HBM_GBS, 4)
            print(json.dumps({"only": w, **rec}), flush=True)
        return
    if w == "mfma_ceiling":
        for kind in ("i8", "f16"):
            for shape, rnd in ((32, True), (32, False), (16, True), (16, False)):
                v = mfma_ceiling(dev, kind, rnd, shape=shape)
                peak = PEAK_I8_TOPS if kind == "i8" else PEAK_F16_TFLOPS
                print(json.dumps({
                    "only": w, "kind": kind,
                    "mfma": f"{shape}x{shape}",
                    "operands": "random" if rnd else "constant",
                    "value": round(v, 1),
                    "unit": "TOPS" if kind == "i8" else "TFLOP/s",
                    "frac_peak": round(v / peak, 4)}), flush=True)
        return
    if w == "config":
        fn = config_step(pkg, dev, args.config,
                         [int(x) for x in args.shape.split(",")],
                         splits=args.splits, rotate=args.rotate)
    elif w == "i8":
        a, bt = (t.to(dev) for t in inputs.c2_matmul_i8())
        c = torch.empty(4096, 4096, dtype=torch.int32, device=dev)
        fn = lambda: pkg.matmul(a, bt, c, b_transposed=True)  # noqa: E731
    elif w in ("f16", "f16nn"):
        x, wt = inputs.c3_linear_f16(4096, 4096, 4096)
        x = x.to(dev)
        bt = w == "f16"
        b = (wt.t().contiguous() if bt else wt).to(dev)
        c = torch.empty(4096, 4096, dtype=torch.float16, device=dev)
        fn = lambda: pkg.matmul(x, b, c, b_transposed=bt)  # noqa: E731
    elif w == "gemv":
        copies = ROTATE_BYTES // (4096 * 4096 * 2) + 1
        ws = [(torch.randn(4096, 4096, device=dev) * 0.02).half()
              for _ in range(copies)]
        x = torch.randn(1, 4096, device=dev).half()
        y = torch.empty(1, 4096, dtype=torch.float16, device=dev)
        it = [0]

        def fn():
            pkg.matmul(x, ws[it[0] % copies], y)
            it[0] += 1
    elif w == "attn":
        q, k, v = (t.to(dev) for t in inputs.c4_attention_f16())
        o = torch.empty_like(q)
        fn = lambda: pkg.attention(q, k, v, o, causal=True)  # noqa: E731
    elif w == "runtime":
        # One command buffer: fill, barrier, 4 C1 matmuls and 4 M=16 split-K
        # matmuls on 2 lanes, barrier, copy; submitted eagerly (lanes are not
        # graph-captured), each command a roctx range.
        g = torch.Generator().manual_seed(2)
        shapes = [(128, 512, 256)] * 4 + [(16, 4096, 4096)] * 4
        table, cb = [], pkg.CommandBuffer()
        out0 = None
        for i, (m, n, k) in enumerate(shapes):
            a = torch.randn(m, k, generator=g).half().to(dev)
            b = torch.randn(k, n, generator=g).half().to(dev)
            c = torch.empty(m, n, dtype=torch.float16, device=dev)
            out0 = c if out0 is None else out0
            table += [a, b, c]
        copy_dst = torch.empty_like(out0)
        table.append(copy_dst)
        cb.fill(pkg.slot(2), b"\x00\x00")
        cb.barrier()
        for i, (m, n, k) in enumerate(shapes):
            cb.dispatch("matmul_f16", pkg.matmul_constants(m, n, k, k, n, n, 0),
                        [pkg.slot(3 * i), pkg.slot(3 * i + 1), pkg.slot(3 * i + 2)])
        cb.barrier()
        cb.copy(pkg.slot(2), pkg.slot(3 * len(shapes)), out0.numel() * 2)
        cb.end()
        fn = lambda: cb.submit(table, max_concurrent=2)  # noqa: E731
        ms = timed_queued(fn, args.steps, args.warmup)
        print(json.dumps({"only": w, "ms_per_step": round(ms, 5),
                          "steps": args.steps}), flush=True)
        return
    elif w == "w8a16_nk":
        # C5 M=1 with the int8 weights stored [N, K] (a torch Linear's
        # layout: the row-dot GEMV), rotating copies past the Infinity Cache
        x, wq, s = (t.to(dev) for t in inputs.c5_w8a16(1))
        wt = wq.t().contiguous()
        copies = ROTATE_BYTES // wt.numel() + 1
        ws = [wt] + [wt.clone() for _ in range(copies - 1)]
        y = torch.empty(1, wt.shape[0], dtype=torch.float16, device=dev)
        it = [0]

        def fn():
            pkg.quantized_matmul(x, ws[it[0] % copies], s, y,
                                 w_transposed=True)
            it[0] += 1
    else:
        m = 1 if w == "w8a16" else 512
        x, wq, s = (t.to(dev) for t in inputs.c5_w8a16(m))
        y = torch.empty(m, wq.shape[1], dtype=torch.float16, device=dev)
        fn = lambda: pkg.quantized_matmul(x, wq, s, y)  # noqa: E731
    ms = timed(fn, args.steps, args.warmup)
    print(json.dumps({"only": w, "ms_per_step": round(ms, 5),
                      "steps": args.steps}), flush=True)


def config_step(pkg, dev, name, shape, splits=0, rotate=False):
    """One launch of MFMA configuration `name` on random operands of
    shape (M, N, K) in the layout the configuration reads, with `splits`
    K splits (split-K tiles); with `rotate`, each launch reads the next of
    enough copies of B to pass the Infinity Cache."""
    import torch
    cfg = next(c for c in pkg.mfma_configs() if c.name == name)
    m, n, k = shape
    g = torch.Generator().manual_seed(0)
    sc = None
    if cfg.a_elem == pkg.ELEM_I8:
        a = torch.randint(-128, 128, (m, k), generator=g).to(torch.int8)
        b = torch.randint(-128, 128,
                          (n, k) if cfg.b_form == pkg.B_FORM_TN else (k, n),
                          generator=g).to(torch.int8)
        c = torch.empty(m, n, dtype=torch.int32, device=dev)
    else:
        a = torch.randn(*((k, m) if cfg.a_transposed else (m, k)),
                        generator=g).half()
        if cfg.b_form == pkg.B_FORM_TN:
            b = torch.randn(n, k, generator=g).half()
        elif cfg.b_form == pkg.B_FORM_NN:
            b = torch.randn(k, n, generator=g).half()
        else:
            b = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8)
            sc = (torch.rand(n, generator=g) * 0.019 + 0.001).half().to(dev)
        c = torch.empty(m, n, dtype=torch.float32 if cfg.c_elem == pkg.ELEM_F32
                        else torch.float16, device=dev)
    a, b = a.to(dev), b.to(dev)
    copies = 1
    if rotate:
        copies = max(1, min(24, ROTATE_BYTES // (b.numel() * b.element_size())
                            + 1))
    bs = [b] + [b.clone() for _ in range(copies - 1)]
    it = [0]

    def step():
        pkg.matmul_mfma_config(cfg.index, a, bs[it[0] % copies], c, scale=sc,
                               splits=splits)
        it[0] += 1
    return step


# SQ counters one rocprofv3 pass can hold (at most 8 SQ counters), and what
# the tuner reads from them per wave.
TUNE_COUNTERS = ("SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES",
                 "SQ_WAIT_ANY", "SQ_INSTS_MFMA", "SQ_VALU_MFMA_BUSY_CYCLES",
                 "SQ_INSTS_LDS", "SQ_INSTS_VALU")


def _find(root, name):
    for d, _, files in os.walk(root):
        if name in files:
            yield os.path.join(d, name)


def tune_counters(pkg, args):
    """Every 4096^3 macro-tile candidate under rocprofv3, one child process
    each: the kernel's median duration and, per wave, MFMA, LDS and VALU
    instructions, the fraction of a wave's life spent waiting, and the MFMA
    pipe's busy fraction. SQ counters come summed over the 32 shader
    engines (8 XCDs x 4), each of 32 SIMDs; wave and wait cycles are in
    quad-cycles, so their ratio is unit-free."""
    import csv
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3")
    if prof is None:
        print(json.dumps({"error": "rocprofv3 not found"}))
        return
    work = tempfile.mkdtemp(prefix="tune_counters_")
    for cfg in pkg.mfma_configs():
        if "_sk" in cfg.name or cfg.tile_m < 128 or "+" in cfg.name:
            # split-K tiles are tuned on the skinny shapes; a column split
            # ("<head>+<tail>") has no ragged round to fill at 4096^3
            continue
        out = os.path.join(work, cfg.name)
        cmd = ["timeout", "-s", "KILL", "90", prof, "--pmc", *TUNE_COUNTERS,
               "--kernel-trace", "-d", out, "-o", "p", "--output-format", "csv",
               "--", sys.executable, os.path.join(ROOT, "bench.py"), "--only",
               "config", "--config", cfg.name, "--no-graph", "--steps", "20",
               "--warmup", "200", "--no-cpu-baseline"]
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                           cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"})
        if r.returncode != 0:
            print(json.dumps({"config": cfg.name, "error": r.returncode}),
                  flush=True)
            if r.returncode in (124, 137, 134, 139):
                break  # a killed or crashed profiler run ends the sweep
            continue
        sums, durs = {}, []
        for path in _find(out, "p_counter_collection.csv"):
            for row in csv.DictReader(open(path)):
                if "gemm_lds_kernel" in row["Kernel_Name"]:
                    sums.setdefault(row["Counter_Name"], []).append(
                        float(row["Counter_Value"]))
        for path in _find(out, "p_kernel_trace.csv"):
            for row in csv.DictReader(open(path)):
                if "gemm_lds_kernel" in row["Kernel_Name"]:
                    durs.append(int(row["End_Timestamp"]) -
                                int(row["Start_Timestamp"]))
        if not sums:
            continue
        avg = {k: sum(v) / len(v) for k, v in sums.items()}
        waves = avg.get("SQ_WAVES", 0.0) or 1.0
        busy = avg.get("SQ_BUSY_CYCLES", 0.0) or 1.0
        durs.sort()
        print(json.dumps({
            "config": cfg.name,
            "us_median": round(durs[len(durs) // 2] / 1000, 2) if durs else None,
            "mfma_per_wave": round(avg.get("SQ_INSTS_MFMA", 0) / waves),
            "lds_insts_per_wave": round(avg.get("SQ_INSTS_LDS", 0) / waves),
            "valu_per_wave": round(avg.get("SQ_INSTS_VALU", 0) / waves),
            "wait_frac": round(avg.get("SQ_WAIT_ANY", 0) /
                               (avg.get("SQ_WAVE_CYCLES", 0) or 1), 3),
            "mfma_busy_frac": round(avg.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) /
                                    (busy * 32), 3)}), flush=True)
    shutil.rmtree(work, ignore_errors=True)


SKINNY_SHAPES = [("f16", 16, 4096, 4096), ("f16", 16, 11008, 4096),
                 ("f16", 16, 4096, 11008), ("f16", 128, 4096, 4096),
                 ("f16", 128, 11008, 4096), ("f16", 128, 4096, 11008),
                 ("w8a16", 512, 11008, 4096), ("w8a16", 128, 11008, 4096),
                 # tile counts stream-K is planned for
                 ("f16", 192, 11008, 4096), ("w8a16", 192, 11008, 11008)]


def skinny_sweep(pkg, dev, args, kind, m, n, k):
    """Every eligible tile at every split count (1..16) and in stream-K runs
    on one skinny shape, with rotating weights: a list of records."""
    import torch
    g = torch.Generator().manual_seed(m + n + k)
    x = (torch.randn(m, k, generator=g) * 0.5).half().to(dev)
    if kind == "f16":
        w0 = (torch.randn(k, n, generator=g) * 0.02).half().to(dev)
        sc, form = None, pkg.B_FORM_NN
        desc = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_F16, pkg.ELEM_F16, m, n, k)
    else:
        w0 = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8).to(dev)
        sc = (torch.rand(n, generator=g) * 0.019 + 0.001).half().to(dev)
        form = pkg.B_FORM_W8A16
        desc = pkg.make_desc(pkg.ELEM_F16, pkg.ELEM_I8, pkg.ELEM_F16, m, n,
                             k, has_scale=True)
    copies = max(1, min(24, ROTATE_BYTES // (w0.numel() * w0.element_size()) + 1))
    ws = [w0] + [w0.clone() for _ in range(copies - 1)]
    y = torch.empty(m, n, dtype=torch.float16, device=dev)
    plan = pkg.plan(desc)
    out = []
    for c in pkg.mfma_configs():
        if (c.b_form != form or c.a_transposed or c.c_elem != pkg.ELEM_F16
                or n % c.tile_n or k % c.tile_k):
            continue
        split = "_sk" in c.name
        if not split and m % c.tile_m:
            continue
        for sp in ((1, 2, 3, 4, 6, 8, 12, 16, pkg.SPLITS_STREAM_K)
                   if split else (0,)):
            if split and sp > 0 and k // sp < c.tile_k:
                continue
            it = [0]

            def fn():
                pkg.matmul_mfma_config(c.index, x, ws[it[0] % copies], y,
                                       scale=sc, splits=sp)
                it[0] += 1
            ms = timed(fn, args.steps, args.warmup)
            out.append({"shape": [kind, m, n, k], "config": c.name,
                        "splits": sp, "us": round(ms * 1000, 2),
                        "planned": c.index == plan.config_index and
                        (not split or
                         (sp == pkg.SPLITS_STREAM_K
                          if plan.stream_k_steps > 0
                          else sp == plan.splits))})
    del ws, x, y
    torch.cuda.empty_cache()
    return out


def tune_skinny(pkg, dev, args):
    """The sweep the planner's skinny tuned entries, its split enumeration
    and its stream-K choice were checked against (skinny_sweep on every
    skinny C3 / C5 shape and two tile counts stream-K is planned for)."""
    for kind, m, n, k in SKINNY_SHAPES:
        for rec in skinny_sweep(pkg, dev, args, kind, m, n, k):
            print(json.dumps(rec), flush=True)


# One pass each: FETCH_SIZE takes 3 of a pass's 4 TCC counters and
# WRITE_SIZE 2, so they cannot share one.
SKINNY_TRAFFIC = ("FETCH_SIZE", "WRITE_SIZE")


def _profile_config(prof, work, tag, counters, rec, steps=20, warmup=100,
                    calibrate=False):
    """One rocprofv3 --pmc pass over `bench.py --only config` for record
    `rec`: {counter: mean per gemm dispatch}, gemm durations (ns) and, with
    `calibrate`, the largest value each counter read for another kernel
    (the 256 MiB calibration copy)."""
    import csv
    import subprocess
    kind, m, n, k = rec["shape"]
    out = os.path.join(work, tag)
    cmd = ["timeout", "-s", "KILL", "90", prof, "--pmc", *counters,
           "--kernel-trace", "-d", out, "-o", "p", "--output-format", "csv",
           "--", sys.executable, os.path.join(ROOT, "bench.py"), "--only",
           "config", "--config", rec["config"], "--shape", f"{m},{n},{k}",
           "--splits", str(rec["splits"]), "--rotate", "--no-graph",
           "--steps", str(steps), "--warmup", str(warmup),
           "--no-cpu-baseline"] + (["--calibrate-copy"] if calibrate else [])
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                       cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"})
    if r.returncode != 0:
        return None, r.returncode
    sums, other, durs = {}, {}, []
    for path in _find(out, "p_counter_collection.csv"):
        for row in csv.DictReader(open(path)):
            v = float(row["Counter_Value"])
            name = row["Counter_Name"]
            if "gemm_lds_kernel" in row["Kernel_Name"]:
                sums.setdefault(name, []).append(v)
            else:
                other[name] = max(other.get(name, 0.0), v)
    for path in _find(out, "p_kernel_trace.csv"):
        for row in csv.DictReader(open(path)):
            if "gemm_lds_kernel" in row["Kernel_Name"]:
                durs.append(int(row["End_Timestamp"]) -
                            int(row["Start_Timestamp"]))
    avg = {k2: sum(v) / len(v) for k2, v in sums.items()}
    return (avg, sorted(durs), other), 0


def tune_skinny_counters(pkg, dev, args):
    """For each skinny shape: the sweep, then the planner's pick and the
    three fastest other candidates under rocprofv3, in three passes (SQ
    counters; FETCH_SIZE; WRITE_SIZE, each scaled by a 256 MiB copy
    measured in the same run). One JSON line per candidate: sweep and profiled
    durations, HBM bytes read and written per dispatch, the rate they
    imply, the fraction of wave cycles spent waiting and the MFMA pipe's
    busy fraction."""
    import shutil
    import tempfile
    prof = shutil.which("rocprofv3")
    if prof is None:
        print(json.dumps({"error": "rocprofv3 not found"}))
        return
    work = tempfile.mkdtemp(prefix="skinny_counters_")
    calib = 256 << 20
    for kind, m, n, k in SKINNY_SHAPES:
        recs = skinny_sweep(pkg, dev, args, kind, m, n, k)
        recs.sort(key=lambda r: r["us"])
        pick = [r for r in recs if r["planned"]][:1]
        cands = pick + [r for r in recs if not r["planned"]][:3]
        for i, rec in enumerate(cands):
            tag = f"{kind}_{m}_{n}_{k}_{i}"
            sq, rc = _profile_config(prof, work, tag + "_sq", TUNE_COUNTERS,
                                     rec)
            if sq is None:
                print(json.dumps({**rec, "error": rc}), flush=True)
                if rc in (124, 137, 134, 139):
                    shutil.rmtree(work, ignore_errors=True)
                    return
                continue
            avg, durs, _ = sq
            waves = avg.get("SQ_WAVES", 0.0) or 1.0
            busy = avg.get("SQ_BUSY_CYCLES", 0.0) or 1.0
            us = durs[len(durs) // 2] / 1000 if durs else None
            moved = {}
            for cn in SKINNY_TRAFFIC:
                tr, rc = _profile_config(prof, work, f"{tag}_{cn}", (cn,),
                                         rec, calibrate=True)
                if tr is None:
                    print(json.dumps({**rec, "counter": cn, "error": rc}),
                          flush=True)
                    if rc in (124, 137, 134, 139):
                        shutil.rmtree(work, ignore_errors=True)
                        return
                    moved[cn] = None
                    continue
                tavg, _, other = tr
                ref = other.get(cn, 0.0)
                moved[cn] = (tavg.get(cn, 0.0) * calib / ref if ref > 0
                             else None)
            tot = (moved["FETCH_SIZE"] or 0) + (moved["WRITE_SIZE"] or 0)
            print(json.dumps({
                **rec, "us_profiled": round(us, 2) if us else None,
                "fetch_mb": round(moved["FETCH_SIZE"] / 1e6, 2)
                if moved["FETCH_SIZE"] else None,
                "write_mb": round(moved["WRITE_SIZE"] / 1e6, 2)
                if moved["WRITE_SIZE"] else None,
                "hbm_gbs": round(tot / (us * 1e3), 1) if us and tot else None,
                "waves": round(waves),
                "wait_frac": round(avg.get("SQ_WAIT_ANY", 0) /
                                   (avg.get("SQ_WAVE_CYCLES", 0) or 1), 3),
                "mfma_busy_frac": round(avg.get("SQ_VALU_MFMA_BUSY_CYCLES", 0)
                                        / (busy * 32), 3)}), flush=True)
    shutil.rmtree(work, ignore_errors=True)


def tune(pkg, inputs, dev, args):
    import torch
    if args.tune_skinny and args.tune_counters:
        return tune_skinny_counters(pkg, dev, args)
    if args.tune_skinny:
        return tune_skinny(pkg, dev, args)
    if args.tune_counters:
        return tune_counters(pkg, args)
    m = n = k = 4096
    g = torch.Generator().manual_seed(0)
    a8 = torch.randint(-128, 128, (m, k), generator=g).to(torch.int8).to(dev)
    b8 = torch.randint(-128, 128, (n, k), generator=g).to(torch.int8).to(dev)
    a16 = torch.randn(m, k, generator=g).half().to(dev)
    b16 = torch.randn(n, k, generator=g).half().to(dev)
    b16n = torch.randn(k, n, generator=g).half().to(dev)
    w8 = torch.randint(-128, 128, (k, n), generator=g).to(torch.int8).to(dev)
    s8 = (torch.rand(n, generator=g) * 0.019 + 0.001).half().to(dev)
    for cfg in pkg.mfma_configs():
        sc = None
        if cfg.a_elem == pkg.ELEM_I8:
            a, b = a8, b8
            c = torch.empty(m, n, dtype=torch.int32, device=dev)
        else:
            a = a16
            b = {pkg.B_FORM_TN: b16, pkg.B_FORM_NN: b16n,
                 pkg.B_FORM_W8A16: w8}[cfg.b_form]
            sc = s8 if cfg.b_form == pkg.B_FORM_W8A16 else None
            c = torch.empty(m, n, dtype=torch.float32 if cfg.c_elem == pkg.ELEM_F32
                            else torch.float16, device=dev)
        try:
            ms = timed(lambda: pkg.matmul_mfma_config(cfg.index, a, b, c,
                                                      scale=sc),
                       args.steps, args.warmup)
        except pkg.MI355XError as ex:  # a skinny split-K tile or a column
            # split: neither runs at 4096^3
            print(json.dumps({"config": cfg.name, "skipped": str(ex)}),
                  flush=True)
            continue
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        peak = PEAK_I8_TOPS if cfg.a_elem == pkg.ELEM_I8 else PEAK_F16_TFLOPS
        print(json.dumps({"config": cfg.name, "ms": round(ms, 4),
                          "tflops_or_tops": round(tf, 1),
                          "frac": round(tf / peak, 4)}), flush=True)


if __name__ == "__main__":
    main()
