"""Benchmark of Plan::execute (C = A*B, FP32, packed VBSR A) on one MI355X.

Default workload: BASELINE configuration 3 -- 4096 block rows, degree 8,
block heights/widths uniform over {8,...,64} (independent), random columns,
RHS 32, seed 1; A and B values uniform in [-1, 1].  The reference publishes
0.95043 ms median for this exact instance on an RTX 5060 Ti
(data/publication/regime_map_seed1.csv:362).

Timing: per-step HIP events recorded on the stream the kernel runs on, created
with hipEventDisableSystemFence: the HIP runtime's timing-only events, which
skip the system-scope cache writeback/invalidate that a default event adds
around the kernel (the runtime documents them as the accurate way to time on
AMD GPUs).  The median of default events is reported beside it.
Every step is synchronised before the next is enqueued, as the reference
times each repetition (bench/benchmark.cpp:148-183: record, run, record,
synchronise).  "cold" steps first read a 1 GiB buffer (untimed, read-only so
no dirty lines are left behind) so that neither L2 nor the 256 MB Infinity
Cache holds A, B or C -- inputs are resident in HBM only.  "hot" steps do not:
the reference's methodology.  `value` is algorithmic bytes / cold median.

Algorithmic work per execute: bytes = 4*S (A once) + 4*rhs*K (B once)
+ 4*rhs*M (C once) + metadata; flops = 2*rhs*S; S = sum of h*w.

Prints one JSON line.  Single GPU only: --gpus N > 1 exits with a message.
"""

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
REFERENCE_MEDIAN_MS = {  # data/publication/regime_map_seed1.csv, row_owned_hybrid, 4096/8/high/random/seed 1
    8: 1.27706, 16: 0.88675, 32: 0.95043, 64: 1.55469}


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--rows", type=int, default=4096)
    p.add_argument("--degree", type=int, default=8)
    p.add_argument("--distribution", default="high")
    p.add_argument("--locality", default="random")
    p.add_argument("--rhs", type=int, default=32)
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--kernel", choices=["plan", "scalar", "valu", "wide_b", "rhs64_splitk", "rhs64_tiles"],
                   default="plan",
                   help="plan = the library's Plan::execute; scalar = the order-preserving kernel; valu = the "
                        "row-owned kernel with plain FP32 multiply-adds instead of MFMA (the measured alternative); "
                        "wide_b = the row-owned kernel reading B through 64-bit addresses, the form it takes past "
                        "the 32-bit offset bound on K; rhs64_splitk / rhs64_tiles = launch_row_owned with the RHS 64 "
                        "kernel forced to the split-k kernel / the tile split (the plan takes the one the matrix's "
                        "rule names)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-parity", action="store_true")
    p.add_argument("--calibrate-copy-mib", type=int, default=0,
                   help="also run a plain device copy of this many MiB (HBM-counter calibration)")
    return p.parse_args()


def algorithmic_work(host, rhs):
    S = int(host.values.size)
    M, K = host.scalar_rows, host.scalar_cols
    R, C, nnzb = host.block_rows, host.block_cols, host.nnzb
    meta = 4 * (R + 1) + 4 * nnzb + 4 * R + 4 * C + 8 * (R + 1) + 8 * (C + 1) + 8 * (nnzb + 1)
    return {"sum_hw": S, "bytes": 4 * S + 4 * rhs * K + 4 * rhs * M + meta, "flops": 2.0 * rhs * S,
            "scalar_rows": M, "scalar_cols": K, "nnzb": nnzb}


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


class TimingEvents:
    """hipEventDisableSystemFence events from the HIP runtime instance torch
    loaded (found by path, so that its stream handles are valid here)."""

    def __init__(self):
        path = None
        with open("/proc/self/maps") as maps:
            for line in maps:
                if "libamdhip64" in line:
                    path = line.split()[-1]
                    break
        if path is None:
            raise RuntimeError("the HIP runtime is not loaded")
        self.hip = ctypes.CDLL(path)
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.events = []

    def create(self):
        event = ctypes.c_void_p()
        if self.hip.hipEventCreateWithFlags(ctypes.byref(event), HIP_EVENT_DISABLE_SYSTEM_FENCE) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")
        self.events.append(event)
        return event

    def record(self, event, stream):
        if self.hip.hipEventRecord(event, ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, start, end):
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), start, end) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def close(self):
        for event in self.events:
            self.hip.hipEventDestroy(event)
        self.events = []


def percentile_95(sorted_values):
    return sorted_values[min(len(sorted_values) - 1, int(len(sorted_values) * 0.95))]


def cpu_baseline(host, b, rhs, budget_s=20.0):
    """The oracle's restatement of cpu_reference (vbsr.cpp:167-201), single thread, on the same instance."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_ffi

    oracle_host = oracle_ffi.HostMatrix(host.block_rows, host.block_cols, **host.arrays())
    t0 = time.perf_counter()
    reference = oracle_ffi.cpu_reference(oracle_host, b, rhs)  # warmup, also the parity reference
    first = time.perf_counter() - t0
    reps = max(1, min(5, int(budget_s / max(first, 1e-3)) - 1))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        oracle_ffi.cpu_reference(oracle_host, b, rhs)
        times.append(time.perf_counter() - t0)
    times.sort()
    return reference, oracle_host, {"median_s": times[len(times) // 2], "p95_s": percentile_95(times), "reps": reps,
                                    "warmup": 1}


def cpu_threads():
    """Host threads this process may use: OMP_NUM_THREADS when set, else its CPU affinity."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    requested = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(allowed, requested) if requested > 0 else allowed)


def cpu_parallel(oracle_host, b, rhs, reference, budget_s=10.0):
    """A multi-core CPU baseline owned by this build (the reference is single-threaded): the oracle's
    cpu_reference with block rows spread over OpenMP threads, bit-identical to the serial result."""
    import numpy as np
    import oracle_ffi

    threads = cpu_threads()
    t0 = time.perf_counter()
    result = oracle_ffi.cpu_reference_threads(oracle_host, b, rhs, threads)  # warmup
    first = time.perf_counter() - t0
    reps = max(3, min(20, int(budget_s / max(first, 1e-3)) - 1))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        oracle_ffi.cpu_reference_threads(oracle_host, b, rhs, threads)
        times.append(time.perf_counter() - t0)
    times.sort()
    return threads, bool(np.array_equal(result, reference)), {"median_s": times[len(times) // 2],
                                                              "p95_s": percentile_95(times), "reps": reps}


def cpu_config1():
    """The CPU-only benchmark configuration 1 (1024 block rows, degree 4, high block sizes, clamped
    local columns, RHS 8, seed 1): the same oracle timing, single thread."""
    import varblockspmm_amd as vb

    host = vb.generate(1024, 1024, 4, "high", "clamped", 1)
    b = vb.make_random_input(host.scalar_cols * 8, 1)
    _, _, timing = cpu_baseline(host, b, 8)
    return {"median_ms": round(timing["median_s"] * 1e3, 3), "p95_ms": round(timing["p95_s"] * 1e3, 3),
            "reps": timing["reps"], "warmup": 1, "sum_hw": int(host.values.size),
            "workload": "config 1: 1024 block rows, degree 4, high block sizes, clamped local columns, rhs 8, seed 1"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the VBSR SpMM path has no multi-GPU code "
              "(it would shard by block rows, with B broadcast to every GPU). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import varblockspmm_amd as vb

    device = "cuda:0"
    print(f"[bench] generating rows={args.rows} degree={args.degree} {args.distribution}/{args.locality} "
          f"rhs={args.rhs} seed={args.seed}", file=sys.stderr, flush=True)
    host = vb.generate(args.rows, args.rows, args.degree, args.distribution, args.locality, args.seed)
    work = algorithmic_work(host, args.rhs)
    b_host = vb.make_random_input(host.scalar_cols * args.rhs, args.seed)

    matrix = vb.Matrix(host)
    plan = vb.Plan(matrix, args.rhs)
    view = matrix.device_view()
    stream = torch.cuda.Stream(device=device)
    b_dev = torch.from_numpy(b_host).to(device)
    c_dev = torch.full((host.scalar_rows * args.rhs,), float("nan"), device=device)
    flush = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=device)  # 1 GiB
    sink = torch.empty((), dtype=torch.float32, device=device)
    torch.cuda.synchronize()

    schedule = matrix.row_schedule()
    if args.kernel in ("rhs64_splitk", "rhs64_tiles"):
        schedule.rhs64_tiles = 1 if args.kernel == "rhs64_tiles" else 0

    def step():
        if args.kernel == "plan":
            plan.execute(b_dev, c_dev, stream)
        elif args.kernel == "valu":
            vb.launch_row_owned_valu(view, schedule, b_dev, c_dev, args.rhs, stream)
        elif args.kernel == "wide_b":
            vb.launch_row_owned_wide_b(view, schedule, b_dev, c_dev, args.rhs, stream)
        elif args.kernel in ("rhs64_splitk", "rhs64_tiles"):
            vb.launch_row_owned(view, schedule, b_dev, c_dev, args.rhs, stream)
        else:
            vb.launch_row_owned_scalar(view, b_dev, c_dev, args.rhs, stream)

    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            step()
    torch.cuda.synchronize()
    first_result = c_dev.cpu().numpy().copy()
    print("[bench] warmup done", file=sys.stderr, flush=True)

    timing = TimingEvents()

    def timed(cold, fenced=False):
        if fenced:  # default events (system-scope fence around the kernel)
            starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
            ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
            record = lambda event: event.record(stream)
            elapsed = lambda start, end: start.elapsed_time(end)
        else:
            starts = [timing.create() for _ in range(args.steps)]
            ends = [timing.create() for _ in range(args.steps)]
            record = lambda event: timing.record(event, stream)
            elapsed = timing.elapsed_ms
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            for i in range(args.steps):
                if cold:
                    # Read-only sweep: evicts L2 and the Infinity Cache without
                    # leaving dirty lines whose write-back would be timed.
                    torch.sum(flush, (0,), out=sink)
                record(starts[i])
                step()
                record(ends[i])
                # One step at a time, as the reference times each repetition
                # (bench/benchmark.cpp:162-167: record, run, record, sync).
                stream.synchronize()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return sorted(elapsed(s, e) for s, e in zip(starts, ends)), wall

    cold_ms, cold_wall = timed(True)
    print("[bench] cold steps done", file=sys.stderr, flush=True)
    hot_ms, hot_wall = timed(False)
    print("[bench] hot steps done", file=sys.stderr, flush=True)
    fenced_ms, _ = timed(True, fenced=True)
    timing.close()
    final_result = c_dev.cpu().numpy()
    bit_stable = bool(np.array_equal(first_result.view(np.uint32), final_result.view(np.uint32)))

    calibration = None
    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * 1024 * 1024 // 4
        src = torch.ones(n, device=device)
        dst = torch.empty(n, device=device)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        calibration = {"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n}
        del src, dst

    median = cold_ms[len(cold_ms) // 2]
    mean = sum(cold_ms) / len(cold_ms)
    hot_median = hot_ms[len(hot_ms) // 2]
    achieved_gbs = work["bytes"] / (mean * 1e-3) / 1e9
    value_gbs = work["bytes"] / (median * 1e-3) / 1e9
    gflops = work["flops"] / (median * 1e-3) / 1e9

    parity = None
    cpu = None
    if not args.no_cpu_baseline or not args.no_parity:
        print("[bench] CPU oracle (baseline + parity)", file=sys.stderr, flush=True)
        reference, oracle_host, cpu_timing = cpu_baseline(host, b_host, args.rhs)
        if not args.no_parity:
            import oracle_ffi

            bound = oracle_ffi.abs_product_sum(oracle_host, b_host, args.rhs)
            max_abs, rel_l2, normwise, elementwise = oracle_ffi.parity_errors(final_result, reference, bound)
            parity = {"normwise": normwise, "rel_l2": rel_l2, "elementwise_vs_abs_bound": elementwise,
                      "max_abs": max_abs, "finite": bool(np.all(np.isfinite(final_result))),
                      "pass": bool(normwise <= 1e-5 and rel_l2 <= 1e-5 and elementwise <= 1e-6)}
        if not args.no_cpu_baseline:
            cpu = {"value": work["bytes"] / cpu_timing["median_s"] / 1e9, "unit": "GB/s", "cores": 1,
                   "kind": "port", "median_ms": cpu_timing["median_s"] * 1e3,
                   "sample": f"full workload: oracle cpu_reference (vbsr.cpp:167-201 restated in C) on the same "
                             f"instance and B, {cpu_timing['warmup']} warmup + {cpu_timing['reps']} reps, "
                             f"single thread; host {platform.processor() or platform.machine()}, "
                             f"nproc {os.cpu_count()}",
                   "config1": cpu_config1()}
            threads, identical, par = cpu_parallel(oracle_host, b_host, args.rhs, reference)
            cpu["parallel"] = {
                "value": work["bytes"] / par["median_s"] / 1e9, "unit": "GB/s", "cores": threads,
                "kind": "build-owned", "median_ms": par["median_s"] * 1e3, "p95_ms": par["p95_s"] * 1e3,
                "bit_identical_to_serial": identical,
                "sample": f"full workload: the same oracle cpu_reference with block rows spread over {threads} "
                          f"OpenMP threads (not in the reference, which is single-threaded), 1 warmup + "
                          f"{par['reps']} reps"}

    traffic = None
    traffic_file = os.path.join(ROOT, "profiles", f"traffic_r{args.rows}_d{args.degree}_{args.distribution}_"
                                f"{args.locality}_n{args.rhs}_s{args.seed}.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as handle:
            traffic = json.load(handle).get("hbm_bytes_per_launch")

    workload = (f"VBSR SpMM C=A*B: {args.rows} block rows x {args.rows} block cols, degree {args.degree}, "
                f"{args.distribution} block sizes, {args.locality} columns, rhs {args.rhs}, seed {args.seed}")
    ref_ms = REFERENCE_MEDIAN_MS.get(args.rhs) if (args.rows, args.degree, args.distribution, args.locality,
                                                    args.seed) == (4096, 8, "high", "random", 1) else None
    line = {
        "metric": "median ms + achieved HBM GB/s & FP32 GFLOP/s (% roofline), 4096 blk-rows deg 8 RHS 32",
        "value": round(value_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean, 5),
        "median_ms": round(median, 5),
        "p95_ms": round(percentile_95(cold_ms), 5),
        "hot_median_ms": round(hot_median, 5),
        "hot_p95_ms": round(percentile_95(hot_ms), 5),
        "default_event_median_ms": round(fenced_ms[len(fenced_ms) // 2], 5),
        "gflops": round(gflops, 1),
        "hbm_roofline_frac": round(value_gbs / HBM_PEAK_GBS, 4),
        "fp32_roofline_frac": round(gflops / 1e3 / FP32_PEAK_TFLOPS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(ref_ms / median, 3) if (ref_ms and args.kernel == "plan") else None,
        "dtype": "f32",
        "data": "synthetic (seeded generator, B = mt19937 uniform[-1,1])",
        "config": {"workload": workload, "kernel": args.kernel, "rhs64_tiles": int(matrix.row_schedule().rhs64_tiles),
                   "sum_hw": work["sum_hw"],
                   "algorithmic_bytes": work["bytes"], "flops": work["flops"], "launches": plan.launch_count(),
                   "timing": "hipEventDisableSystemFence events on the kernel's stream, each step synchronised "
                             "before the next (as bench/benchmark.cpp:148-183); cold = 1 GiB read-only sweep before "
                             "each step (untimed); hot = no sweep; default_event_median_ms = cold median with default "
                             "(system-fenced) events"},
        "roofline": {"bound": "hbm" if args.rhs <= 32 else "mfma", "achieved": round(achieved_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel_avg_ms": round(mean, 5)},
        "cpu_baseline": cpu,
        "parity": parity,
        "bit_stable": bit_stable,
        "wall_s": {"cold_steps": round(cold_wall, 3), "hot_steps": round(hot_wall, 3)},
    }
    if args.rhs == 64:
        achieved_tf = work["flops"] / (mean * 1e-3) / 1e12
        line["roofline"].update({"achieved": round(achieved_tf, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(achieved_tf / FP32_PEAK_TFLOPS, 4)})
    if calibration:
        line["calibration"] = calibration
    print(json.dumps(line), flush=True)
    plan.close()
    matrix.close()


if __name__ == "__main__":
    main()
