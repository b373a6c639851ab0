"""Throughput of the scan! / mapreduce hot path on one MI355X.

A step is one pass of the path over one batch of synthetic Float32 data at
n = 2^28 (BASELINE.json's headline configuration):
    scan!(+, dst, src)                 inclusive, 2*4*n bytes
    mapreduce!(identity, +, out, src)  full reduction, 4*n bytes
Inputs are resident in HBM before timing starts. `value` is algorithmic GB/s
of the whole step (12*n bytes / step time). The JSON line also carries the
per-kernel roofline of the dominant kernel (the scan), measured with HIP
events on the stream the kernels run on, the measured copy ceiling, and the
CPU baseline (the oracle's restatement of Base.accumulate! / Base.mapreduce,
timed on this host).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--all [--all-json PATH]]
  --all       also time every BASELINE.json configuration (stderr table, and
              the rows inside the JSON line as "all_configs")
  --all-json  also write those rows, with the copy ceiling, to PATH
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

PEAK_HBM_GBPS = 8000.0
N = 2**28


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_calls(fn, reps, batches=5, with_min=False):
    """Average seconds per call: `batches` event-timed batches of `reps`
    back-to-back calls on the current stream; returns the median batch
    (and the fastest batch when with_min)."""
    s = torch.cuda.current_stream()
    out = []
    for _ in range(batches):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        e1.synchronize()
        out.append(e0.elapsed_time(e1) / 1e3 / reps)
    med = float(np.median(out))
    return (med, float(np.min(out))) if with_min else med


def load_traffic():
    """HBM bytes per scan launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), if recorded."""
    p = os.path.join(REPO, "profiles", "traffic_scan_f32_2p28.json")
    if os.path.exists(p):
        with open(p) as fh:
            return json.load(fh).get("hbm_bytes_per_launch")
    return None


def _cpu_rate(oracle, x, y, threads, budget_s):
    """GB/s of steps (scan + sum over x) on `threads` host threads."""
    n = x.shape[0]
    oracle.baseline_scan_add_f32(x[: 1 << 20], y[: 1 << 20], threads)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.baseline_scan_add_f32(x, y, threads)
        oracle.baseline_sum_f32(x, threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 400:
            break
    return reps * 12 * n / el / 1e9, reps, el


def cpu_baseline(oracle, budget_s=12.0, single_budget_s=4.0):
    """The reference's CPU path (Base.accumulate! + Base.mapreduce) restated in
    C: multithreaded (two-pass chunked scan + chunked sum, OpenMP) on the whole
    workload, and single-threaded (the sequential left folds) on 2^24 elements."""
    threads = max(1, min(16, os.cpu_count() or 1))
    x = np.random.default_rng(20261201).random(N, dtype=np.float32)
    y = np.empty_like(x)
    gbps, reps, el = _cpu_rate(oracle, x, y, threads, budget_s)
    xs, ys = x[: 1 << 24], y[: 1 << 24]
    g1, reps1, el1 = _cpu_rate(oracle, xs, ys, 1, single_budget_s)
    return {"value": round(gbps, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} steps of the same workload (2^28 F32 two-pass chunked scan + chunked sum, "
                      f"Float32 arithmetic, OpenMP) on {threads} host threads, {el:.1f} s",
            "single_thread": {"value": round(g1, 3), "unit": "GB/s", "cores": 1,
                              "sample": f"{reps1} steps of sequential accumulate + sum over the first 2^24 "
                                        f"elements, {el1:.1f} s"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--all", action="store_true")
    ap.add_argument("--all-json", default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweep", action="store_true",
                    help="the reference's scan/mapreduce size sweep (perfs/julia/benchmarks)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the scan/mapreduce path here is single-GPU "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__
    kf = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    g = torch.Generator(device=dev).manual_seed(20261201)
    src = torch.rand(N, device=dev, generator=g, dtype=torch.float32)
    dst = torch.empty_like(src)
    out = torch.empty(1, device=dev, dtype=torch.float32)
    tmp_scan = kf.get_allocation(kf.Scan1D, kf.identity, "+", src)
    tmp_red = kf.get_allocation(kf.MapReduce1D, kf.identity, "+", src)

    def do_scan():
        kf.scan_("+", dst, src, tmp=tmp_scan)

    def do_reduce():
        kf.mapreduce_(kf.identity, "+", out, src, tmp=tmp_red)

    def step():
        do_scan()
        do_reduce()

    log(f"bench: warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    log(f"bench: timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_s = e0.elapsed_time(e1) / 1e3 / args.steps
    value = 12 * N / step_s / 1e9

    # per-kernel averages over the timed pattern (events on the launch stream)
    scan_s, scan_min = time_calls(do_scan, 20, batches=10, with_min=True)
    red_s, red_min = time_calls(do_reduce, 20, batches=10, with_min=True)
    cbuf = torch.empty_like(src)

    def do_copy():
        kf.vcopy_(cbuf, src)

    def do_dtod():
        cbuf.copy_(src)

    copy_s = time_calls(do_copy, 20)
    dtod_s = time_calls(do_dtod, 20)
    copy_gbps = 8 * N / copy_s / 1e9
    dtod_gbps = 8 * N / dtod_s / 1e9
    ceiling = max(copy_gbps, dtod_gbps)
    scan_gbps = 8 * N / scan_s / 1e9
    red_gbps = 4 * N / red_s / 1e9
    log(f"scan {scan_s*1e6:.1f} us {scan_gbps:.0f} GB/s | reduce {red_s*1e6:.1f} us {red_gbps:.0f} GB/s | "
        f"copy kernel {copy_gbps:.0f} GB/s, hipMemcpyDtoD {dtod_gbps:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        from oracle import oracle
        log("bench: cpu baseline")
        cpu = cpu_baseline(oracle)

    line = {
        "metric": "scan!/mapreduce GB/s and % HBM roofline at n=2^28 Float32, 1xMI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: U[0,1) Float32, torch.Generator seed 20261201, resident in HBM",
        "config": {"workload": "scan!(+, dst, src) inclusive + mapreduce!(identity, +, out, src), "
                               "Float32 n=2^28 (BASELINE.json configs[1] size, Float32 as in the metric)",
                   "n": N, "bytes_per_step": 12 * N},
        "roofline": {"bound": "hbm", "kernel": "scan_kernel<float,OpAdd,MapIdentity>",
                     "achieved": round(scan_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(scan_gbps / PEAK_HBM_GBPS, 4), "traffic": load_traffic(),
                     "avg_launch_us": round(scan_s * 1e6, 2), "algorithmic_bytes_per_launch": 8 * N},
        "kernels": {
            "scan_gbps": round(scan_gbps, 1), "scan_frac_of_copy": round(scan_gbps / ceiling, 4),
            "mapreduce_gbps": round(red_gbps, 1), "mapreduce_frac_of_copy": round(red_gbps / ceiling, 4),
            "mapreduce_frac_of_peak": round(red_gbps / PEAK_HBM_GBPS, 4), "mapreduce_avg_launch_us": round(red_s * 1e6, 2),
            "scan_gbps_best_batch": round(8 * N / scan_min / 1e9, 1),
            "mapreduce_gbps_best_batch": round(4 * N / red_min / 1e9, 1),
            "copy_kernel_gbps": round(copy_gbps, 1), "hipMemcpyDtoD_gbps": round(dtod_gbps, 1),
            "copy_ceiling_gbps": round(ceiling, 1),
        },
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 4),
    }
    if args.all:
        line["all_configs"] = bench_all(kf, dev, ceiling, args.all_json)
    if args.sweep:
        line["sweep"] = bench_sweep(kf, dev, ceiling)
    print(json.dumps(line), flush=True)


def _graph_time(fn, reps=20):
    """Seconds per call of fn, captured `reps` times in one HIP graph."""
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    return time_calls(graph.replay, 1) / reps


def bench_sweep(kf, dev, ceiling):
    """The reference's own size sweep (perfs/julia/benchmarks/
    scan_perf_comparison.jl:129-131, mapreduce_perf_comparison.jl:121-122):
    n in 10^6..10^9 for Float32, Float64 and UInt8, scan!(+) inclusive and
    mapreduce(identity, +). HIP-graph timed; GB/s of algorithmic bytes."""
    rows = []
    g = torch.Generator(device=dev).manual_seed(20261201)
    for n in (10**6, 10**7, 10**8, 10**9):
        for dt in (torch.float32, torch.float64, torch.uint8):
            if dt == torch.uint8:
                x = torch.randint(0, 4, (n,), device=dev, generator=g, dtype=dt)
            else:
                x = torch.rand(n, device=dev, generator=g, dtype=dt)
            es = x.element_size()
            y = torch.empty_like(x)
            o = torch.empty(1, device=dev, dtype=dt)
            ts = kf.get_allocation(kf.Scan1D, kf.identity, "+", x)
            tr = kf.get_allocation(kf.MapReduce1D, kf.identity, "+", x)
            for what, bytes_, fn in (
                    ("scan", 2 * es * n, lambda: kf.scan_("+", y, x, tmp=ts)),
                    ("mapreduce", es * n, lambda: kf.mapreduce_(kf.identity, "+", o, x, tmp=tr))):
                sec = _graph_time(fn, reps=20 if n < 10**9 else 5)
                gb = bytes_ / sec / 1e9
                rows.append({"op": what, "n": n, "dtype": str(dt).replace("torch.", ""),
                             "us": round(sec * 1e6, 2), "gbps": round(gb, 1),
                             "elems_per_s": round(n / sec, 1), "frac_copy": round(gb / ceiling, 4)})
                log(f"  {what:9s} {str(dt):14s} n={n:>10d} {sec*1e6:10.1f} us {gb:8.0f} GB/s "
                    f"{gb/ceiling*100:5.1f}% of copy")
            del x, y, ts, tr
    return rows


def bench_all(kf, dev, ceiling, json_path=None):
    """Every BASELINE.json configuration: GB/s, % of peak, % of the copy ceiling."""
    rows = []
    g = torch.Generator(device=dev).manual_seed(20261201)

    def rec(name, bytes_, fn, reps=20):
        # captured in a HIP graph so that host launch overhead does not hide
        # the kernel time of the small configurations
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        s = time_calls(graph.replay, 1) / reps
        gb = bytes_ / s / 1e9
        rows.append({"config": name, "us": round(s * 1e6, 2), "gbps": round(gb, 1),
                     "frac_peak": round(gb / PEAK_HBM_GBPS, 4), "frac_copy": round(gb / ceiling, 4)})
        log(f"  {name:48s} {s*1e6:10.1f} us {gb:8.0f} GB/s  {gb/ceiling*100:5.1f}% of copy")

    def tmp_for(kind, src, **kw):
        return kf.get_allocation(kind, kf.identity, "+", src, **kw)

    x = torch.rand(10**6, device=dev, generator=g)
    y = torch.empty_like(x)
    t1 = tmp_for(kf.Scan1D, x)
    rec("C1 scan F32 incl n=1e6", 8e6, lambda: kf.scan_("+", y, x, tmp=t1))
    del x, y
    xi = torch.randint(0, 16, (2**28,), device=dev, generator=g, dtype=torch.int32)
    yi = torch.empty_like(xi)
    t2 = tmp_for(kf.Scan1D, xi)
    rec("C2 scan Int32 incl n=2^28", 8 * 2**28, lambda: kf.scan_("+", yi, xi, tmp=t2))
    rec("C2 scan Int32 excl n=2^28", 8 * 2**28, lambda: kf.scan_("+", yi, xi, exclusive=True, tmp=t2))
    o = torch.empty(1, device=dev, dtype=torch.int32)
    xr = torch.randint(-2**31, 2**31 - 1, (2**28,), device=dev, generator=g, dtype=torch.int32)
    t3 = tmp_for(kf.MapReduce1D, xr)
    rec("C3c mapreduce max Int32 n=2^28", 4 * 2**28, lambda: kf.mapreduce_(kf.identity, max, o, xr, tmp=t3))
    del xi, yi, xr
    xf = torch.randn(2**30, device=dev, generator=g)
    of = torch.empty(1, device=dev)
    t3f = tmp_for(kf.MapReduce1D, xf)
    rec("C3a mapreduce abs2,+ F32 n=2^30", 4 * 2**30, lambda: kf.mapreduce_(kf.abs2, "+", of, xf, tmp=t3f), reps=10)
    del xf
    xd = torch.randn(2**28, device=dev, generator=g, dtype=torch.float64)
    od = torch.empty(1, device=dev, dtype=torch.float64)
    t3d = tmp_for(kf.MapReduce1D, xd)
    rec("C3b mapreduce abs2,+ F64 n=2^28", 8 * 2**28, lambda: kf.mapreduce_(kf.abs2, "+", od, xd, tmp=t3d))
    del xd
    ab = torch.empty(2**26, 2, device=dev)
    ab[:, 0].uniform_(0.9, 1.0, generator=g)
    ab[:, 1].normal_(generator=g)
    yab = torch.empty_like(ab)
    t4 = kf.get_allocation(kf.Scan1D, kf.identity, kf.affine, ab)
    rec("C4 affine scan n=2^26", 16 * 2**26, lambda: kf.scan_(kf.affine, yab, ab, tmp=t4))
    del ab, yab
    t = torch.rand(2**28, device=dev, generator=g) * 2 - 1
    A1 = t.as_strided((4096, 65536), (1, 4096))
    t5 = kf.KernelBuffer(kf.MapReduce2D, 64 << 20, dev)  # >= every dims plan below
    d1 = torch.empty(65536, device=dev)
    rec("C5a dims=1 4096x65536", 4 * 2**28 + 4 * 65536, lambda: kf.mapreduce_(kf.identity, "+", d1, A1, dims=1, tmp=t5))
    A2 = t.as_strided((65536, 4096), (1, 65536))
    d2 = torch.empty(65536, device=dev)
    rec("C5b dims=2 65536x4096", 4 * 2**28 + 4 * 65536, lambda: kf.mapreduce_(kf.identity, "+", d2, A2, dims=2, tmp=t5))
    V1 = A1[:, ::2]
    d1v = torch.empty(32768, device=dev)
    rec("C5c dims=1 view 4096x(65536/2)", 4 * 2**27 + 4 * 32768,
        lambda: kf.mapreduce_(kf.identity, "+", d1v, V1, dims=1, tmp=t5))
    V2 = A2[:, ::2]
    rec("C5d dims=2 view 65536x(4096/2)", 4 * 2**27 + 4 * 65536,
        lambda: kf.mapreduce_(kf.identity, "+", d2, V2, dims=2, tmp=t5))
    # beyond the BASELINE configs: vector operands and layouts off the vector path
    import operator
    xv = torch.rand(4096, device=dev, generator=g)
    rec("X1 matvec 65536x4096 F32", 4 * 2**28 + 8 * 65536 + 4 * 4096,
        lambda: kf.matvec_(operator.mul, "+", d2, A2, xv, tmp=t5))
    xr = torch.rand(4096, device=dev, generator=g)
    rec("X2 vecmat 4096x65536 F32", 4 * 2**28 + 8 * 65536,
        lambda: kf.vecmat_(operator.mul, "+", d1, xr, A1, tmp=t5))
    xs = torch.rand(2**28, device=dev, generator=g)
    ys = torch.empty_like(xs)
    ts = tmp_for(kf.Scan1D, xs)
    of1 = torch.empty(1, device=dev)
    t3s = tmp_for(kf.MapReduce1D, xs)
    rec("X3 scan F32 unaligned view x[1:] n=2^28-1", 8 * (2**28 - 1), lambda: kf.scan_("+", ys[1:], xs[1:], tmp=ts))
    rec("X4 mapreduce F32 unaligned view x[1:]", 4 * (2**28 - 1),
        lambda: kf.mapreduce_(kf.identity, "+", of1, xs[1:], tmp=t3s))
    del xs, ys
    xd = torch.rand(2**27, device=dev, generator=g, dtype=torch.float64)
    yd = torch.empty_like(xd)
    td = tmp_for(kf.Scan1D, xd)
    rec("X5 scan F64 incl n=2^27", 16 * 2**27, lambda: kf.scan_("+", yd, xd, tmp=td))
    del xd, yd
    xb = torch.randint(0, 255, (2**30,), device=dev, generator=g, dtype=torch.uint8)
    yb = torch.empty_like(xb)
    tb = tmp_for(kf.Scan1D, xb)
    rec("X6 scan UInt8 incl n=2^30", 2 * 2**30, lambda: kf.scan_("+", yb, xb, tmp=tb))
    del xb, yb
    for n, label in ((10**5, "10^5"), (2**21, "2^21"), (2**23, "2^23")):
        xs = torch.rand(n, device=dev, generator=g)
        ys = torch.empty_like(xs)
        ts = tmp_for(kf.Scan1D, xs)
        rec(f"X7 scan F32 incl n={label}", 8 * n, lambda: kf.scan_("+", ys, xs, tmp=ts))
    if json_path:
        os.makedirs(os.path.dirname(os.path.abspath(json_path)), exist_ok=True)
        with open(json_path, "w") as fh:
            json.dump({"copy_ceiling_gbps": ceiling, "rows": rows}, fh, indent=1)
    return rows


if __name__ == "__main__":
    main()
