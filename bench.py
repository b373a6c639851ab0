"""Throughput of the scan! / mapreduce hot path on one MI355X.

A step is one pass of the path over one batch of synthetic Float32 data at
n = 2^28 (BASELINE.json's headline configuration):
    scan!(+, dst, src)                 inclusive, 2*4*n bytes
    mapreduce!(identity, +, out, src)  full reduction, 4*n bytes
Inputs are resident in HBM before timing starts. `value` is algorithmic GB/s
of the whole step (12*n bytes / step time). The JSON line also carries the
per-kernel roofline of the dominant kernel (the scan), measured with HIP
events on the stream the kernels run on, the measured copy and read
ceilings (kf_bw_probe kernels and hipMemcpyDtoD), and the CPU baseline (the
oracle's restatement of Base.accumulate! / Base.mapreduce, timed on this
host).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--all [--all-json PATH]]
  --all          also time every BASELINE.json configuration (stderr table,
                 and the rows inside the JSON line as "all_configs")
  --all-json     also write those rows, with the ceilings, to PATH
  --sweep        the reference's 10^6..10^9 size sweep
  --sweep-2d     the reference's matvec / vecmat shape sweep (n*p = 10^7..10^9)
  --timeline [large|mid|reduce]  only the per-tile phases of the scan, or the
                 per-workgroup phases of the full reduction (instrumented library)
  --pmc-run      only the marked dispatch sequence of every configuration,
                 for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs
  --pmc-summary  FETCH_DIR WRITE_DIR CASES_LOG OUT_JSON: per-configuration
                 HBM bytes from those two runs (no GPU)
  --trace-summary TRACE_DIR BENCH_JSON OUT_MD: per-row kernel tables of a
                 rocprofv3 --kernel-trace run of --all / --sweep (no GPU)
"""
import argparse
import json
import os
import statistics
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
    """HBM bytes per launch of the headline scan (row H1 of the per-config
    rocprofv3 --pmc summary: FETCH_SIZE + WRITE_SIZE, scaled by the
    copy-kernel calibration), if recorded."""
    p = os.path.join(REPO, "profiles", "traffic_all_configs.json")
    if os.path.exists(p):
        with open(p) as fh:
            h = json.load(fh)["configs"].get("H1")
        if h:
            return int(round((h["fetch_bytes"] + h["write_bytes"]) / h["dispatches_per_call"]))
    return None


def load_config_traffic():
    """{config key: HBM bytes / algorithmic bytes} per BASELINE configuration,
    from the rocprofv3 --pmc summary in profiles/, if recorded."""
    p = os.path.join(REPO, "profiles", "traffic_all_configs.json")
    if os.path.exists(p):
        with open(p) as fh:
            return {k: v["ratio"] for k, v in json.load(fh)["configs"].items()}
    return {}


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
    ap.add_argument("--sweep-2d", action="store_true",
                    help="the reference's matvec/vecmat shape sweep (perfs/julia/benchmarks)")
    ap.add_argument("--timeline", nargs="?", const="large", choices=("large", "mid", "quat", "reduce"),
                    help="only the per-tile scan timeline (libkfhip_timeline.so): the large "
                         "scans (default), the mid sizes of the reference's sweep, the "
                         "quaternion scans, or the reductions' per-workgroup timeline")
    ap.add_argument("--pmc-run", action="store_true",
                    help="only the dispatch sequence for rocprofv3 --pmc (see pmc_run)")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "CASES_LOG", "OUT_JSON"),
                    help="summarise two --pmc-run profiles (FETCH_SIZE, WRITE_SIZE); no GPU needed")
    ap.add_argument("--trace-summary", nargs=3, metavar=("TRACE_DIR", "BENCH_JSON", "OUT_MD"),
                    help="per-row kernel tables from a rocprofv3 --kernel-trace run of --all/--sweep; no GPU needed")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(*args.trace_summary)
        return
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the scan/mapreduce path here is single-GPU "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__
    kf = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.pmc_run:
        pmc_run(kf, dev)
        return
    if args.timeline == "reduce":
        print(json.dumps({"reduce_timeline": reduce_timeline(dev)}), flush=True)
        return
    if args.timeline:
        cases = {"large": TIMELINE_CASES, "mid": MID_TIMELINE_CASES, "quat": QUAT_TIMELINE_CASES}[args.timeline]
        print(json.dumps({"scan_timeline": scan_timeline(dev, cases)}), flush=True)
        return

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
    ceil = measure_ceilings(kf, dev, src)
    copy_ceiling, read_ceiling = ceil["copy_ceiling_gbps"], ceil["read_ceiling_gbps"]
    scan_gbps = 8 * N / scan_s / 1e9
    red_gbps = 4 * N / red_s / 1e9
    log(f"scan {scan_s*1e6:.1f} us {scan_gbps:.0f} GB/s ({scan_gbps/copy_ceiling*100:.1f}% of copy ceiling) | "
        f"reduce {red_s*1e6:.1f} us {red_gbps:.0f} GB/s ({red_gbps/read_ceiling*100:.1f}% of read ceiling)")
    log("ceilings: " + ", ".join(f"{k} {v:.0f}" for k, v in ceil.items()))

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
            "scan_gbps": round(scan_gbps, 1), "scan_frac_of_copy_ceiling": round(scan_gbps / copy_ceiling, 4),
            "scan_frac_of_rw_bound": round(scan_gbps / ceil["rw_bound_gbps"], 4),
            "mapreduce_gbps": round(red_gbps, 1), "mapreduce_frac_of_read_ceiling": round(red_gbps / read_ceiling, 4),
            "mapreduce_frac_of_peak": round(red_gbps / PEAK_HBM_GBPS, 4), "mapreduce_avg_launch_us": round(red_s * 1e6, 2),
            "scan_gbps_best_batch": round(8 * N / scan_min / 1e9, 1),
            "mapreduce_gbps_best_batch": round(4 * N / red_min / 1e9, 1),
            **{k: round(v, 1) for k, v in ceil.items()},
        },
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 4),
    }
    if args.all:
        line["all_configs"] = bench_all(kf, dev, ceil, args.all_json, cpu=not args.no_cpu)
    if args.sweep:
        line["sweep"] = bench_sweep(kf, dev, ceil)
    if args.sweep_2d:
        line["sweep_2d"] = bench_sweep_2d(kf, dev, ceil)
    print(json.dumps(line), flush=True)


_MARKER = {}


def _mark(kf, dev, begin):
    """Marker fills around each measured row, so that a kernel trace can be
    split by row: begin = a 16-byte kf_fill (one fill_kernel workgroup of
    256 lanes), end = a 4-byte one (one fill_elems_kernel workgroup of 64)."""
    t = _MARKER.get(dev)
    if t is None:
        t = _MARKER[dev] = torch.zeros(4, dtype=torch.int32, device=dev)
    kf.setvalue_(t if begin else t[:1], 1 if begin else 2)


def measure_ceilings(kf, dev, src):
    """Copy and read ceilings on the same 1 GiB buffer (2^28 Float32): GB/s
    of algorithmic bytes (copy 2 x bytes, read 1 x bytes) of every
    kf_bw_probe kernel and of torch's device-to-device copy
    (hipMemcpyDtoD); each ceiling is the best of its kind. This plays the
    part of the reference's vendor memcpy benchmark
    (perfs/cuda_cpp/cub_nvcc/cub_memcpy_benchmark.cu, bytes = 2N)."""
    import ctypes
    L, K = kf._lib.lib(), kf._lib
    nbytes = src.numel() * src.element_size()
    cbuf = torch.empty_like(src)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    scratch = torch.empty(L.kf_bw_probe_scratch_bytes(nbytes), dtype=torch.uint8, device=dev)

    def probe(kind, dst):
        def fn():
            rc = L.kf_bw_probe(kind, ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()), nbytes,
                               ctypes.c_void_p(scratch.data_ptr()), scratch.numel(),
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            K.check(rc, "kf_bw_probe")
        return fn

    out = {}
    for name, kind in (("copy_kernel_gbps", K.BW_COPY), ("copy_tiled_gbps", K.BW_COPY_TILED),
                       ("copy_ordered_gbps", K.BW_COPY_ORDERED)):
        out[name] = 2 * nbytes / time_calls(probe(kind, cbuf), 20) / 1e9
    out["hipMemcpyDtoD_gbps"] = 2 * nbytes / time_calls(lambda: cbuf.copy_(src), 20) / 1e9
    torch.cuda.synchronize()
    assert torch.equal(cbuf, src), "copy probe mismatch"
    for name, kind in (("read_kernel_gbps", K.BW_READ), ("read_tiled_gbps", K.BW_READ_TILED)):
        out[name] = nbytes / time_calls(probe(kind, sink), 20) / 1e9
    # write-only: kf_fill of the same 1 GiB (nontemporal 16-byte stores) and
    # the write probe (plain 16-byte stores, the faster of the two)
    val = ctypes.create_string_buffer(b"\0" * 4, 4)

    def fill():
        K.check(L.kf_fill(ctypes.c_void_p(cbuf.data_ptr()), cbuf.numel(), ctypes.cast(val, ctypes.c_void_p), 4,
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "kf_fill")
    out["write_fill_gbps"] = nbytes / time_calls(fill, 20) / 1e9
    out["write_kernel_gbps"] = nbytes / time_calls(probe(K.BW_WRITE, cbuf), 20) / 1e9
    out["copy_ceiling_gbps"] = max(out[k] for k in ("copy_kernel_gbps", "copy_tiled_gbps", "copy_ordered_gbps",
                                                    "hipMemcpyDtoD_gbps"))
    out["read_ceiling_gbps"] = max(out["read_kernel_gbps"], out["read_tiled_gbps"])
    # a copy cannot beat reading its bytes at the best read rate and writing
    # them at the write rate one after the other: bytes/R_read + bytes/R_write
    out["write_ceiling_gbps"] = max(out["write_kernel_gbps"], out["write_fill_gbps"])
    out["rw_bound_gbps"] = 2.0 / (1.0 / out["read_ceiling_gbps"] + 1.0 / out["write_ceiling_gbps"])
    del cbuf, scratch
    return out


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


def bench_sweep(kf, dev, ceil):
    """The reference's own size sweep (perfs/julia/benchmarks/
    scan_perf_comparison.jl:129-131, mapreduce_perf_comparison.jl:121-122):
    n in 10^6..10^9 for Float32, Float64 and UInt8, scan!(+) inclusive and
    mapreduce(identity, +). HIP-graph timed; GB/s of algorithmic bytes, as a
    fraction of the 1 GiB ceiling of its kind and of a same-size copy (the
    best of kf_bw_probe's copies over the scan's bytes) or read (the best
    read probe over the reduction's bytes): below ~100 MB launch latency and
    the first tiles' ramp bound copies too."""
    import ctypes
    L, K = kf._lib.lib(), kf._lib
    rows = []
    g = torch.Generator(device=dev).manual_seed(20261201)

    def probe_us(kinds, nbytes, dst, src, scratch):
        best = None
        for kind in kinds:
            def fn():
                K.check(L.kf_bw_probe(kind, ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()), nbytes,
                                      ctypes.c_void_p(scratch.data_ptr()), scratch.numel(),
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "kf_bw_probe")
            t = _graph_time(fn, reps=20 if nbytes < 10**9 else 5) if kind != K.BW_COPY_ORDERED else \
                time_calls(fn, 20)  # the ordered copy takes its epoch from a host counter: no graph
            best = t if best is None else min(best, t)
        return best

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
            nb = n * es // 16 * 16
            pscr = torch.empty(L.kf_bw_probe_scratch_bytes(nb), dtype=torch.uint8, device=dev)
            sink = torch.zeros(4, dtype=torch.int32, device=dev)
            same = {"scan": probe_us((K.BW_COPY, K.BW_COPY_ORDERED), nb, y, x, pscr),
                    "mapreduce": probe_us((K.BW_READ, K.BW_READ_TILED), nb, sink, x, pscr)}
            for what, bytes_, fn in (
                    ("scan", 2 * es * n, lambda: kf.scan_("+", y, x, tmp=ts)),
                    ("mapreduce", es * n, lambda: kf.mapreduce_(kf.identity, "+", o, x, tmp=tr))):
                _mark(kf, dev, True)
                sec = _graph_time(fn, reps=20 if n < 10**9 else 5)
                _mark(kf, dev, False)
                gb = bytes_ / sec / 1e9
                c = ceil["copy_ceiling_gbps"] if what == "scan" else ceil["read_ceiling_gbps"]
                rows.append({"op": what, "n": n, "dtype": str(dt).replace("torch.", ""),
                             "us": round(sec * 1e6, 2), "gbps": round(gb, 1),
                             "elems_per_s": round(n / sec, 1), "frac_ceiling": round(gb / c, 4),
                             "same_size_probe_us": round(same[what] * 1e6, 2),
                             "frac_same_size": round(same[what] / sec, 4)})
                log(f"  {what:9s} {str(dt):14s} n={n:>10d} {sec*1e6:10.1f} us {gb:8.0f} GB/s "
                    f"{gb/c*100:5.1f}% of the {'copy' if what == 'scan' else 'read'} ceiling, "
                    f"same-size {'copy' if what == 'scan' else 'read'} {same[what]*1e6:.1f} us "
                    f"({same[what]/sec*100:.0f}%)")
            del x, y, ts, tr, pscr
    return rows


def bench_sweep_2d(kf, dev, ceil):
    """The reference's matvec / vecmat sweeps (perfs/julia/benchmarks/
    matvec_perf_comparison.jl:77-88, vecmat_perf_comparison.jl:59-70): n x p
    column-major matrices of n*p in {10^7, 10^8, 10^9} elements, n = 10^k
    (k = 0..log10(total), 1..log10(total)-1 at 10^9), Float32, Float64 and
    UInt8; matvec!(*, +, y, A, x) (y[i] = sum_j A[i,j] x[j]) and
    vecmat!(*, +, y, x, A) (y[j] = sum_i x[i] A[i,j]). HIP-graph timed; GB/s
    of algorithmic bytes (A, x and y once each), as a fraction of the read
    ceiling and of a same-size read (the best read probe over A's bytes)."""
    import ctypes
    import operator
    L, K = kf._lib.lib(), kf._lib
    rows = []
    g = torch.Generator(device=dev).manual_seed(20261201)
    tmp = kf.KernelBuffer(kf.MapReduce2D, 64 << 20, dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    for total in (10**7, 10**8, 10**9):
        top = round(np.log10(total))
        ks = range(0, top + 1) if total <= 10**8 else range(1, top)
        for dt in (torch.float32, torch.float64, torch.uint8):
            es = torch.empty(0, dtype=dt).element_size()
            flat = (torch.randint(0, 4, (total,), device=dev, generator=g, dtype=dt) if dt == torch.uint8
                    else torch.rand(total, device=dev, generator=g, dtype=dt))
            nb = total * es // 16 * 16
            pscr = torch.empty(L.kf_bw_probe_scratch_bytes(nb), dtype=torch.uint8, device=dev)
            same = None
            for kind in (K.BW_READ, K.BW_READ_TILED):
                def fn():
                    K.check(L.kf_bw_probe(kind, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(flat.data_ptr()), nb,
                                          ctypes.c_void_p(pscr.data_ptr()), pscr.numel(),
                                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "kf_bw_probe")
                t = _graph_time(fn, reps=20 if nb < 10**9 else 5)
                same = t if same is None else min(same, t)
            for k in ks:
                n = 10**k
                p = total // n
                A = flat[:n * p].as_strided((n, p), (1, n))
                xr = torch.ones(p, device=dev, dtype=dt)
                xc = torch.ones(n, device=dev, dtype=dt)
                yr = torch.empty(n, device=dev, dtype=dt)
                yc = torch.empty(p, device=dev, dtype=dt)
                for what, bytes_, fn in (
                        ("matvec", es * (n * p + p + n), lambda: kf.matvec_(operator.mul, "+", yr, A, xr, tmp=tmp)),
                        ("vecmat", es * (n * p + n + p), lambda: kf.vecmat_(operator.mul, "+", yc, xc, A, tmp=tmp))):
                    _mark(kf, dev, True)
                    sec = _graph_time(fn, reps=20 if total < 10**9 else 5)
                    _mark(kf, dev, False)
                    gb = bytes_ / sec / 1e9
                    c = ceil["read_ceiling_gbps"]
                    rows.append({"op": what, "total": total, "n": n, "p": p, "dtype": str(dt).replace("torch.", ""),
                                 "us": round(sec * 1e6, 2), "gbps": round(gb, 1), "frac_ceiling": round(gb / c, 4),
                                 "same_size_read_us": round(same * 1e6, 2), "frac_same_size": round(same / sec, 4)})
                    log(f"  {what} {str(dt):14s} n={n:>10d} p={p:>10d} {sec*1e6:10.1f} us {gb:8.0f} GB/s "
                        f"{gb/c*100:5.1f}% of the read ceiling, same-size read {same*1e6:.1f} us "
                        f"({same/sec*100:.0f}%)")
                del A, xr, xc, yr, yc
            del flat, pscr
    return rows


_HOST = {}
_HOST_USED = set()


def _host(t, out=False):
    """Host (numpy) copy of a device tensor's storage span, cached by
    tensor, or an uninitialised host array of its size for outputs."""
    key = (t.data_ptr(), t.numel(), t.dtype, out)
    _HOST_USED.add(key)
    if key not in _HOST:
        if out:
            _HOST[key] = np.empty(tuple(t.shape), dtype=torch.empty(0, dtype=t.dtype).numpy().dtype)
        else:
            _HOST[key] = t.contiguous().cpu().numpy()
    return _HOST[key]


def _cpu_prep(make):
    """The CPU baseline of one configuration: prep() copies its inputs
    (the same seeded data the GPU row used) to the host and returns
    run(threads), one call of the oracle's restatement of the reference's
    CPU path (Base.accumulate! / Base.mapreduce, or their chunked
    Threads.@threads variant)."""
    def prep():
        from oracle import oracle
        return make(oracle, _host)
    return prep


def config_cases(kf, dev):
    """(key, name, algorithmic bytes, fn, reps, elements, cpu prep or None)
    for every BASELINE.json configuration (C1-C5) and the extra rows
    (X1-X10); each case's inputs are alive until the next case is
    requested."""
    import operator
    g = torch.Generator(device=dev).manual_seed(20261201)

    def tmp_for(kind, src):
        return kf.get_allocation(kind, kf.identity, "+", src)

    # the bench step's two calls (Float32 n=2^28), for their counters
    xh = torch.rand(2**28, device=dev, generator=g)
    yh = torch.empty_like(xh)
    oh = torch.empty(1, device=dev)
    th, trh = tmp_for(kf.Scan1D, xh), tmp_for(kf.MapReduce1D, xh)
    yield "H1", "H1 scan F32 incl n=2^28 (bench step)", 8 * 2**28, lambda: kf.scan_("+", yh, xh, tmp=th), 20, \
        2**28, _cpu_prep(lambda o, h: (lambda t: o.baseline_scan_add_f32(h(xh), h(yh, True), t)))
    yield "H2", "H2 mapreduce F32 n=2^28 (bench step)", 4 * 2**28, \
        lambda: kf.mapreduce_(kf.identity, "+", oh, xh, tmp=trh), 20, \
        2**28, _cpu_prep(lambda o, h: (lambda t: o.baseline_sum_f32(h(xh), t)))
    del xh, yh
    x = torch.rand(10**6, device=dev, generator=g)
    y = torch.empty_like(x)
    t1 = tmp_for(kf.Scan1D, x)
    yield "C1", "C1 scan F32 incl n=1e6", 8e6, lambda: kf.scan_("+", y, x, tmp=t1), 20, \
        10**6, _cpu_prep(lambda o, h: (lambda t: o.baseline_scan_add_f32(h(x), h(y, True), t)))
    del x, y
    xi = torch.randint(0, 16, (2**28,), device=dev, generator=g, dtype=torch.int32)
    yi = torch.empty_like(xi)
    t2 = tmp_for(kf.Scan1D, xi)
    yield "C2i", "C2 scan Int32 incl n=2^28", 8 * 2**28, lambda: kf.scan_("+", yi, xi, tmp=t2), 20, \
        2**28, _cpu_prep(lambda o, h: (lambda t: o.baseline_scan_add_i32(h(xi), h(yi, True), False, t)))
    yield "C2e", "C2 scan Int32 excl n=2^28", 8 * 2**28, lambda: kf.scan_("+", yi, xi, exclusive=True, tmp=t2), 20, \
        2**28, _cpu_prep(lambda o, h: (lambda t: o.baseline_scan_add_i32(h(xi), h(yi, True), True, t)))
    o = torch.empty(1, device=dev, dtype=torch.int32)
    xr = torch.randint(-2**31, 2**31 - 1, (2**28,), device=dev, generator=g, dtype=torch.int32)
    t3 = tmp_for(kf.MapReduce1D, xr)
    yield "C3c", "C3c mapreduce max Int32 n=2^28", 4 * 2**28, lambda: kf.mapreduce_(kf.identity, max, o, xr, tmp=t3), 20, \
        2**28, _cpu_prep(lambda o_, h: (lambda t: o_.baseline_max_i32(h(xr), t)))
    del xi, yi, xr
    xf = torch.randn(2**30, device=dev, generator=g)
    of = torch.empty(1, device=dev)
    t3f = tmp_for(kf.MapReduce1D, xf)
    yield "C3a", "C3a mapreduce abs2,+ F32 n=2^30", 4 * 2**30, lambda: kf.mapreduce_(kf.abs2, "+", of, xf, tmp=t3f), 10, \
        2**30, _cpu_prep(lambda o, h: (lambda t: o.baseline_sum_abs2(h(xf), t)))
    del xf
    xd = torch.randn(2**28, device=dev, generator=g, dtype=torch.float64)
    od = torch.empty(1, device=dev, dtype=torch.float64)
    t3d = tmp_for(kf.MapReduce1D, xd)
    yield "C3b", "C3b mapreduce abs2,+ F64 n=2^28", 8 * 2**28, lambda: kf.mapreduce_(kf.abs2, "+", od, xd, tmp=t3d), 20, \
        2**28, _cpu_prep(lambda o, h: (lambda t: o.baseline_sum_abs2(h(xd), t)))
    del xd
    ab = torch.empty(2**26, 2, device=dev)
    ab[:, 0].uniform_(0.9, 1.0, generator=g)
    ab[:, 1].normal_(generator=g)
    yab = torch.empty_like(ab)
    t4 = kf.get_allocation(kf.Scan1D, kf.identity, kf.affine, ab)
    yield "C4", "C4 affine scan n=2^26", 16 * 2**26, lambda: kf.scan_(kf.affine, yab, ab, tmp=t4), 20, \
        2**26, _cpu_prep(lambda o, h: (lambda t: o.baseline_scan_affine_f32(h(ab), h(yab, True), t)))
    del ab, yab
    t = torch.rand(2**28, device=dev, generator=g) * 2 - 1
    A1 = t.as_strided((4096, 65536), (1, 4096))
    t5 = kf.KernelBuffer(kf.MapReduce2D, 64 << 20, dev)  # >= every dims plan below
    d1 = torch.empty(65536, device=dev)
    yield "C5a", "C5a dims=1 4096x65536", 4 * 2**28 + 4 * 65536, \
        lambda: kf.mapreduce_(kf.identity, "+", d1, A1, dims=1, tmp=t5), 20, \
        2**28, _cpu_prep(lambda o, h: (lambda th: o.baseline_sum_dims_f32(h(t), 4096, 65536, 4096, 1, h(d1, True), th)))
    A2 = t.as_strided((65536, 4096), (1, 65536))
    d2 = torch.empty(65536, device=dev)
    yield "C5b", "C5b dims=2 65536x4096", 4 * 2**28 + 4 * 65536, \
        lambda: kf.mapreduce_(kf.identity, "+", d2, A2, dims=2, tmp=t5), 20, \
        2**28, _cpu_prep(lambda o, h: (lambda th: o.baseline_sum_dims_f32(h(t), 65536, 4096, 65536, 2, h(d2, True), th)))
    V1 = A1[:, ::2]
    d1v = torch.empty(32768, device=dev)
    yield "C5c", "C5c dims=1 view 4096x(65536/2)", 4 * 2**27 + 4 * 32768, \
        lambda: kf.mapreduce_(kf.identity, "+", d1v, V1, dims=1, tmp=t5), 20, \
        2**27, _cpu_prep(lambda o, h: (lambda th: o.baseline_sum_dims_f32(h(t), 4096, 32768, 8192, 1, h(d1v, True), th)))
    V2 = A2[:, ::2]
    yield "C5d", "C5d dims=2 view 65536x(4096/2)", 4 * 2**27 + 4 * 65536, \
        lambda: kf.mapreduce_(kf.identity, "+", d2, V2, dims=2, tmp=t5), 20, \
        2**27, _cpu_prep(lambda o, h: (lambda th: o.baseline_sum_dims_f32(h(t), 65536, 2048, 131072, 2, h(d2, True), th)))
    # beyond the BASELINE configs: vector operands and layouts off the vector path
    xv = torch.rand(4096, device=dev, generator=g)
    yield "X1", "X1 matvec 65536x4096 F32", 4 * 2**28 + 8 * 65536 + 4 * 4096, \
        lambda: kf.matvec_(operator.mul, "+", d2, A2, xv, tmp=t5), 20, 2**28, None
    xr = torch.rand(4096, device=dev, generator=g)
    yield "X2", "X2 vecmat 4096x65536 F32", 4 * 2**28 + 8 * 65536, \
        lambda: kf.vecmat_(operator.mul, "+", d1, xr, A1, tmp=t5), 20, 2**28, None
    del t, A1, A2, V1, V2
    xs = torch.rand(2**28, device=dev, generator=g)
    ys = torch.empty_like(xs)
    ts = tmp_for(kf.Scan1D, xs)
    of1 = torch.empty(1, device=dev)
    t3s = tmp_for(kf.MapReduce1D, xs)
    yield "X3", "X3 scan F32 unaligned view x[1:] n=2^28-1", 8 * (2**28 - 1), \
        lambda: kf.scan_("+", ys[1:], xs[1:], tmp=ts), 20, 2**28 - 1, None
    yield "X8", "X8 scan F32 x[1:] -> aligned dst n=2^28-1", 8 * (2**28 - 1), \
        lambda: kf.scan_("+", ys[:-1], xs[1:], tmp=ts), 20, 2**28 - 1, None
    yield "X4", "X4 mapreduce F32 unaligned view x[1:]", 4 * (2**28 - 1), \
        lambda: kf.mapreduce_(kf.identity, "+", of1, xs[1:], tmp=t3s), 20, 2**28 - 1, None
    del xs, ys
    xd = torch.rand(2**27, device=dev, generator=g, dtype=torch.float64)
    yd = torch.empty_like(xd)
    td = tmp_for(kf.Scan1D, xd)
    yield "X5", "X5 scan F64 incl n=2^27", 16 * 2**27, lambda: kf.scan_("+", yd, xd, tmp=td), 20, 2**27, None
    del xd, yd
    xb = torch.randint(0, 255, (2**30,), device=dev, generator=g, dtype=torch.uint8)
    yb = torch.empty_like(xb)
    tb = tmp_for(kf.Scan1D, xb)
    yield "X6", "X6 scan UInt8 incl n=2^30", 2 * 2**30, lambda: kf.scan_("+", yb, xb, tmp=tb), 20, 2**30, None
    del xb, yb
    for n, label in ((10**5, "10^5"), (2**21, "2^21"), (2**23, "2^23")):
        xs = torch.rand(n, device=dev, generator=g)
        ys = torch.empty_like(xs)
        ts = tmp_for(kf.Scan1D, xs)
        yield f"X7-{label}", f"X7 scan F32 incl n={label}", 8 * n, lambda: kf.scan_("+", ys, xs, tmp=ts), 20, n, None
    # the reference's non-commutative test case (test/tests/scan/scan_test.jl:22-33):
    # QuaternionF64 at its n = 10^6 and 2^24, QuaternionF32 at 2^26, Hamilton products
    for key, n, dt, label in (("X9-QuaternionF64", 10**6, torch.float64, "QuaternionF64 n=10^6"),
                              ("X9-QuaternionF64-2^24", 2**24, torch.float64, "QuaternionF64 n=2^24"),
                              ("X9-QuaternionF32", 2**26, torch.float32, "QuaternionF32 n=2^26")):
        q = torch.randn(n, 4, device=dev, generator=g, dtype=dt)
        q = q / q.norm(dim=1, keepdim=True)
        yq = torch.empty_like(q)
        tq = kf.get_allocation(kf.Scan1D, kf.identity, "*", q)
        yield key, f"X9 scan {label}", 2 * q.numel() * q.element_size(), \
            lambda: kf.scan_("*", yq, q, tmp=tq), 20, n, None
        del q, yq
    # multi-array reductions (mapreduce1d!(f, op, dst, (x, y[, z]))): the dot
    # product and the reference's three-array sum(a .* b .* c)
    import operator
    xs = [torch.rand(2**28, device=dev, generator=g) for _ in range(3)]
    om = torch.empty(1, device=dev)
    tm = kf.get_allocation(kf.MapReduce1D, kf.prod3, "+", tuple(xs))
    yield "X10-dot", "X10 mapreduce(*, +, x, y) F32 n=2^28", 8 * 2**28, \
        lambda: kf.mapreduce1d_(operator.mul, "+", om, (xs[0], xs[1]), tmp=tm), 10, 2**28, None
    yield "X10-xyz", "X10 mapreduce(a*b*c, +, a, b, c) F32 n=2^28", 12 * 2**28, \
        lambda: kf.mapreduce1d_(kf.prod3, "+", om, tuple(xs), tmp=tm), 10, 2**28, None
    del xs


def _cpu_seconds(run, budget_s):
    """Seconds per call of run(): one untimed call (page faults of the
    output), then calls until budget_s has passed (at least one)."""
    run()
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 200:
            return el / reps, reps


def cpu_row(cpu_prep, bytes_, elems, threads, budget_s=1.0):
    """The reference's CPU path for one configuration on this host, on the
    GPU row's own data: `threads` OpenMP threads (chunked) and one thread
    (sequential), each timed over about budget_s of calls."""
    _HOST_USED.clear()
    run = cpu_prep()
    tm, nm = _cpu_seconds(lambda: run(threads), budget_s)
    t1, n1 = _cpu_seconds(lambda: run(1), budget_s)
    for k in [k for k in _HOST if k not in _HOST_USED]:  # keep only this case's host copies
        del _HOST[k]
    return {"kind": "port", "threads": threads, "gbps": round(bytes_ / tm / 1e9, 3),
            "gelems_per_s": round(elems / tm / 1e9, 4), "ms": round(tm * 1e3, 3), "calls": nm,
            "single_thread_gbps": round(bytes_ / t1 / 1e9, 3), "single_thread_gelems_per_s": round(elems / t1 / 1e9, 4),
            "single_thread_ms": round(t1 * 1e3, 3), "single_thread_calls": n1}


def bench_all(kf, dev, ceil, json_path=None, cpu=True):
    """Every configuration of config_cases: GB/s, % of peak, % of the ceiling
    of its kind (scans: the copy ceiling; reductions: the read ceiling), and
    the HBM traffic ratio recorded by rocprofv3 --pmc when profiles/ holds it."""
    rows = []
    traffic = load_config_traffic()
    threads = max(1, min(16, os.cpu_count() or 1))
    for key, name, bytes_, fn, reps, elems, cpu_prep in config_cases(kf, dev):
        # captured in a HIP graph so that host launch overhead does not hide
        # the kernel time of the small configurations
        _mark(kf, dev, True)
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        # replayed for 250 ms before it is timed: in the kernel trace of this
        # loop the 4 GiB reduction (C3a) ran at 636 us per call for its first
        # 90 ms and at 606 us from one call to the next after that, on the same
        # buffer; alone in a process it runs at 608 us from its first call.
        # The step is a device transient, not a property of the kernel, so
        # each row is timed in the steady state, as the median of five replays.
        t_end = time.perf_counter() + 0.25
        while time.perf_counter() < t_end:
            graph.replay()
            torch.cuda.synchronize()
        s = statistics.median(time_calls(graph.replay, 1) for _ in range(5)) / reps
        _mark(kf, dev, False)
        del graph
        gb = bytes_ / s / 1e9
        kind = "copy" if " scan " in f" {name} " else "read"
        c = ceil[f"{kind}_ceiling_gbps"]
        row = {"config": name, "us": round(s * 1e6, 2), "gbps": round(gb, 1),
               "gelems_per_s": round(elems / s / 1e9, 3),
               "frac_peak": round(gb / PEAK_HBM_GBPS, 4), "ceiling": kind, "frac_ceiling": round(gb / c, 4),
               "hbm_traffic_ratio": traffic.get(key)}
        if kind == "copy":
            row["frac_rw_bound"] = round(gb / ceil["rw_bound_gbps"], 4)
        if cpu and cpu_prep is not None:
            row["cpu"] = cpu_row(cpu_prep, bytes_, elems, threads)
        rows.append(row)
        log(f"  {name:48s} {s*1e6:10.1f} us {gb:8.0f} GB/s {elems / s / 1e9:8.2f} Gelem/s "
            f"{gb/c*100:5.1f}% of {kind} ceiling"
            + (f"  traffic {row['hbm_traffic_ratio']:.4f}x" if row["hbm_traffic_ratio"] else "")
            + (f"  | CPU {row['cpu']['threads']} thr {row['cpu']['gbps']:.1f} GB/s, 1 thr "
               f"{row['cpu']['single_thread_gbps']:.1f} GB/s" if "cpu" in row else ""))
    _HOST.clear()
    if json_path:
        os.makedirs(os.path.dirname(os.path.abspath(json_path)), exist_ok=True)
        with open(json_path, "w") as fh:
            json.dump({"ceilings": ceil, "rows": rows}, fh, indent=1)
    return rows


# ---------------------------------------------------------------------------
# Per-tile timeline of the scan (libkfhip_timeline.so, built with KF_TIMELINE)
# ---------------------------------------------------------------------------
TIMELINE_CASES = (("C4 affine n=2^26", 5, 2**26), ("affine n=2^27", 5, 2**27), ("affine n=2^28", 5, 2**28),
                  ("Float64 n=2^26", 1, 2**26), ("Float64 n=2^27", 1, 2**27), ("Float32 n=2^28", 0, 2**28))
# Mid sizes: UInt8 and Float32 at equal bytes, from one generation of
# resident tiles to many.
MID_TIMELINE_CASES = (("Float32 n=10^6 (C1)", 0, 10**6), ("UInt8 n=10^7", 4, 10**7), ("UInt8 n=10^8", 4, 10**8), ("UInt8 n=3*10^8", 4, 3 * 10**8),
                      ("UInt8 n=2^30", 4, 2**30), ("Float32 n=2.5*10^6", 0, 25 * 10**5),
                      ("Float32 n=2.5*10^7", 0, 25 * 10**6), ("Float32 n=10^8", 0, 10**8),
                      ("Float64 n=10^7", 1, 10**7))
# Quaternion products (unit quaternions): the reference's test size and the
# large arrays of the wide tiles.
QUAT_TIMELINE_CASES = (("QuaternionF64 n=10^6", 7, 10**6), ("QuaternionF64 n=2^24", 7, 2**24),
                       ("QuaternionF32 n=2^24", 6, 2**24), ("QuaternionF32 n=2^26", 6, 2**26))


def scan_timeline(dev, cases=TIMELINE_CASES):
    """Per-tile phases of the decoupled-lookback scan from the instrumented
    library: each tile's thread 0 stamps the 100 MHz realtime counter at its
    start, once its tile is scanned (loads done), once its prefix is known
    (lookback done) and once its stores are issued. Per case: kernel time
    (events, uninstrumented calls of the same library), tile phases
    (medians), peak resident tiles, the steady-state bandwidth (bytes of the
    tiles that finish between full residency and the last tile's start,
    over that window) and the drain (last tile start to kernel end)."""
    import ctypes
    path = os.path.join(REPO, "kernelforge.jl_amd", "libkfhip_timeline.so")
    L = ctypes.CDLL(path)
    P, I, I64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    L.kf_scan.argtypes = [I, I, I, I, I, P, I64, P, I64, I64, P, SZ, P]
    L.kf_scan_scratch_bytes.argtypes = [I, I, I64]
    L.kf_scan_scratch_bytes.restype = SZ
    L.kf_debug_scan_timeline.argtypes = [P]
    g = torch.Generator(device=dev).manual_seed(20261201)
    rows = []
    for label, dt, n in cases:
        if dt == 5:
            x = torch.empty(n, 2, device=dev)
            x[:, 0].uniform_(0.9, 1.0, generator=g)
            x[:, 1].normal_(generator=g)
            op, es = 3, 8
        elif dt == 4:
            x = torch.randint(0, 256, (n,), device=dev, generator=g, dtype=torch.uint8)
            op, es = 0, 1
        elif dt in (6, 7):  # QuaternionF32 / QuaternionF64 (unit quaternions), Hamilton product
            x = torch.randn(n, 4, device=dev, generator=g, dtype=torch.float32 if dt == 6 else torch.float64)
            x /= x.norm(dim=1, keepdim=True)
            op, es = 4, 4 * x.element_size()
        else:
            x = torch.rand(n, device=dev, generator=g, dtype=torch.float64 if dt == 1 else torch.float32)
            op, es = 0, x.element_size()
        y = torch.empty_like(x)
        sb = L.kf_scan_scratch_bytes(dt, op, n)
        scr = torch.zeros(sb, dtype=torch.uint8, device=dev)

        def call():
            rc = L.kf_scan(op, 0, 0, dt, 0, ctypes.c_void_p(x.data_ptr()), 1, ctypes.c_void_p(y.data_ptr()), 1, n,
                           ctypes.c_void_p(scr.data_ptr()), sb, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == 0
        call()
        torch.cuda.synchronize()
        t = time_calls(call, 10)
        tiles_max = (sb - 256) // 128
        buf = torch.zeros(tiles_max * 6, dtype=torch.int64, device=dev)
        L.kf_debug_scan_timeline(ctypes.c_void_p(buf.data_ptr()))
        call()
        torch.cuda.synchronize()
        L.kf_debug_scan_timeline(None)
        a = buf.cpu().numpy().reshape(-1, 6)
        a = a[a[:, 0] > 0]
        t0 = a[:, 0].min()
        st, sc, pf, en = ((a[:, k] - t0) * 0.01 for k in range(4))  # microseconds
        ev = np.concatenate([np.stack([st, np.ones_like(st)], 1), np.stack([en, -np.ones_like(en)], 1)])
        ev = ev[np.argsort(ev[:, 0], kind="stable")]
        active = np.cumsum(ev[:, 1])
        full = ev[np.argmax(active >= 0.95 * active.max()), 0]
        last = st.max()
        tile_bytes = 2 * es * n / len(a)
        # no steady window when every tile is resident at once (one generation)
        one_generation = len(a) <= active.max() or last <= full
        steady = None if one_generation else ((en >= full) & (en <= last)).sum() * tile_bytes / (last - full) / 1e3
        row = {"case": label, "us": round(t * 1e6, 1), "gbps": round(2 * es * n / t / 1e9), "tiles": len(a),
               "peak_resident": int(active.max()), "span_us": round(float(en.max()), 1),
               "tile_life_us": round(float(np.median(en - st)), 2), "load_scan_us": round(float(np.median(sc - st)), 2),
               "lookback_us": round(float(np.median(pf - sc)), 2), "store_issue_us": round(float(np.median(en - pf)), 2),
               "ramp_us": round(float(full), 2), "steady_gbps": None if steady is None else round(float(steady)),
               "drain_us": round(float(en.max() - last), 1),
               "tiles_per_xcd": np.bincount(a[:, 4].astype(int) & 15, minlength=8)[:8].tolist()}
        rows.append(row)
        log(json.dumps(row))
        del x, y, scr, buf
    return rows


REDUCE_TIMELINE_CASES = (("Float32 n=10^6", 0, 10**6), ("Float32 n=10^7", 0, 10**7), ("Float32 n=10^8", 0, 10**8),
                         ("Float64 n=10^7", 1, 10**7), ("UInt8 n=10^7", 4, 10**7), ("UInt8 n=10^8", 4, 10**8))


def reduce_timeline(dev, cases=REDUCE_TIMELINE_CASES):
    """Per-workgroup phases of the one-launch full reduction (mapreduce of
    identity, +) from the instrumented library: each workgroup's thread 0
    stamps the 100 MHz realtime counter at its start, once its loads are
    folded into its partial and once its slot is published (the last
    workgroup: once the fold is done). Per case: time per call (HIP graph of
    uninstrumented calls of the same library), grid, span, the spread of
    workgroup starts, median load phase, and the last workgroup's own
    phases: start, loads, wait for the slots, and the fold's completion
    after the last slot was published."""
    import ctypes
    import __graft_entry__
    kf = __graft_entry__.load_package()
    D, K = kf._lib.debug_lib(), kf._lib
    g = torch.Generator(device=dev).manual_seed(20261201)
    rows = []
    for label, dt, n in cases:
        if dt == 4:
            x = torch.randint(0, 256, (n,), device=dev, generator=g, dtype=torch.uint8)
        else:
            x = torch.rand(n, device=dev, generator=g, dtype=torch.float64 if dt == 1 else torch.float32)
        out = torch.empty(1, dtype=x.dtype, device=dev)
        sb = D.kf_reduce_scratch_bytes(dt, n)
        scr = torch.zeros(sb, dtype=torch.uint8, device=dev)

        def call():
            rc = D.kf_reduce(K.OP_ADD, K.MAP_IDENTITY, dt, ctypes.c_void_p(x.data_ptr()), n, 1,
                             ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(scr.data_ptr()), sb,
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == 0, D.kf_last_error()
        t = _graph_time(call)
        L, sink, nb = K.lib(), torch.zeros(4, dtype=torch.int32, device=dev), x.numel() * x.element_size()

        def probe(kind):
            return lambda: K.check(L.kf_bw_probe(kind, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                                 nb, None, 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                                   "kf_bw_probe")
        t_read = min(_graph_time(probe(K.BW_READ)), _graph_time(probe(K.BW_READ_TILED)))
        wmax = 1 << 16
        buf = torch.zeros(wmax * 6, dtype=torch.int64, device=dev)
        D.kf_debug_reduce_timeline(ctypes.c_void_p(buf.data_ptr()))
        for _ in range(3):  # the last of three back-to-back calls, as in the graph
            call()
        torch.cuda.synchronize()
        D.kf_debug_reduce_timeline(None)
        a = buf.cpu().numpy().reshape(-1, 6)
        grid = int(a[:, 5].max())
        a = a[:grid]
        t0 = a[:, 0].min()
        st, ld, en = ((a[:, k] - t0) * 0.01 for k in range(3))  # microseconds
        last_pub = float(en[:-1].max()) if grid > 1 else float(ld[-1])
        row = {"case": label, "us": round(t * 1e6, 2), "gbps": round(x.numel() * x.element_size() / t / 1e9),
               "read_probe_us": round(t_read * 1e6, 2), "frac_of_read_probe": round(t_read / t, 3),
               "grid": grid, "span_us": round(float(en.max()), 2), "start_spread_us": round(float(st.max()), 2),
               "load_us_median": round(float(np.median(ld - st)), 2), "load_us_max": round(float((ld - st).max()), 2),
               "last_wg_start_us": round(float(st[-1]), 2), "last_wg_loaded_us": round(float(ld[-1]), 2),
               "last_slot_published_us": round(last_pub, 2), "fold_done_us": round(float(en[-1]), 2),
               "fold_after_last_slot_us": round(float(en[-1]) - last_pub, 2),
               "wgs_per_xcd": np.bincount(a[:, 3].astype(int) & 15, minlength=8)[:8].tolist()}
        rows.append(row)
        log(json.dumps(row))
        del x, scr, buf
    return rows


# ---------------------------------------------------------------------------
# Per-configuration HBM traffic (rocprofv3 --pmc)
# ---------------------------------------------------------------------------
PMC_REPS = 3
CAL_BYTES = 1 << 30


def pmc_run(kf, dev):
    """The dispatch sequence that `rocprofv3 --pmc` counts: a calibration copy
    of CAL_BYTES (kf_copy, 1 GiB read + 1 GiB written), then every case of
    config_cases PMC_REPS times, each case preceded by a marker (a 16-byte
    kf_fill, one fill_kernel workgroup) so that the summary can split the
    dispatches by case."""
    marker = torch.zeros(4, dtype=torch.int32, device=dev)

    def begin():  # a 16-byte fill: one fill_kernel workgroup of 256 lanes
        kf.setvalue_(marker, 1)

    def end():  # a 4-byte fill: one fill_elems_kernel workgroup of 64 lanes
        kf.setvalue_(marker[:1], 2)

    a = torch.rand(CAL_BYTES // 4, device=dev)
    b = torch.empty_like(a)
    cases = [["CAL", "kf_copy calibration, 1 GiB -> 1 GiB", 2 * CAL_BYTES]]
    begin()
    kf.vcopy_(b, a)
    end()
    torch.cuda.synchronize()
    del a, b
    for key, name, bytes_, fn, reps, *_ in config_cases(kf, dev):
        fn()  # outside the counted segment: first-call setup
        torch.cuda.synchronize()
        begin()
        for _ in range(PMC_REPS):
            fn()
        end()
        torch.cuda.synchronize()
        cases.append([key, name, bytes_])
        log(f"pmc: {key}")
    print(json.dumps({"pmc_cases": cases}), flush=True)


def _read_counters(path):
    """[(kernel name, grid size, {counter: value})] in dispatch order from a
    rocprofv3 counter_collection.csv (one row per dispatch and counter)."""
    import csv
    import glob
    files = glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {path}")
    disp = {}
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                k = (int(r["Dispatch_Id"]), r.get("Process_Id", ""))
                d = disp.setdefault(k, [r["Kernel_Name"], int(r["Grid_Size"]), {}])
                d[2][r["Counter_Name"]] = d[2].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [disp[k] for k in sorted(disp)]


def _segments(dispatches):
    """The dispatches between each begin marker (fill_kernel, grid 256) and
    the following end marker (fill_elems_kernel, grid 64)."""
    segs, cur = [], None
    for name, grid, ctr in dispatches:
        if "fill_kernel" in name and "fill_elems" not in name and grid == 256:
            cur = []
            segs.append(cur)
        elif "fill_elems_kernel" in name and grid == 64:
            cur = None
        elif cur is not None:
            cur.append((name, grid, ctr))
    return segs


def trace_summary(trace_dir, bench_json, out_md):
    """Markdown tables of a `rocprofv3 --kernel-trace` run of `bench.py --all
    [--sweep]`: the dispatches between each row's markers, grouped by kernel
    and grid, with the kernel time per call of the row (the sum over its
    kernels of duration x dispatches / calls of its most frequent kernel)
    and GB/s of the row's algorithmic bytes at that time."""
    import csv
    import glob
    import statistics
    files = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_trace.csv under {trace_dir}")
    disp = []
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                disp.append((int(r["Start_Timestamp"]), r["Kernel_Name"], grid,
                             (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    disp.sort()
    segs = _segments([(name, grid, {"us": us}) for _, name, grid, us in disp])
    line = [json.loads(x) for x in open(bench_json) if x.startswith("{")][0]
    rows = [(r["config"], r["gbps"] * r["us"] * 1e3) for r in line.get("all_configs", [])]
    rows += [(f"sweep {r['op']} {r['dtype']} n={r['n']}",
              r["gbps"] * r["us"] * 1e3) for r in line.get("sweep", [])]
    if len(segs) != len(rows):
        raise SystemExit(f"{len(segs)} marked segments, {len(rows)} rows")
    out = ["| row | kernel | grid (work-items) | dispatches | avg µs | min µs | max µs | kernel µs per call | GB/s at that |",
           "|---|---|---|---|---|---|---|---|---|"]
    for (label, nbytes), seg in zip(rows, segs):
        groups = {}
        for name, grid, c in seg:
            groups.setdefault((name.split("(")[0].replace("void ", "").replace("kf::", ""), grid), []).append(c["us"])
        calls = max(len(v) for v in groups.values())
        per_call = sum(sum(v) for v in groups.values()) / calls
        first = True
        for (name, grid), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            out.append(f"| {label if first else ''} | `{name}` | {grid} | {len(v)} | {statistics.mean(v):.2f} | "
                       f"{min(v):.2f} | {max(v):.2f} | " + (f"{per_call:.2f} | {nbytes / per_call / 1e3:.0f} |"
                                                              if first else " | |"))
            first = False
    with open(out_md, "w") as fh:
        fh.write("\n".join(out) + "\n")
    print("\n".join(out))


def pmc_summary(fetch_dir, write_dir, cases_json, out_json):
    """Per-case HBM bytes per call from a FETCH_SIZE run and a WRITE_SIZE run
    of `bench.py --pmc-run`, each scaled by what the counter reads for the
    calibration copy of known size, against the case's algorithmic bytes."""
    cases = None
    with open(cases_json) as fh:
        for line in fh:
            if line.startswith('{"pmc_cases"'):
                cases = json.loads(line)["pmc_cases"]
    keys = [c[0] for c in cases]
    algo = {c[0]: c[2] for c in cases}
    names = {c[0]: c[1] for c in cases}
    fetch = _segments(_read_counters(fetch_dir))
    write = _segments(_read_counters(write_dir))
    if len(fetch) != len(keys) or len(write) != len(keys):
        raise SystemExit(f"segments: fetch {len(fetch)}, write {len(write)}, cases {len(keys)}")

    def total(seg, ctr):
        return sum(c.get(ctr, 0.0) for _, _, c in seg) * 1024.0  # counters are KiB per dispatch

    f_cal = CAL_BYTES / total(fetch[0], "FETCH_SIZE")
    w_cal = CAL_BYTES / total(write[0], "WRITE_SIZE")
    out = {"calibration": {"fetch_scale": f_cal, "write_scale": w_cal,
                           "kernel": "kf_copy 1 GiB -> 1 GiB (copy_kernel)"}, "configs": {}}
    for i, key in enumerate(keys[1:], 1):
        fb = total(fetch[i], "FETCH_SIZE") * f_cal / PMC_REPS
        wb = total(write[i], "WRITE_SIZE") * w_cal / PMC_REPS
        kern = sorted({f"{n.split('(')[0]} (grid {g})" for n, g, _ in fetch[i]})
        out["configs"][key] = {"name": names.get(key, key), "fetch_bytes": fb, "write_bytes": wb,
                               "algorithmic_bytes": algo[key], "ratio": (fb + wb) / algo[key],
                               "dispatches_per_call": len(fetch[i]) / PMC_REPS, "kernels": kern}
    with open(out_json, "w") as fh:
        json.dump(out, fh, indent=1)
    for key, v in out["configs"].items():
        print(f"{key:8s} {v['name']:48s} fetch {v['fetch_bytes']:.4g} write {v['write_bytes']:.4g} "
              f"algo {v['algorithmic_bytes']:.4g} ratio {v['ratio']:.4f}")


if __name__ == "__main__":
    main()
