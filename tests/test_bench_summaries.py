"""bench.py's trace and counter summaries (host-only parsing): the marker
split, the per-row kernel tables and the calibrated traffic ratios, on
small synthetic rocprofv3 CSVs."""
import csv
import json
import os

import bench


def _write_trace(path, dispatches):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "run_kernel_trace.csv"), "w", newline="") as fh:
        w = csv.DictWriter(fh, ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
                                "End_Timestamp"])
        w.writeheader()
        t = 1000
        for name, grid, us in dispatches:
            w.writerow({"Kernel_Name": name, "Grid_Size_X": grid, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
                        "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
            t += int(us * 1000) + 500


BEGIN = ("kf::fill_kernel(uint4*, uint4, long)", 256, 1.0)
END = ("kf::fill_elems_kernel(unsigned char*, long, long, kf::FillValue, int)", 64, 1.0)


def test_segments_keep_only_marked_dispatches():
    d = [("noise", 1, {}), (BEGIN[0], 256, {}), ("a", 10, {}), ("b", 20, {}), (END[0], 64, {}),
         ("between", 5, {}), (BEGIN[0], 256, {}), ("c", 30, {}), (END[0], 64, {})]
    segs = bench._segments(d)
    assert [[x[0] for x in s] for s in segs] == [["a", "b"], ["c"]]


def test_trace_summary_per_row_time(tmp_path):
    trace = tmp_path / "trace"
    # row 1: two launches per call (level 0 + fold), 3 calls; row 2: one launch, 2 calls
    _write_trace(str(trace), [BEGIN, ("void kf::reduce_once_kernel<float>(x)", 4096, 150.0),
                              ("void kf::reduce_once_kernel<float, fold>(x)", 64, 4.0)] * 1 +
                 [("void kf::reduce_once_kernel<float>(x)", 4096, 152.0), ("void kf::reduce_once_kernel<float, fold>(x)", 64, 6.0)] * 2 +
                 [END, BEGIN, ("void kf::scan_kernel<float>(x)", 100, 300.0), ("void kf::scan_kernel<float>(x)", 100, 320.0), END])
    bj = tmp_path / "bench.json"
    bj.write_text("log line\n" + json.dumps({"all_configs": [{"config": "R1", "gbps": 1.0, "us": 1.0},
                                                             {"config": "R2", "gbps": 2.0, "us": 1.0}]}) + "\n")
    out = tmp_path / "rows.md"
    bench.trace_summary(str(trace), str(bj), str(out))
    rows = [l for l in out.read_text().splitlines() if l.startswith("| R")]
    # R1: (150 + 152 + 152 + 4 + 6 + 6) / 3 = 156.67 us per call
    assert "| 156.67 |" in rows[0]
    assert "| 310.00 |" in rows[1]


def test_pmc_summary_calibrates_on_the_copy(tmp_path):
    def counters(path, ctr, values):
        os.makedirs(path, exist_ok=True)
        with open(os.path.join(path, "run_counter_collection.csv"), "w", newline="") as fh:
            w = csv.DictWriter(fh, ["Dispatch_Id", "Process_Id", "Kernel_Name", "Grid_Size", "Counter_Name",
                                    "Counter_Value"])
            w.writeheader()
            for i, (name, grid, v) in enumerate(values):
                w.writerow({"Dispatch_Id": i, "Process_Id": 1, "Kernel_Name": name, "Grid_Size": grid,
                            "Counter_Name": ctr, "Counter_Value": v})
    cal = bench.CAL_BYTES / 1024
    seq = lambda k_copy, k_case: [(BEGIN[0], 256, 0), ("kf::copy_kernel", 1, k_copy), (END[0], 64, 0),
                                  (BEGIN[0], 256, 0)] + [("kf::scan_kernel", 2, k_case)] * bench.PMC_REPS + [(END[0], 64, 0)]
    # the FETCH counter reads half the bytes, WRITE the true bytes (as on gfx950)
    counters(str(tmp_path / "f"), "FETCH_SIZE", seq(cal / 2, 1024 / 2))
    counters(str(tmp_path / "w"), "WRITE_SIZE", seq(cal, 2048))
    log = tmp_path / "cases.log"
    log.write_text(json.dumps({"pmc_cases": [["CAL", "copy", 2 * bench.CAL_BYTES], ["X", "case", 3 * 1024 * 1024]]}) + "\n")
    out = tmp_path / "t.json"
    bench.pmc_summary(str(tmp_path / "f"), str(tmp_path / "w"), str(log), str(out))
    r = json.loads(out.read_text())
    assert abs(r["calibration"]["fetch_scale"] - 2.0) < 1e-12
    assert r["configs"]["X"]["fetch_bytes"] == 1024 * 1024
    assert r["configs"]["X"]["write_bytes"] == 2048 * 1024
    assert abs(r["configs"]["X"]["ratio"] - 1.0) < 1e-12


def test_cpu_row_times_both_thread_counts_and_reports_elements():
    calls = []

    def prep():
        return lambda threads: calls.append(threads)
    row = bench.cpu_row(prep, 2e9, 5e8, 16, budget_s=0.01)
    assert set(calls) == {16, 1}
    assert row["kind"] == "port" and row["threads"] == 16
    # bytes / seconds and elements / seconds of the same timing
    assert abs(row["gbps"] / row["gelems_per_s"] - 4.0) < 1e-2
    assert abs(row["single_thread_gbps"] / row["single_thread_gelems_per_s"] - 4.0) < 1e-2
    assert row["calls"] >= 1 and row["single_thread_calls"] >= 1
