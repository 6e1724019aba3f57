"""bench.py's measurement tooling on synthetic rocprofv3 output (CPU only).

trace_summary cuts a kernel trace at idle gaps and reports each workload's
timed launches; traffic_summary turns FETCH_SIZE / WRITE_SIZE counter runs
into bytes per call, scaled by the calibration copy, and keeps the committed
entries of workloads it has no runs for.
"""
import csv
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

TRACE_FIELDS = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Workgroup_Size_X",
                "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
MX = "void ga::(anonymous namespace)::mx_pp_kernel<true, false, 0>(ga_f4gemm_kargs, float*)"
DEC = ("void ga::(anonymous namespace)::mx_decode_kernel<4, 8, true, false, false, 3, 0, "
       "false>(ga_f4gemm_kargs, int, int, float*, ga_splitk_ws_handle const*)")
RED = "void ga::(anonymous namespace)::splitk_reduce_kernel<8>(ga::ReduceArgs)"
TORCH = "void at::native::elementwise_kernel<128, 4>(int, float*)"


class Trace:
    def __init__(self):
        self.rows, self.t = [], 0

    def launch(self, name, us, wg, nwg, gap_ns=300):
        self.t += gap_ns
        self.rows.append({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name,
                          "Start_Timestamp": self.t, "End_Timestamp": self.t + int(us * 1000),
                          "Workgroup_Size_X": wg, "Grid_Size_X": wg * nwg,
                          "Grid_Size_Y": 1, "Grid_Size_Z": 1})
        self.t += int(us * 1000)

    def idle(self, ms):
        self.t += int(ms * 1e6)

    def write(self, d):
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, "p_kernel_trace.csv"), "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=TRACE_FIELDS)
            w.writeheader()
            w.writerows(self.rows)


def table_rows(text):
    return [[c.strip() for c in line.strip("|").split("|")] for line in text.splitlines()[2:]]


def test_trace_summary_cuts_workloads_at_idle_gaps(tmp_path):
    tr = Trace()
    # a time_gemm run: warmup, 100 timed launches, 10 timed one by one
    for us in [400.0] * 90 + [370.0] * 100 + [371.0] * 10:
        tr.launch(MX, us, 512, 256)
    tr.idle(2.0)
    # a split call: K-slice kernel and reduce interleaved (last 100 of each)
    for i in range(120):
        tr.launch(DEC, 45.0 + (i >= 20), 64, 256)
        tr.launch(RED, 4.0 + (i >= 20) * 0.5, 256, 64)
    tr.idle(2.0)
    for _ in range(50):  # data generation: no library kernel
        tr.launch(TORCH, 10.0, 128, 100)
    tr.idle(2.0)
    for _ in range(40):  # two library kernels in one piece: not one workload
        tr.launch(MX, 10.0, 512, 256)
        tr.launch(DEC, 10.0, 64, 256)
    tr.write(str(tmp_path / "prof"))
    rows = table_rows(bench.trace_summary(str(tmp_path)))
    assert len(rows) == 2
    run, kernel, grid, n, t110, t100, red = rows[0]
    assert (run, kernel, grid, n) == ("1", "`mx_pp_kernel<true, false, 0>`", "256 x 512", "200")
    assert float(t110) == pytest.approx(370.0) and float(t100) == pytest.approx(370.1)
    assert red == "-"
    run, kernel, grid, n, t110, t100, red = rows[1]
    assert kernel.startswith("`mx_decode_kernel<4, 8,") and grid == "256 x 64" and n == "120"
    assert float(t100) == pytest.approx(46.0) and float(red) == pytest.approx(4.5)


COUNTER_FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
BS = "void ga::(anonymous namespace)::bs_pp_kernel<0, 1>(ga_opus_gemm_kargs)"
QUANT = "void ga::(anonymous namespace)::quant_1x128_kernel<0, 4, 2>(ga::QuantArgs)"
COPY = "__amd_rocclr_copyBuffer"


def write_counters(d, ctr, copy_kib, call_kib, calls):
    os.makedirs(d, exist_ok=True)
    rows, i = [], 0
    for _ in range(2):  # the calibration copies of 512 MiB
        i += 1
        rows.append({"Dispatch_Id": i, "Kernel_Name": COPY, "Counter_Name": ctr,
                     "Counter_Value": copy_kib})
    i += 1  # a set-up quantiser: not part of the call
    rows.append({"Dispatch_Id": i, "Kernel_Name": QUANT, "Counter_Name": ctr,
                 "Counter_Value": 999999.0})
    for _ in range(calls):
        i += 1
        rows.append({"Dispatch_Id": i, "Kernel_Name": BS, "Counter_Name": ctr,
                     "Counter_Value": call_kib})
    with open(os.path.join(d, "p_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COUNTER_FIELDS)
        w.writeheader()
        w.writerows(rows)


def test_traffic_summary_scales_and_keeps_committed_entries(tmp_path, monkeypatch):
    repo = tmp_path / "repo"
    os.makedirs(repo / "profiles")
    kept = {"kernel": None, "bytes_per_launch": 123, "log2_k_split": 0}
    with open(repo / "profiles" / "traffic.json", "w") as f:
        json.dump({"note": "old", "workloads": {"some_other_workload": kept}}, f)
    monkeypatch.setattr(bench, "ROOT", str(repo))
    wl = "fp8_blockscale_1x128_128x128_8192x8192x8192_f32out"
    runs = tmp_path / "traffic"
    # FETCH_SIZE reads half of the copy's bytes (factor 2), WRITE_SIZE all of them
    write_counters(str(runs / wl / "FETCH_SIZE"), "FETCH_SIZE", 262144.0, 1000.0, 5)
    write_counters(str(runs / wl / "WRITE_SIZE"), "WRITE_SIZE", 524288.0, 300.0, 5)
    bench.traffic_summary(str(runs), 5)
    with open(repo / "profiles" / "traffic.json") as f:
        got = json.load(f)["workloads"]
    assert got["some_other_workload"] == kept
    e = got[wl]
    assert e["fetch_factor"] == pytest.approx(2.0) and e["write_factor"] == pytest.approx(1.0)
    assert e["fetch_bytes"] == 2 * 1000 * 1024 and e["write_bytes"] == 300 * 1024
    assert e["bytes_per_launch"] == e["fetch_bytes"] + e["write_bytes"]
    assert e["dispatches"] == 5
