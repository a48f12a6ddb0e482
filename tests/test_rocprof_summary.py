"""The rocprofv3 CSV reducer: keys by (name, grid threads, workgroup threads) and
agrees between the kernel trace (X, Y, Z columns) and the counter collection
(totals)."""
import csv
import json

from bpd_substrate_amd import rocprof_summary as rs


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_trace_and_counters_share_keys(tmp_path):
    t = tmp_path / "t.csv"
    _write(t, ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Workgroup_Size_X", "Workgroup_Size_Y",
               "Workgroup_Size_Z", "Start_Timestamp", "End_Timestamp", "VGPR_Count"],
           [["k(a, b)", 512, 4, 1, 512, 1, 1, 1000, 3000, 60],
            ["k(a, b)", 512, 4, 1, 512, 1, 1, 5000, 9000, 60],
            ["k(a, b)", 256, 1, 1, 256, 1, 1, 0, 1500, 60]])
    c = tmp_path / "c.csv"
    _write(c, ["Kernel_Name", "Grid_Size", "Workgroup_Size", "Counter_Name", "Counter_Value"],
           [["k(a, b)", 2048, 512, "FETCH_SIZE", 10.0], ["k(a, b)", 2048, 512, "FETCH_SIZE", 30.0],
            ["k(a, b)", 256, 256, "FETCH_SIZE", 7.0]])
    out = tmp_path / "s.json"
    assert rs.main(["--trace", str(t), "--fetch", str(c), "-o", str(out)]) == 0
    s = json.loads(out.read_text())
    big, small = "k(a, b)|2048|512", "k(a, b)|256|256"
    assert s["trace"][big]["n"] == 2 and s["trace"][big]["avg_us"] == 3.0 and s["trace"][big]["median_us"] == 3.0
    assert s["trace"][big]["min_us"] == 2.0 and s["trace"][big]["max_us"] == 4.0
    assert s["trace"][small]["n"] == 1 and s["trace"][small]["avg_us"] == 1.5
    assert s["fetch"][big]["FETCH_SIZE"] == {"n": 2, "mean": 20.0, "median": 20.0}
    assert s["fetch"][small]["FETCH_SIZE"]["mean"] == 7.0
