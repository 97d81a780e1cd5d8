"""CPU check of bench.py's rocprofv3 summary grouping on a synthetic SQLite
database: runs of one GEMM kernel at different shapes get separate groups
(#2, ...), and the split-K reduction launched after every split-K launch does
not split the split-K kernel's run (bench.py runs data-parallel at each split-K
shape first, which separates the split-K runs of two shapes)."""

import os
import sqlite3
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import bench  # noqa: E402


def _db(path, rows):
    con = sqlite3.connect(path)
    con.execute("create table k (name text, grid_x int, duration int, start int)")
    con.executemany("insert into k values (?, ?, ?, ?)", [(n, g, d, i) for i, (n, g, d) in enumerate(rows)])
    con.execute("create view kernels as select * from k")
    con.commit()
    con.close()


def test_summary_groups(tmp_path, capsys):
    rows = [("g9_a16w16_f16_dp_4w", 65536, 180_000)] * 3
    # bench.py's split-K cases: data-parallel at the shape, then split-K, whose
    # segment kernel and reduction alternate
    rows += [("g9_a16w16_f16_dp_4w", 4096, 120_000)] * 2
    rows += [("g9_a16w16_f16_splitk_4w", 65536, 30_000), ("g9_splitk_reduce_f16", 131072, 10_000)] * 4
    # a second shape (the segment kernel's grid is the same 256 workgroups)
    rows += [("g9_a16w16_f16_dp_4w", 8192, 130_000)] * 2
    rows += [("g9_a16w16_f16_splitk_4w", 65536, 40_000), ("g9_splitk_reduce_f16", 262144, 12_000)] * 2
    # the first DP kernel again
    rows += [("g9_a16w16_f16_dp_4w", 65536, 190_000)] * 2
    _db(str(tmp_path / "kt_results.db"), rows)
    bench.summarize_rocpd(str(tmp_path))
    out = {l.split()[0] + "@" + l.split()[1]: l.split() for l in capsys.readouterr().out.splitlines()
           if l.startswith("g9_")}
    assert out["g9_a16w16_f16_dp_4w@65536"][2] == "3"
    assert out["g9_a16w16_f16_dp_4w#2@65536"][2] == "2"
    assert out["g9_a16w16_f16_splitk_4w@65536"][2] == "4"
    assert float(out["g9_a16w16_f16_splitk_4w@65536"][3]) == 30.0
    assert out["g9_a16w16_f16_splitk_4w#2@65536"][2] == "2"
    assert out["g9_splitk_reduce_f16@131072"][2] == "4"
    assert out["g9_splitk_reduce_f16@262144"][2] == "2"


def test_csv_kernel_trace_and_counters(tmp_path, capsys):
    """The same grouping from rocprofv3's CSV output (the reference's protocol
    writes CSV): a kernel trace gives durations, a counter collection the
    per-dispatch medians of every counter."""
    import csv

    trace = tmp_path / "kt_kernel_trace.csv"
    rows = [("g9_a16w16_f16_dp_4w", 65536, 180)] * 3 + [("g9_a16w16_f16_dp_4w", 4096, 120)] * 2 \
        + [("g9_a16w16_f16_dp_4w", 65536, 200)] * 2
    with open(trace, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp",
                    "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"])
        t = 0
        for i, (n, g, us) in enumerate(rows):
            w.writerow(["KERNEL_DISPATCH", i + 1, n, t, t + us * 1000, g, 1, 1])
            t += us * 1000 + 5000
    pmc = tmp_path / "p_counter_collection.csv"
    with open(pmc, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value",
                    "Start_Timestamp", "End_Timestamp"])
        for d in range(4):
            for cn, v in (("FETCH_SIZE", 100 + d), ("WRITE_SIZE", 50)):
                w.writerow([d + 1, 65536, "g9_a4w4_bf16out_dp_4w", cn, v, d * 100000, d * 100000 + 60000])
    bench.summarize_rocpd(str(tmp_path))
    out = capsys.readouterr().out
    lines = {l.split()[0] + "@" + l.split()[1]: l.split() for l in out.splitlines() if l.startswith("g9_a16w16")}
    assert lines["g9_a16w16_f16_dp_4w@65536"][2:4] == ["3", "180.00"]
    assert lines["g9_a16w16_f16_dp_4w#2@65536"][2:4] == ["2", "200.00"]
    assert lines["g9_a16w16_f16_dp_4w@4096"][2] == "2"
    pm = [l for l in out.splitlines() if l.startswith("g9_a4w4")]
    assert pm == ["g9_a4w4_bf16out_dp_4w                            grid=65536 dispatches=4 median_us=60.00  "
                  "FETCH_SIZE=101.5  WRITE_SIZE=50"]
