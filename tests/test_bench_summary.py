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
