"""The per-family benches on the GPU: the correctness check matches on the
reference's inputs for every family and both wave counts, the perf table
prints, and --rocprof mode issues its launches through prepared launches."""

import importlib

import pytest

from gfx950_gluon_tutorials_amd.gemm.utils import family_bench as fb

pytestmark = pytest.mark.gpu

SMALL_K = {"a16w16": 512, "a8w8": 1024, "a4w4": 1024}


@pytest.mark.parametrize("route", ["intra_wave", "inter_wave"])
@pytest.mark.parametrize("fam", ["a16w16", "a8w8", "a4w4"])
def test_family_bench_checks_and_times(gpu, capsys, route, fam):
    print(f"\n[case] {route}/{fam} bench K={SMALL_K[fam]}", flush=True)
    m = importlib.import_module(f"gfx950_gluon_tutorials_amd.gemm.{route}.{fam}.bench")
    assert fb.main(fam, m.matmul, m.NUM_WARPS, ["--K", str(SMALL_K[fam])]) == 0
    out = capsys.readouterr().out
    assert "differ" not in out and out.count("match") == (2 if fam == "a16w16" else 1)
    row = [ln for ln in out.splitlines() if ln.startswith(f"4096 4096 {SMALL_K[fam]} ")]
    assert len(row) == 1 and all(float(x) > 0 for x in row[0].split()[3:])
    assert fb.main(fam, m.matmul, m.NUM_WARPS, ["--K", str(SMALL_K[fam]), "--rocprof", "--iters", "5",
                                                 "--rotating-buffer-size", "64"]) == 0
    assert "5 iterations done" in capsys.readouterr().out
