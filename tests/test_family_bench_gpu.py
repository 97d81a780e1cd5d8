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


@pytest.mark.parametrize("extra", [["--layout", "bshd", "--hq", "8", "--hk", "2", "--d", "64", "--dtype", "fp16"],
                                   ["--hq", "4", "--hk", "4", "--variant", "3"]])
def test_attention_bench_checks_times_and_rocprof(gpu, capsys, extra):
    from gfx950_gluon_tutorials_amd.attention import bench as ab

    print(f"\n[case] attention bench {extra}", flush=True)
    assert ab.main(["--seqlen", "1024", *extra]) == 0
    out = capsys.readouterr().out
    assert ": match" in out and "MISMATCH" not in out
    assert any(ln.startswith("1024 ") and float(ln.split()[1]) > 0 for ln in out.splitlines())
    assert ab.main(["--seqlen", "1024", "--rocprof", "--n-iters", "4", "--rotating-sets", "2", *extra]) == 0
    assert "4 iterations done (2 rotating set(s))" in capsys.readouterr().out
