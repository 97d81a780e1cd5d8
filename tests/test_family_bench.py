"""CPU checks of the per-family bench's command line (the reference's
kernels/gemm/*/*/bench.py options and K lists)."""

import pytest

from gfx950_gluon_tutorials_amd.gemm.utils import family_bench as fb


def test_k_lists_are_the_reference_benches():
    # a16w16/bench.py:85-95, a8w8/bench.py:73-82, a4w4/bench.py:167-177
    assert [k for _, _, k in fb.gemm_sizes("a16w16")] == [512, 1024, 2048, 3072, 4096, 8192, 16384, 32768]
    assert [k for _, _, k in fb.gemm_sizes("a8w8")] == [1024, 2048, 3072, 4096, 8192, 16384, 32768]
    assert [k for _, _, k in fb.gemm_sizes("a4w4")] == [1024, 2048, 3072, 4096, 8192, 16384, 32768, 65536]
    assert fb.gemm_sizes("a4w4", 65536) == [(4096, 4096, 65536)]
    with pytest.raises(ValueError, match="Available K values"):
        fb.gemm_sizes("a8w8", 512)


def test_options():
    a = fb.parse_args("a16w16", ["--K", "8192", "--dtype", "bf16", "--rocprof", "--rotating-buffer-size", "1024"])
    assert (a.K, a.dtype, a.rocprof, a.rotating_buffer_size, a.iters) == (8192, ["bf16"], True, 1024, 1000)
    assert fb.parse_args("a4w4", ["--version", "1"]).version == 1
    with pytest.raises(SystemExit):
        fb.parse_args("a8w8", ["--dtype", "fp16"])  # only a16w16 takes --dtype, as in the reference


def test_every_family_module_has_a_bench_entry():
    import importlib

    for route in ("intra_wave", "inter_wave"):
        for fam in ("a16w16", "a8w8", "a4w4"):
            m = importlib.import_module(f"gfx950_gluon_tutorials_amd.gemm.{route}.{fam}.bench")
            assert m.NUM_WARPS == (4 if route == "intra_wave" else 8)


def test_attention_bench_options():
    from gfx950_gluon_tutorials_amd.attention import bench as ab

    a = ab.parse_args([])
    assert (a.dtype, a.layout, a.batch, a.hq, a.hk, a.d, a.seqlen, a.n_iters) == ("bf16", "bhsd", 1, 64, 64, 128,
                                                                                   8192, 1000)
    assert ab.SEQLENS == [1024, 2048, 4096, 8192, 16384]  # kernels/attention/bench.py:99
    # One set of B=1, HQ=HK=64, S=1024, D=128 bf16 holds 64 MiB: 8 sets span 512 MiB; S=16384 needs one.
    assert ab.rotating_set_count(ab.parse_args(["--seqlen", "1024"]), 1024) == 8
    assert ab.rotating_set_count(ab.parse_args([]), 16384) == 1
    assert ab.rotating_set_count(ab.parse_args(["--rotating-sets", "3"]), 1024) == 3
