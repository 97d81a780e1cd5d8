"""Phase accounting of profiling.py on synthetic stamps (the GPU side only
fills the buffer; the arithmetic is checked here)."""

import numpy as np
import pytest

from gfx950_gluon_tutorials_amd import profiling


def _stamps(pro, loop, epi, clock_hz=1.5e9, start_ticks=1000, n=4):
    rows = []
    for w in range(n):
        t0 = 10_000 + 7 * w
        t = [t0, t0 + pro, t0 + pro + loop + 10 * w, t0 + pro + loop + 10 * w + epi]
        r = [start_ticks + w + int(round((x - t0) / clock_hz * profiling.REALTIME_HZ)) for x in t]
        rows.append([v for pair in zip(t, r) for v in pair])
    return np.array(rows, dtype=np.uint64)


def test_efficiency_and_clock():
    stages = 128
    ideal = stages * profiling.CYCLES_PER_STAGE
    s = profiling.phase_stats(_stamps(3000, int(ideal / 0.9), 8000), stages)
    assert s["ideal_loop_cycles"] == ideal
    assert abs(s["mfma_efficiency"] - 0.9) < 1e-3
    assert abs(s["clock_ghz"] - 1.5) < 0.01
    assert s["prologue_cycles"] == 3000 and s["epilogue_cycles"] == 8000
    assert s["loop_cycles_max"] - s["loop_cycles_min"] == 30


def test_per_xcd_clock_and_end():
    # 16 workgroups: the odd ones (XCDs 1, 3, 5, 7) run at 1.2 GHz, the even ones at 1.5 GHz.
    stages = 64
    loop = stages * profiling.CYCLES_PER_STAGE
    fast = _stamps(1000, loop, 1000, clock_hz=1.5e9, n=16)
    slow = _stamps(1000, loop, 1000, clock_hz=1.2e9, n=16)
    d = np.where((np.arange(16) % 2 == 1)[:, None], slow, fast)
    s = profiling.phase_stats(d, stages)
    assert len(s["xcd_clock_ghz"]) == profiling.NUM_XCDS == 8
    assert all(abs(c - (1.2 if x % 2 else 1.5)) < 0.01 for x, c in enumerate(s["xcd_clock_ghz"]))
    cycles = 1000 + loop + 1000
    assert abs(s["xcd_end_us"][1] - cycles / 1.2e3) < 1.0 and abs(s["xcd_end_us"][0] - cycles / 1.5e3) < 1.0


def test_cycles_per_stage_matches_the_mfma_rates():
    # 256x256 tile, K per stage, over 4 SIMDs at the dtype's FLOP/clock/SIMD.
    for dt, flop_per_clk in (("fp16", 1024), ("bf16", 1024), ("bf8", 2048), ("mxfp4", 4096)):
        assert 256 * 256 * profiling.STAGE_K[dt] * 2 / (4 * flop_per_clk) == profiling.CYCLES_PER_STAGE


def test_rejects_stamps_from_another_launch():
    bad = _stamps(3000, 100000, 8000)
    bad[:, 4] = bad[:, 2] - 5  # loop end before loop start
    with pytest.raises(ValueError):
        profiling.phase_stats(bad, 64)


def test_sk_stats_bandwidth_and_fractions():
    # 4 workgroups, each: 200000 shader cycles over 10000 ticks of 100 MHz (2 GHz), one partial
    # load of 20000 cycles (10 us) and one store of 30000 (15 us), 5000 cycles of flag waits.
    d = np.zeros((4, 8), dtype=np.uint64)
    for i in range(4):
        d[i] = [1000, 10, 1000 + 200000, 10 + 10000, 5000, 20000, 30000, (1 << 32) | 1]
    r = profiling.sk_stats(d.ravel(), 256, 256, 64, 8192)
    assert r["clock_ghz"] == 2.0
    assert r["partial_loads"] == 4 and r["partial_stores"] == 4
    assert r["fixup_bytes"] == 8 * 256 * 256 * 4
    assert r["load_us_per_partial"] == 10.0 and r["store_us_per_partial"] == 15.0
    assert r["per_cu_gbs"] == round(262144 / 12.5e-6 / 1e9, 1)
    assert r["wait_frac"] == 0.025 and r["fixup_frac"] == 0.25


def test_sk_stats_rejects_stamps_of_another_launch():
    with pytest.raises(ValueError):
        profiling.sk_stats(np.zeros(16, dtype=np.uint64), 256, 256, 64, 8192)


def test_operand_study_kinds():
    import torch

    g = torch.Generator().manual_seed(0)
    for kind in profiling.OPERAND_KINDS:
        a, b = profiling._study_operands(kind, 32, 16, 64, g)
        assert a.shape == (32, 64) and b.shape == (16, 64) and a.dtype == b.dtype == torch.float16
    a, b = profiling._study_operands("b_const", 8, 8, 32, g)
    assert torch.all(b == b[0, 0]) and a.unique().numel() > 1
    a, b = profiling._study_operands("k_const", 8, 8, 32, g)
    assert torch.all(a == a[:, :1]) and torch.all(b == b[:, :1])
    with pytest.raises(ValueError):
        profiling._study_operands("uniform", 8, 8, 32, g)


def test_perf_table_rows_take_registers_from_the_build(tmp_path):
    """The reference's table columns, one row per measured kernel, registers
    and spills looked up by kernel name in the build's resource table."""
    res = tmp_path / "lib.so.resources.json"
    res.write_text('[{"kernel": "g9_a16w16_f16_dp_4w", "agpr": 256, "vgpr_total": 512, "sgpr": 80, '
                   '"vgpr_spill": 0, "sgpr_spill": 0, "scratch_bytes": 0, "lds_bytes": 135168}]')
    rows = [{"dtype": "fp16", "waves": 4, "M": 4096, "N": 4096, "K": 8192, "tflops": 1481.2, "mfma_efficiency": 0.9421},
            {"dtype": "mxfp4km", "waves": 4, "M": 4096, "N": 4096, "K": 8192, "tflops": 4772.0,
             "mfma_efficiency": 0.884}]
    table = profiling.perf_table(rows, str(res)).splitlines()
    assert table[0] == "| Kernel | M x N x K | TFLOPS | VGPRs | Spills | MFMA Eff. |"
    assert table[2] == "| g9_a16w16_f16_dp_4w | 4096x4096x8192 | 1481 | 512 | 0 | 94.21% |"
    assert table[3] == "| g9_a4w4km_bf16out_dp_4w | 4096x4096x8192 | 4772 | ? | ? | 88.40% |"
