"""Phase timing and main-loop MFMA efficiency of the data-parallel kernels.

The reference measures "MFMA efficiency" -- the fraction of main-loop cycles
the SIMD's matrix pipe is busy -- from ATT thread traces of one wave
(``scripts/process_json.py:52-235``, ``docs/mfma_efficiency.md``).  The ATT
decoder is not available here, so this build records the phases directly: the
timing library (``libg9gemm_timing.so``, the same kernels compiled with
``-DG9_TIMING``) has thread 0 of every workgroup stamp the shader clock and the
100 MHz clock at kernel entry, main-loop start, main-loop end and kernel end.

Per workgroup (all its SIMDs run the same schedule):

* prologue = loop start - entry, loop = loop end - loop start, epilogue =
  end - loop end, in shader-clock cycles;
* ideal loop cycles = stages x 2048: a 256x256 tile stage is
  256*256*K_stage*2 FLOP spread over 4 SIMDs at 1024 (FP16/BF16, K_stage 64),
  2048 (BF8, K_stage 128) or 4096 (MXFP4, K_stage 256) FLOP/clock/SIMD, which
  is 2048 cycles for every type and for both wave counts;
* MFMA efficiency = ideal / loop (per SIMD, the figure the reference quotes);
* clock = shader cycles / 100 MHz ticks over the kernel: the effective shader
  clock.  (s_memtime counts shader cycles: an MFMA stream on an idle chip
  reads 2.40 GHz, the part's peak clock.)

Measurements are taken at steady state: operands rotating over >= 512 MiB of
sets and the kernel running back to back for a settle time first.  A single
launch on an idle chip runs at a higher clock, where memory latency costs
more cycles; under sustained load the kernels run at 1.6-2.2 GHz.

Usage (on a GPU box, after ``python -m gfx950_gluon_tutorials_amd.build
--timing``)::

    python -m gfx950_gluon_tutorials_amd.profiling --dtypes fp16,bf8,mxfp4 --K 8192 --waves 4,8

The stamps cost a few scalar instructions per workgroup; the main loop is
compiled unchanged.
"""

from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np

CYCLES_PER_STAGE = 2048
STAGE_K = {"fp16": 64, "bf16": 64, "bf8": 128, "mxfp4": 256, "mxfp4ps": 256, "mxfp4km": 256}
REALTIME_HZ = 100e6
NUM_XCDS = 8


def phase_stats(stamps: np.ndarray, stages: int, cycles_per_stage: int = CYCLES_PER_STAGE) -> dict:
    """Summarises raw stamps (workgroups x 8 uint64: clock/realtime pairs at
    entry, loop start, loop end, end) into medians and spreads; the ideal loop
    is stages x cycles_per_stage MFMA cycles per SIMD."""
    d = np.asarray(stamps, dtype=np.int64).reshape(-1, 8)
    t = d[:, 0::2]
    r = d[:, 1::2]
    pro = t[:, 1] - t[:, 0]
    loop = t[:, 2] - t[:, 1]
    epi = t[:, 3] - t[:, 2]
    ticks = r[:, 3] - r[:, 0]
    if (ticks <= 0).any() or (loop <= 0).any():
        raise ValueError("stamps are not increasing: was the last launch a DP launch of the timing build?")
    clock = (t[:, 3] - t[:, 0]) / (ticks / REALTIME_HZ)
    ideal = stages * cycles_per_stage
    loop_med = float(np.median(loop))
    # Workgroups are dispatched round-robin over the XCDs (workgroup i runs on
    # XCD i % 8 of an MI355X); each XCD runs at its own clock.
    xcds = min(NUM_XCDS, d.shape[0])
    xcd = np.arange(d.shape[0]) % xcds
    xcd_clock = [float(np.median(clock[xcd == x])) / 1e9 for x in range(xcds)]
    xcd_end = [float(np.median(r[xcd == x, 3] - r[:, 0].min())) / REALTIME_HZ * 1e6 for x in range(xcds)]
    return {
        "workgroups": int(d.shape[0]),
        "stages": stages,
        "clock_ghz": round(float(np.median(clock)) / 1e9, 4),
        "span_us": round(float(r[:, 3].max() - r[:, 0].min()) / REALTIME_HZ * 1e6, 2),
        "start_skew_us": round(float(r[:, 0].max() - r[:, 0].min()) / REALTIME_HZ * 1e6, 3),
        "workgroup_us": round(float(np.median(ticks)) / REALTIME_HZ * 1e6, 2),
        "end_spread_us": round(float(r[:, 3].max() - np.median(r[:, 3])) / REALTIME_HZ * 1e6, 3),
        "prologue_cycles": int(np.median(pro)),
        "loop_cycles": int(loop_med),
        "loop_cycles_min": int(loop.min()),
        "loop_cycles_max": int(loop.max()),
        "epilogue_cycles": int(np.median(epi)),
        "ideal_loop_cycles": ideal,
        "mfma_efficiency": round(ideal / loop_med, 4),
        "loop_fraction": round(loop_med / float(np.median(t[:, 3] - t[:, 0])), 4),
        "xcd_clock_ghz": [round(c, 3) for c in xcd_clock],
        "xcd_end_us": [round(e, 2) for e in xcd_end],
    }


def _inputs(dtype: str, M: int, N: int, K: int, dev, seed: int = 0):
    import torch

    from . import quant

    g = torch.Generator().manual_seed(seed)
    if dtype in ("fp16", "bf16"):
        tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
        a = (torch.randn(M, K, generator=g) * 0.1).to(tdt).to(dev)
        b = (torch.randn(N, K, generator=g) * 0.1).to(tdt).to(dev)
        return a, b.T, torch.empty(M, N, dtype=tdt, device=dev)
    if dtype == "bf8":
        qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=g).to(dev))
        qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=g).to(dev))
        return qa, qb.T, torch.empty(M, N, dtype=torch.bfloat16, device=dev), sa, sb
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=g).to(dev))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=g).to(dev))
    if dtype == "mxfp4ps":  # preshuffled scales (g9_gemm_a4w4_preshuffled)
        sa, sb = quant.preshuffle_e8m0(sa), quant.preshuffle_e8m0(sb)
    if dtype == "mxfp4km":  # K-major scale views, as the reference bench passes them
        sa, sb = sa.t().contiguous().t(), sb.t().contiguous().t()
    return pa, pb, sa, sb, torch.empty(M, N, dtype=torch.bfloat16, device=dev)


def _set_bytes(dtype: str, M: int, N: int, K: int) -> int:
    if dtype in ("fp16", "bf16"):
        return (M * K + N * K + M * N) * 2
    if dtype == "bf8":
        return M * K + N * K + 2 * M * N
    return (M * K + N * K) // 2 + (M + N) * K // 32 + 2 * M * N


def measure(dtype: str, M: int, N: int, K: int, waves: int, settle_s: float = 0.8, rotate_mb: int = 512) -> dict:
    """Phase statistics of one launch at steady state: the operands rotate
    over sets of >= rotate_mb MiB (cold caches, as in the benchmark) and the
    kernel runs back to back for settle_s seconds first, so the clocks have
    settled (a single launch on an idle chip runs at a higher clock and sees
    its memory latency as fewer cycles).  Also returns the average launch time
    of 40 launches just before the stamped one."""
    import ctypes
    import time

    import torch

    from . import _lib
    from .gemm import _launch

    lib = _lib.load()
    if not hasattr(lib, "g9_timing_read"):
        raise RuntimeError(f"{_lib.LIB_PATH} is not the timing build (python -m gfx950_gluon_tutorials_amd.build --timing)")
    lib.g9_timing_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    lib.g9_timing_capacity.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    nsets = max(2, -(-rotate_mb * 2**20 // _set_bytes(dtype, M, N, K)))
    sets = [_inputs(dtype, M, N, K, dev, seed) for seed in range(nsets)]

    def run(i):
        x = sets[i % nsets]
        if dtype in ("fp16", "bf16"):
            _launch.gemm_a16w16(x[0], x[1], x[2], waves=waves)
        elif dtype == "bf8":
            _launch.gemm_a8w8(x[0], x[1], x[2], a_scale=x[3], b_scale=x[4], waves=waves)
        else:
            _launch.gemm_a4w4(x[0], x[1], x[2], x[3], x[4], waves=waves)

    i = 0
    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            run(i)
            i += 1
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(40):
        run(i)
        i += 1
    e1.record()
    torch.cuda.synchronize()
    launch_us = e0.elapsed_time(e1) / 40 * 1e3
    run(i)
    torch.cuda.synchronize()
    tiles = -(-M // 256) * -(-N // 256)
    n = min(tiles, lib.g9_timing_capacity())
    buf = np.zeros(n * 8, dtype=np.uint64)
    _lib.check(lib.g9_timing_read(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes), "g9_timing_read")
    out = phase_stats(buf, K // STAGE_K[dtype])
    out.update({"dtype": dtype, "M": M, "N": N, "K": K, "waves": waves, "launch_us": round(launch_us, 2),
                "tflops": round(2.0 * M * N * K / launch_us / 1e6, 1), "rotating_sets": nsets})
    return out


def measure_fmha(dtype: str, B: int, H: int, S: int, variant: int = 4, settle_s: float = 0.8, D: int = 128) -> dict:
    """Phase statistics of one flash-attention launch (g9_fmha_fwd, bhsd,
    head dim D = 128 or 64) at steady state, as ``measure``.  The loop covers
    all key tiles of 8192 / D keys (64 or 128; an even count); each costs 2048
    ideal MFMA cycles per SIMD (2 waves x 32 MFMAs 32x32x16 x 32 cycles)."""
    import ctypes
    import time

    import torch

    from . import _lib
    from .attention import MetaData, compute_flops, fmha_v3, fmha_v4

    lib = _lib.load()
    if not hasattr(lib, "g9_fmha_timing_read"):
        raise RuntimeError(f"{_lib.LIB_PATH} is not the timing build (python -m gfx950_gluon_tutorials_amd.build --timing)")
    lib.g9_fmha_timing_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    dev = torch.device("cuda:0")
    tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
    g = torch.Generator().manual_seed(0)
    q, k, v = ((torch.randn(B, H, S, D, generator=g)).to(tdt).to(dev) for _ in range(3))
    o = torch.empty_like(q)
    md = MetaData(sm_scale=D**-0.5)
    md.max_seqlens_q = md.max_seqlens_k = S
    md.layout = "bhsd"
    fn = fmha_v4.run_gluon_attention if variant == 4 else fmha_v3.run_gluon_attention
    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        for _ in range(5):
            fn(q, k, v, o, md)
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        fn(q, k, v, o, md)
    e1.record()
    torch.cuda.synchronize()
    launch_us = e0.elapsed_time(e1) / 20 * 1e3
    fn(q, k, v, o, md)
    torch.cuda.synchronize()
    wgs = B * H * -(-S // 256)
    n = min(wgs, lib.g9_timing_capacity())
    buf = np.zeros(n * 8, dtype=np.uint64)
    _lib.check(lib.g9_fmha_timing_read(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes), "g9_fmha_timing_read")
    tiles = (-(-S // (8192 // D)) + 1) // 2 * 2
    out = phase_stats(buf, tiles, CYCLES_PER_STAGE)
    out.update({"kernel": f"fmha_v{variant}", "dtype": dtype, "B": B, "H": H, "S": S, "D": D,
                "launch_us": round(launch_us, 2), "tflops": round(compute_flops(B, H, S, S, D, False) / launch_us / 1e6, 1)})
    return out


def sk_stats(stamps: np.ndarray, M: int, N: int, stage_k: int, K: int) -> dict:
    """Summarises stream-K stamps (persistent workgroups x 8 uint64: clock and
    100 MHz clock at entry and exit, flag-wait / partial-load / partial-store
    cycles, (loads << 32) | stores) into the fixup's cost and bandwidth."""
    d = np.asarray(stamps, dtype=np.uint64).reshape(-1, 8).astype(np.int64)
    span = d[:, 2] - d[:, 0]
    ticks = d[:, 3] - d[:, 1]
    if (span <= 0).any() or (ticks <= 0).any():
        raise ValueError("stamps are not increasing: was the last launch a stream-K launch of the timing build?")
    clock = float(np.median(span / (ticks / REALTIME_HZ)))
    nl = d[:, 7] >> 32
    ns = d[:, 7] & 0xFFFFFFFF
    tile_bytes = 256 * 256 * 4
    moved = int((nl.sum() + ns.sum()) * tile_bytes)
    fix = d[:, 5] + d[:, 6]
    per_load_us = float(d[:, 5].sum() / max(1, nl.sum()) / clock * 1e6)
    per_store_us = float(d[:, 6].sum() / max(1, ns.sum()) / clock * 1e6)
    active = fix > 0
    return {
        "workgroups": int(d.shape[0]),
        "clock_ghz": round(clock / 1e9, 4),
        "span_us": round(float(d[:, 3].max() - d[:, 1].min()) / REALTIME_HZ * 1e6, 2),
        "partial_loads": int(nl.sum()),
        "partial_stores": int(ns.sum()),
        "fixup_bytes": moved,
        "load_us_per_partial": round(per_load_us, 3),
        "store_us_per_partial": round(per_store_us, 3),
        # Each partial is 256 KiB; one workgroup moves it at this rate ...
        "per_cu_gbs": round(tile_bytes / ((per_load_us + per_store_us) / 2 * 1e-6) / 1e9, 1),
        # ... and the workgroups that hand off do so at about the same time
        # (segment starts and ends), so this is the aggregate during fixups.
        "aggregate_gbs": round(moved / (float(np.mean(fix[active])) / clock) / 1e9, 1) if active.any() else 0.0,
        "wait_frac": round(float(d[:, 4].sum() / span.sum()), 4),
        "fixup_frac": round(float(fix.sum() / span.sum()), 4),
    }


def measure_sk(dtype: str, M: int, N: int, K: int, waves: int, settle_s: float = 0.8) -> dict:
    """Stream-K fixup cost at steady state (timing build): how long partial
    tiles take to store and reload, their bandwidth, and the share of time
    spent waiting for predecessors."""
    import ctypes
    import time

    import torch

    from . import _lib
    from .gemm import _launch

    lib = _lib.load()
    if not hasattr(lib, "g9_timing_read"):
        raise RuntimeError(f"{_lib.LIB_PATH} is not the timing build (python -m gfx950_gluon_tutorials_amd.build --timing)")
    lib.g9_timing_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    dev = torch.device("cuda:0")
    x = _inputs(dtype, M, N, K, dev)
    if dtype in ("fp16", "bf16"):
        run = lambda: _launch.gemm_a16w16(x[0], x[1], x[2], waves=waves, schedule="streamk")
    elif dtype == "bf8":
        run = lambda: _launch.gemm_a8w8(x[0], x[1], x[2], a_scale=x[3], b_scale=x[4], waves=waves, schedule="streamk")
    else:
        run = lambda: _launch.gemm_a4w4(x[0], x[1], x[2], x[3], x[4], waves=waves, schedule="streamk")
    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        for _ in range(10):
            run()
        torch.cuda.synchronize()
    run()
    torch.cuda.synchronize()
    tiles = -(-M // 256) * -(-N // 256)
    units = tiles * (K // STAGE_K[dtype])
    n = min(units, lib.g9_streamk_workgroups())
    buf = np.zeros(n * 8, dtype=np.uint64)
    _lib.check(lib.g9_timing_read(buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes), "g9_timing_read")
    out = sk_stats(buf, M, N, STAGE_K[dtype], K)
    out.update({"dtype": dtype, "M": M, "N": N, "K": K, "waves": waves, "tiles": tiles})
    return out


OPERAND_KINDS = ("randn", "zeros", "a_const", "b_const", "sign_only", "k_const")


def _study_operands(kind: str, M: int, N: int, K: int, g):
    import torch

    def rnd(rows):
        return torch.randn(rows, K, generator=g) * 0.1

    if kind == "randn":
        a, b = rnd(M), rnd(N)
    elif kind == "zeros":
        a, b = torch.zeros(M, K), torch.zeros(N, K)
    elif kind == "a_const":  # A = 0.1 everywhere (the MFMAs' second operand), B random
        a, b = torch.full((M, K), 0.1), rnd(N)
    elif kind == "b_const":  # B = 0.1 everywhere (the MFMAs' first operand), A random
        a, b = rnd(M), torch.full((N, K), 0.1)
    elif kind == "sign_only":  # +-0.1 with random signs: only the sign bits vary
        a = (torch.randint(0, 2, (M, K), generator=g) * 0.2 - 0.1)
        b = (torch.randint(0, 2, (N, K), generator=g) * 0.2 - 0.1)
    elif kind == "k_const":  # every row constant along K
        a = (torch.randn(M, 1, generator=g) * 0.1).expand(M, K).contiguous()
        b = (torch.randn(N, 1, generator=g) * 0.1).expand(N, K).contiguous()
    else:
        raise ValueError(f"unknown operand kind {kind!r}; choose from {OPERAND_KINDS}")
    return a.half(), b.half()


def operand_study(kinds, M: int = 4096, N: int = 4096, K: int = 8192, waves: int = 4, settle_s: float = 1.0,
                  nsets: int = 4) -> list:
    """Launch time of the FP16 data-parallel kernel on differently distributed
    operands.  The instruction stream and the memory traffic are the same for
    every kind; only the values differ, so under the board's power limit the
    differences are the data-dependent part of the energy per launch.  Each
    kind runs back to back for settle_s seconds before 8 timed batches of 40
    launches (median)."""
    import time

    import torch

    from .gemm import _launch

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(7)
    out = []
    for kind in kinds:
        sets = []
        for _ in range(nsets):
            a, b = _study_operands(kind, M, N, K, g)
            sets.append((a.to(dev), b.to(dev).T, torch.empty(M, N, dtype=torch.float16, device=dev)))

        def run(i):
            x = sets[i % nsets]
            _launch.gemm_a16w16(x[0], x[1], x[2], waves=waves)

        i = 0
        t_end = time.perf_counter() + settle_s
        while time.perf_counter() < t_end:
            for _ in range(20):
                run(i)
                i += 1
            torch.cuda.synchronize()
        times = []
        for _ in range(8):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(40):
                run(i)
                i += 1
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / 40 * 1e3)
        us = float(np.median(times))
        out.append({"kind": kind, "M": M, "N": N, "K": K, "waves": waves, "launch_us": round(us, 2),
                    "tflops": round(2.0 * M * N * K / us / 1e6, 1)})
        del sets
        torch.cuda.empty_cache()
    return out


KERNEL_BASE = {"fp16": "g9_a16w16_f16", "bf16": "g9_a16w16_bf16", "bf8": "g9_a8w8_bf16out",
               "mxfp4": "g9_a4w4_bf16out", "mxfp4km": "g9_a4w4km_bf16out", "mxfp4ps": "g9_a4w4ps_bf16out"}


def perf_table(results: list[dict], resources_path: str) -> str:
    """The reference's perf table (scripts/run_perf_table.py:265-391, printed
    as in scripts/README.md: TFLOPS | VGPRs | Spills | MFMA Eff.), one row per
    measured data-parallel kernel, registers and spills from the regular
    build's code-object table (``<lib>.resources.json``, which the timing
    build's kernels match: the stamps add no registers to the loop)."""
    with open(resources_path) as f:
        res = {r["kernel"]: r for r in json.load(f)}
    lines = ["| Kernel | M x N x K | TFLOPS | VGPRs | Spills | MFMA Eff. |",
             "|---|---|---|---|---|---|"]
    for r in results:
        name = f"{KERNEL_BASE[r['dtype']]}_dp_{r['waves']}w"
        k = res.get(name, {})
        spills = k.get("vgpr_spill", 0) + k.get("sgpr_spill", 0) if k else "?"
        lines.append(f"| {name} | {r['M']}x{r['N']}x{r['K']} | {r['tflops']:.0f} | {k.get('vgpr_total', '?')} | "
                     f"{spills} | {100 * r['mfma_efficiency']:.2f}% |")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--dtypes", default="fp16,bf8,mxfp4")
    ap.add_argument("--M", type=int, default=4096)
    ap.add_argument("--N", type=int, default=4096)
    ap.add_argument("--K", default="8192", help="comma-separated list")
    ap.add_argument("--waves", default="4")
    ap.add_argument("--json", help="also write the results to this file")
    ap.add_argument("--table", action="store_true",
                    help="also print the reference's perf table (TFLOPS, VGPRs, spills, MFMA efficiency) in markdown")
    ap.add_argument("--streamk", action="store_true",
                    help="stream-K fixup cost instead (give --M/--N/--K; e.g. 8192 1280 8192)")
    ap.add_argument("--fmha", help="flash-attention forward instead: B,H,S[,D] (e.g. 32,8,8192; D 128 or 64); "
                    "--dtypes fp16/bf16, --waves is ignored")
    ap.add_argument("--variants", default="4", help="with --fmha: 3, 4 or 3,4")
    ap.add_argument("--operands", help="FP16 launch time per operand distribution instead "
                    f"(comma-separated from {','.join(OPERAND_KINDS)})")
    args = ap.parse_args(argv)
    results = []
    if args.fmha:
        B, H, S, *rest = (int(x) for x in args.fmha.split(","))
        D = rest[0] if rest else 128
        for dt in args.dtypes.split(","):
            for var in (int(x) for x in args.variants.split(",")):
                r = measure_fmha(dt, B, H, S, var, D=D)
                results.append(r)
                print(f"fmha_v{var} {dt} B={B} H={H} S={S} D={D}: {r['launch_us']:.1f} us/launch "
                      f"({r['tflops']:.0f} TFLOPS)  loop MFMA eff {r['mfma_efficiency']:.3f}  clock "
                      f"{r['clock_ghz']:.3f} GHz  prologue {r['prologue_cycles']}  loop {r['loop_cycles']} (ideal "
                      f"{r['ideal_loop_cycles']})  epilogue {r['epilogue_cycles']} cycles | workgroup "
                      f"{r['workgroup_us']:.1f} us, span {r['span_us']:.1f} us", flush=True)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(results, f, indent=1)
        return 0
    if args.operands:
        for w in (int(v) for v in args.waves.split(",")):
            for r in operand_study(args.operands.split(","), args.M, args.N, int(args.K.split(",")[0]), w):
                results.append(r)
                print(f"fp16 {args.M}x{args.N}x{r['K']} waves={w} operands {r['kind']:10s}: "
                      f"{r['launch_us']:.1f} us/launch ({r['tflops']:.0f} TFLOPS)", flush=True)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(results, f, indent=1)
        return 0
    if args.streamk:
        for dt in args.dtypes.split(","):
            for K in (int(k) for k in args.K.split(",")):
                for w in (int(v) for v in args.waves.split(",")):
                    r = measure_sk(dt, args.M, args.N, K, w)
                    results.append(r)
                    print(f"stream-K {dt:6s} {args.M}x{args.N}x{K} waves={w}: {r['workgroups']} workgroups, "
                          f"{r['tiles']} tiles, span {r['span_us']:.1f} us at {r['clock_ghz']:.2f} GHz; "
                          f"{r['partial_stores']} partial stores + {r['partial_loads']} loads = "
                          f"{r['fixup_bytes'] / 2**20:.0f} MiB; per 256 KiB partial: store {r['store_us_per_partial']:.2f} us, "
                          f"load {r['load_us_per_partial']:.2f} us ({r['per_cu_gbs']:.0f} GB/s per CU, "
                          f"~{r['aggregate_gbs']:.0f} GB/s aggregate); time in flag waits {100 * r['wait_frac']:.1f}%, "
                          f"in fixups {100 * r['fixup_frac']:.1f}%", flush=True)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(results, f, indent=1)
        return 0
    for dt in args.dtypes.split(","):
        for K in (int(k) for k in args.K.split(",")):
            for w in (int(v) for v in args.waves.split(",")):
                r = measure(dt, args.M, args.N, K, w)
                results.append(r)
                print(f"{dt:6s} {args.M}x{args.N}x{K} waves={w}: {r['launch_us']:.1f} us/launch "
                      f"({r['tflops']:.0f} TFLOPS)  loop MFMA eff {r['mfma_efficiency']:.3f}  "
                      f"clock {r['clock_ghz']:.3f} GHz  prologue {r['prologue_cycles']}  "
                      f"loop {r['loop_cycles']} (ideal {r['ideal_loop_cycles']})  epilogue {r['epilogue_cycles']} cycles  "
                      f"| workgroup {r['workgroup_us']:.1f} us, span {r['span_us']:.1f} us (start skew "
                      f"{r['start_skew_us']:.2f}, last end +{r['end_spread_us']:.2f} after the median) | per-XCD clock "
                      f"{min(r['xcd_clock_ghz']):.3f}-{max(r['xcd_clock_ghz']):.3f} GHz, median end "
                      f"{min(r['xcd_end_us']):.1f}-{max(r['xcd_end_us']):.1f} us",
                      flush=True)
    if args.table:
        from . import build as _b

        print(perf_table(results, _b.LIB_PATH + ".resources.json"), flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(results, f, indent=1)
    return 0


if __name__ == "__main__":
    if not os.environ.get("G9_LIBRARY"):
        from . import build as _b

        os.environ["G9_LIBRARY"] = _b.LIB_TIMING_PATH
    sys.exit(main())
