"""Benchmark of the gfx950 GEMM hot path (one MI355X).

Metric: TFLOPS and fraction of the dense MFMA peak for the
4096x4096x8192 NT GEMM in fp16 (headline ``value``), bf8 and mxfp4.

A "step" is one GEMM launch over one set of synthetic operands already
resident in HBM.  The operands rotate over several sets (>= 512 MiB in total)
so every launch starts with cold caches, as in the reference's protocol
(kernels/gemm/intra_wave/a16w16/bench.py:190-241).  Timing: W untimed warm-up
launches, continued until --settle-ms of load has passed (the chip's clocks
need a few hundred ms of load to settle; the reference's protocol likewise
discards 900 of 1000 dispatches), then K launches bracketed by synchronize +
HIP events on the launch stream; ms_per_step is the average launch time and
TFLOPS = 2*M*N*K / t.

The JSON line also carries the roofline of the dominant kernel (MFMA-bound:
achieved TFLOP/s vs the published dense peak) with the HBM traffic per launch
read from the committed rocprof counter summary when present, the other
dtypes, the stream-K shapes, split-K against data-parallel on grids of 16-128
tiles, the grouped (MoE) GEMMs, the flash-attention forward (fmha_v4 and
fmha_v3 at B=32 H=8 S=8192 D=128, bf16 and fp16, against the reference's
published bf16 numbers), the host time per launch of a one-tile GEMM (matmul
wrapper, prepared launch, torch.matmul), and a CPU baseline: torch.matmul in
fp32 on the dequantized operands timed on this host on a bounded row sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# Published dense MFMA peaks of one MI355X, TFLOP/s.
PEAK = {"fp16": 2500.0, "bf16": 2500.0, "bf8": 5000.0, "mxfp4": 10100.0, "mxfp4ps": 10100.0, "mxfp4km": 10100.0}
# The reference's published MI355X numbers for the same shapes (4-wave,
# kernels/gemm/intra_wave/a16w16/v9_beyond_hotloop/README.md:180,
# kernels/gemm/inter_wave/a8w8/README.md:61, kernels/gemm/inter_wave/a4w4/v0_sliceMN/README.md:60).
REFERENCE_TFLOPS = {"fp16": 1608.0, "bf8": 3215.0, "mxfp4": 4986.0, "mxfp4ps": 4986.0, "mxfp4km": 4986.0}
# 8-wave: kernels/gemm/inter_wave/a16w16/README.md:120, kernels/gemm/inter_wave/a8w8/README.md:61,
# kernels/gemm/inter_wave/a4w4/README.md:17.
REFERENCE_TFLOPS_8W = {"fp16": 1478.0, "bf8": 2949.0, "mxfp4": 4479.0}
# BF16 and the headline-K shapes (4-wave, 8-wave): scripts/plot_perf_summary.py:53-58.
REFERENCE_TFLOPS["bf16"] = 1696.0
REFERENCE_TFLOPS_8W["bf16"] = 1573.6
HEADLINE_K = {"bf8": (16384, 3476.0, 3131.1), "mxfp4": (32768, 5804.0, 5195.9), "mxfp4ps": (32768, 5804.0, None),
              "mxfp4km": (32768, 5804.0, None)}
# MXFP4 scale layouts: mxfp4 row-major (M x K/32 bytes, BASELINE's configuration),
# mxfp4km K-major views of (K/32, M) storage (what the reference bench passes,
# kernels/gemm/intra_wave/a4w4/bench.py:137-146), mxfp4ps preshuffled.  Only
# the 4-wave kernels read the last two as they are.
FOUR_WAVE_ONLY = ("mxfp4ps", "mxfp4km")
# How each MXFP4 case passes its E8M0 scales (recorded in its per_dtype entry).
SCALE_LAYOUTS = {
    "mxfp4": "row-major (M, K/32), contiguous",
    "mxfp4km": "K-major: (K/32, M) storage viewed as (M, K/32), as the reference bench builds them "
               "(kernels/gemm/intra_wave/a4w4/bench.py:137-146)",
    "mxfp4ps": "preshuffled (quant.preshuffle_e8m0)",
}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
# Flash-attention forward: the reference's tuned shape and its published
# numbers (bf16, kernels/attention/README.md:619-632; no fp16 figure).
FMHA_SHAPE = {"B": 32, "H": 8, "S": 8192, "D": 128}
FMHA_REFERENCE_TFLOPS = {("bf16", 4): 1261.0, ("bf16", 3): 1189.0}
# The reference attention bench's defaults and sequence-length sweep
# (kernels/attention/bench.py:100, :107-113): B=1, HQ=HK=64, bhsd, bf16.
FMHA_SWEEP_SEQLENS = (1024, 2048, 4096, 8192, 16384)
FMHA_SWEEP_SHAPE = {"B": 1, "H": 64}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--settle-ms", type=float, default=600.0,
                   help="keep warming up until this much time has passed (the MI355X's clocks take a few "
                        "hundred ms of load to settle; timed launches before that run up to 15%% slower)")
    p.add_argument("--dtypes", default="fp16,bf16,bf8,mxfp4,mxfp4km,mxfp4ps",
                   help="comma list of fp16,bf16,bf8,mxfp4,mxfp4km,mxfp4ps (mxfp4 with K-major scale views as the "
                        "reference bench passes them / with preshuffled scales, 4-wave)")
    p.add_argument("--headline-k", type=int, default=1,
                   help="also time bf8 at K=16384 and mxfp4 at K=32768, the reference's headline shapes")
    p.add_argument("--streamk", type=int, default=1, help="also time the stream-K shapes (0/1)")
    p.add_argument("--waves", default="4,8", help="wave schedules to time: 4 (1 wave/SIMD), 8 (2 waves/SIMD)")
    p.add_argument("--moe", type=int, default=1, help="also time the grouped (MoE) GEMMs (0/1)")
    p.add_argument("--splitk", type=int, default=1,
                   help="also time split-K against data-parallel on grids of <= 128 tiles (0/1)")
    p.add_argument("--vendor", type=int, default=1,
                   help="also time ROCm's hipBLASLt (torch.matmul / torch._scaled_mm) on the same shapes, "
                        "interleaved with ours, for fp16/bf16/bf8 at K=8192 (0/1)")
    p.add_argument("--fmha", type=int, default=1,
                   help="also time the flash-attention forward at B=32 H=8 S=8192 D=128 (0/1)")
    p.add_argument("--fmha-only", type=int, default=0,
                   help="time only the flash-attention forward (--steps / --warmup / --settle-ms launches of each "
                        "case) and print its object (for profilers)")
    p.add_argument("--fmha-sweep", type=int, default=0,
                   help="time only the flash-attention forward over the reference bench's sequence-length sweep "
                        "(B=1, HQ=HK=64, bf16, head dims 128 and 64, v4 and v3) and print its object")
    p.add_argument("--energy", type=float, default=0.0,
                   help="energy per launch instead: ours vs hipBLASLt for fp16 and bf16, this many seconds of "
                        "back-to-back launches per side and round (two interleaved rounds), amd-smi power sampled")
    p.add_argument("--cpu-baseline", type=int, default=1)
    p.add_argument("--prepared", type=int, default=0,
                   help="launch the per-dtype GEMM cases through PreparedGemm (arguments bound once per rotating "
                        "set) instead of the matmul wrappers, as the reference's scripts/benchmark_prepared.py does")
    p.add_argument("--launch-overhead", type=int, default=1,
                   help="host time per launch of a one-tile GEMM: matmul wrapper, prepared launch, torch.matmul")
    p.add_argument("--rotate-mb", type=int, default=512)
    p.add_argument("--serialized", type=int, default=0,
                   help="also time serialized dispatches with HIP events (mean of the last 100 of 1000); the events "
                        "add the per-dispatch gaps, so this reads slower than the reference's protocol, which takes "
                        "kernel durations from a rocprofv3 trace with AMD_SERIALIZE_KERNEL=3 "
                        "(profiles/reference_protocol_4096.txt)")
    p.add_argument("--only", default="", help="run one case only, e.g. fp16 (for profilers)")
    p.add_argument("--telemetry-s", type=float, default=3.0,
                   help="run the headline case this long while sampling board power and clock (0: skip)")
    p.add_argument("--ksweep", type=int, default=0,
                   help="instead: time fp16/bf8/mxfp4 at M=N=4096 over the reference benches' K sweep, 4 and 8 waves")
    p.add_argument("--pair", type=int, default=0,
                   help="profiler target: run our 4-wave kernel and hipBLASLt on the --only dtype (fp16 by "
                        "default) N times each at 4096x4096x8192, then exit")
    p.add_argument("--summarize", default="",
                   help="print a per-kernel summary of the rocprofv3 SQLite output under this directory and exit")
    p.add_argument("--copy-mb", type=int, default=0,
                   help="also launch a plain device copy of this many MiB 10 times (counter calibration)")
    return p.parse_args()


LAUNCH_SHAPE = (256, 256, 512)


def launch_overhead(dev, calls: int = 2000) -> dict:
    """Host time per launch (us) of a one-tile FP16 GEMM issued back to back
    without synchronising: the a16w16 matmul wrapper, a prepared launch
    (PreparedGemm: one g9_plan_launch call, the counterpart of the
    reference's scripts/benchmark_prepared.py) and torch.matmul (hipBLASLt),
    beside the GPU time per launch of the wrapper's loop.  The host side is
    what bounds small GEMMs issued one after another."""
    import torch

    from gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16 import matmul as m16
    from gfx950_gluon_tutorials_amd.gemm.prepared import PreparedGemm

    M, N, K = LAUNCH_SHAPE
    gen = torch.Generator().manual_seed(0)
    a = torch.randn(M, K, generator=gen).half().to(dev)
    bt = torch.randn(N, K, generator=gen).half().to(dev).T
    c = torch.empty(M, N, dtype=torch.half, device=dev)
    prep = PreparedGemm.a16w16([(a, bt, c)])
    out = {"shape": list(LAUNCH_SHAPE), "calls": calls}
    for name, fn in (("matmul_us", lambda: m16(a, bt, c)), ("prepared_us", prep),
                     ("torch_matmul_us", lambda: torch.matmul(a, bt, out=c))):
        for _ in range(100):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        host = time.perf_counter() - t0
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(host / calls * 1e6, 2)
        if name == "matmul_us":
            out["gpu_us_per_launch"] = round(e0.elapsed_time(e1) / calls * 1e3, 2)
    print(f"# launch overhead, host us per call ({M}x{N}x{K} fp16, {calls} back-to-back calls): matmul "
          f"{out['matmul_us']}, prepared {out['prepared_us']}, torch.matmul {out['torch_matmul_us']} "
          f"(GPU {out['gpu_us_per_launch']} us per launch)", flush=True)
    return out


def copy_calibration(mb: int, dev) -> None:
    """A plain copy kernel of known size: its FETCH_SIZE / WRITE_SIZE readings
    give the scale between those counters and bytes moved."""
    import torch

    n = mb * 2**20 // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"# copy calibration: 10 x {mb} MiB device copies", flush=True)


def make_case(dtype: str, M: int, N: int, K: int, seed: int, dev, nsets: int, waves: int = 4,
              prepared: bool = False):
    """Returns launch(i, schedule) running the drop-in wrapper of `waves` on
    operand set i, or with `prepared` a PreparedGemm over the sets (one per
    schedule, bound at its first launch), as the reference's
    scripts/benchmark_prepared.py times its kernels."""
    import torch

    from gfx950_gluon_tutorials_amd import quant
    if waves == 4:
        from gfx950_gluon_tutorials_amd.gemm.intra_wave.a4w4 import matmul as m4
        from gfx950_gluon_tutorials_amd.gemm.intra_wave.a8w8 import matmul as m8
        from gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16 import matmul as m16
    else:
        from gfx950_gluon_tutorials_amd.gemm.inter_wave.a4w4 import matmul as m4
        from gfx950_gluon_tutorials_amd.gemm.inter_wave.a8w8 import matmul as m8
        from gfx950_gluon_tutorials_amd.gemm.inter_wave.a16w16 import matmul as m16

    gen = torch.Generator().manual_seed(seed)
    sets = []
    for _ in range(nsets):
        if dtype in ("fp16", "bf16"):
            tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
            a = (torch.randn(M, K, generator=gen) * 0.1).to(tdt).to(dev)
            b = (torch.randn(N, K, generator=gen) * 0.1).to(tdt).to(dev)
            c = torch.empty(M, N, dtype=tdt, device=dev)
            sets.append((a, b.T, c))
        elif dtype == "bf8":
            qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=gen).to(dev))
            qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=gen).to(dev))
            sets.append((qa, qb.T, sa, sb))
        elif dtype in ("mxfp4", "mxfp4ps", "mxfp4km"):
            pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen).to(dev))
            pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen).to(dev))
            if dtype == "mxfp4ps":  # the scales' one-off layout change happens here, outside any timing
                sa, sb = quant.preshuffle_e8m0(sa), quant.preshuffle_e8m0(sb)
            if dtype == "mxfp4km":  # (K/32, M) storage viewed as (M, K/32), as the reference bench does
                sa, sb = sa.t().contiguous().t(), sb.t().contiguous().t()
            sets.append((pa, pb, sa, sb))
        else:
            raise ValueError(dtype)

    def launch(i, schedule="dp"):
        s = sets[i % len(sets)]
        if dtype in ("fp16", "bf16"):
            m16(s[0], s[1], s[2], schedule=schedule)
        elif dtype == "bf8":
            m8(s[0], s[1], a_scale=s[2], b_scale=s[3], out_dtype=torch.bfloat16, schedule=schedule)
        else:
            m4(s[0], s[1], s[2], s[3], schedule=schedule)

    if not prepared:
        return launch
    from gfx950_gluon_tutorials_amd.gemm.prepared import PreparedGemm

    plans = {}

    def bind(schedule):
        if dtype in ("fp16", "bf16"):
            return PreparedGemm.a16w16(sets, schedule=schedule, waves=waves)
        out = [torch.empty(M, N, dtype=torch.bfloat16, device=dev) for _ in sets]
        if dtype == "bf8":
            return PreparedGemm.a8w8([(qa, qb, c, sa, sb) for (qa, qb, sa, sb), c in zip(sets, out)],
                                     schedule=schedule, waves=waves)
        return PreparedGemm.a4w4([(pa, pb, sa, sb, c) for (pa, pb, sa, sb), c in zip(sets, out)],
                                 schedule=schedule, waves=waves)

    def launch_prepared(i, schedule="dp"):
        p = plans.get(schedule)
        if p is None:
            p = plans[schedule] = bind(schedule)
        p(i)

    return launch_prepared


def set_bytes(dtype, M, N, K):
    if dtype in ("fp16", "bf16"):
        return (M * K + N * K + M * N) * 2
    if dtype == "bf8":
        return M * K + N * K + 2 * M * N
    return (M * K + N * K) // 2 + (M + N) * K // 32 + 2 * M * N


def time_case(launch, steps, warmup, schedule="dp", settle_s=0.0):
    """Average ms per launch of `steps` back-to-back launches, after `warmup`
    untimed launches that continue (in blocks of 20) until `settle_s` seconds
    of warm-up have passed."""
    import torch

    t0 = time.perf_counter()
    for i in range(warmup):
        launch(i, schedule)
    torch.cuda.synchronize()
    i = warmup
    while time.perf_counter() - t0 < settle_s:
        for _ in range(20):
            launch(i, schedule)
            i += 1
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        launch(i, schedule)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per launch


def _smi_sample(exe: str):
    """One amd-smi reading: (socket power W, mean GFX clock MHz over the XCDs)."""
    import subprocess

    out = subprocess.run([exe, "metric", "-g", "0", "-p", "-c", "--json"], capture_output=True, text=True,
                         timeout=10).stdout
    d = json.loads(out)
    g = d[0] if isinstance(d, list) else d
    if isinstance(g, dict) and "gpu_data" in g:
        g = g["gpu_data"][0]
    pw = g.get("power", {}).get("socket_power")
    pw = pw.get("value") if isinstance(pw, dict) else pw
    clk = [v["clk"]["value"] for k, v in g.get("clock", {}).items()
           if k.startswith("gfx_") and isinstance(v, dict) and isinstance(v.get("clk"), dict)]
    return (float(pw) if pw not in (None, "N/A") else None), (sum(clk) / len(clk) if clk else None)


def telemetry(launch, secs: float):
    """Runs `launch` back to back for `secs` seconds while a child amd-smi
    process samples the board power and GFX clock; returns the medians over
    the second half of the window and the launch time there (None without
    amd-smi).  Evidence for the power limit: the FP16/BF16 GEMMs hold the
    board at its 1400 W cap with the clock well below its 2.4 GHz peak."""
    import shutil
    import statistics as st
    import threading

    import torch

    exe = shutil.which("amd-smi") or "/opt/rocm/bin/amd-smi"
    if not os.path.exists(exe):
        return None
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            try:
                samples.append((time.perf_counter(), *_smi_sample(exe)))
            except Exception:  # a failed reading is skipped
                pass

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t0 = time.perf_counter()
    blocks, i = [], 0
    while time.perf_counter() - t0 < secs:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(50):
            launch(i)
            i += 1
        e1.record()
        torch.cuda.synchronize()
        blocks.append((time.perf_counter(), e0.elapsed_time(e1) / 50))
    stop.set()
    th.join(timeout=15)
    half = t0 + secs / 2
    pw = [p for t, p, c in samples if t >= half and p is not None]
    ck = [c for t, p, c in samples if t >= half and c is not None]
    ms = [m for t, m in blocks if t >= half]
    if not pw or not ck or not ms:
        return None
    return {"seconds": secs, "samples": len(pw), "power_w": st.median(pw), "gfx_clock_mhz": round(st.median(ck)),
            "launch_us": round(st.median(ms) * 1e3, 2), "tool": "amd-smi metric -p -c"}


def time_serialized(launch, n=1000, last=100):
    """An event-timed approximation of the reference's timing protocol
    (kernels/gemm/README.md:89-94): every dispatch completes before the next
    is issued (as with AMD_SERIALIZE_KERNEL=3) and the mean of the last `last`
    of `n` is reported (ms).  The reference takes each duration from a
    rocprofv3 kernel trace; events around a dispatch also include the gap
    before the kernel starts, several microseconds, so this reads slower."""
    import torch

    start = [torch.cuda.Event(enable_timing=True) for _ in range(last)]
    stop = [torch.cuda.Event(enable_timing=True) for _ in range(last)]
    launch(0)
    torch.cuda.synchronize()
    for i in range(n):
        j = i - (n - last)
        if j >= 0:
            start[j].record()
        launch(i)
        if j >= 0:
            stop[j].record()
        torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(start, stop)) / last


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _dequantized_operands(dtype: str, M: int, N: int, K: int, seed: int, dev):
    """The BASELINE configuration's operands of `dtype`, drawn as make_case
    draws them (CPU generator, quantized on the GPU), dequantized to fp32 on
    the host with the oracle's formulas (not timed)."""
    import numpy as np
    import torch

    from gfx950_gluon_tutorials_amd import quant
    from oracle import gemm_ref as R

    gen = torch.Generator().manual_seed(seed)
    if dtype == "fp16":
        a = (torch.randn(M, K, generator=gen) * 0.1).half().float().numpy()
        b = (torch.randn(N, K, generator=gen) * 0.1).half().float().numpy()
        return a, b
    if dtype == "bf8":
        qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=gen).to(dev))
        qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=gen).to(dev))
        a = R.e5m2_to_f32(qa.view(torch.uint8).cpu().numpy()) * np.float32(sa.item())
        b = R.e5m2_to_f32(qb.view(torch.uint8).cpu().numpy()) * np.float32(sb.item())
        return a, b
    pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen).to(dev))
    pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen).to(dev))
    return (R.mxfp4_dequant(pa.cpu().numpy(), sa.cpu().numpy()),
            R.mxfp4_dequant(pb.cpu().numpy(), sb.cpu().numpy()))


def cpu_baseline(M: int, N: int, K: int, dev, seeds: dict) -> dict:
    """The reference's CPU path (torch.matmul in fp32 on the dequantized
    operands, oracle.gemm_ref.torch_matmul_f32) on this host, for the fp16,
    bf8 and mxfp4 configurations at their full size: 1 warm-up, then the
    median of 3; dequantization is outside the timing.  The headline fields
    are fp16's; per_dtype holds all three."""
    import torch

    from oracle import gemm_ref as R

    per = {}
    for dt in ("fp16", "bf8", "mxfp4"):
        a, b = _dequantized_operands(dt, M, N, K, seeds[dt], dev)
        R.torch_matmul_f32(a, b)  # warm-up
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            R.torch_matmul_f32(a, b)
            times.append(time.perf_counter() - t0)
        t = sorted(times)[1]
        per[dt] = {"tflops": round(2.0 * M * N * K / t / 1e12, 4), "seconds": round(t, 4),
                   "sample": f"full {M}x{N}x{K}, seed {seeds[dt]}"}
        print(f"# cpu baseline {dt}: {per[dt]['tflops']:.3f} TFLOPS ({t:.3f} s, torch.matmul fp32, "
              f"{torch.get_num_threads()} threads)", flush=True)
        del a, b
    return {
        "value": per["fp16"]["tflops"],
        "unit": "TFLOPS",
        "cores": int(torch.get_num_threads()),
        "kind": "port",
        "sample": f"torch.matmul fp32 of the dequantized operands at the full {M}x{N}x{K} size of each BASELINE "
                  f"configuration (fp16 seed 1, bf8 seed 2, mxfp4 seed 3), 1 warm-up then median of 3, "
                  f"dequantization untimed (oracle.gemm_ref.torch_matmul_f32); value = fp16",
        "per_dtype": per,
        "torch_threads": int(torch.get_num_threads()),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": _cpu_model(),
    }


def summarize_rocpd(path: str) -> None:
    """Per-kernel summary of rocprofv3 output (its SQLite ``*_results.db``):
    dispatch counts and durations from the kernel trace, and per-dispatch
    medians of every collected counter."""
    import glob
    import sqlite3
    import statistics as st

    dbs = sorted(glob.glob(os.path.join(path, "**", "*.db"), recursive=True))
    if not dbs:
        csvs = sorted(glob.glob(os.path.join(path, "**", "*_kernel_trace.csv"), recursive=True)
                      + glob.glob(os.path.join(path, "**", "*_counter_collection.csv"), recursive=True))
        if not csvs:
            print(f"no rocprofv3 databases or CSV files under {path}")
        for f in csvs:
            summarize_csv(f, path)
        return
    for db in dbs:
        con = sqlite3.connect(db)
        views = {r[0] for r in con.execute("select name from sqlite_master where type='view'")}
        print(f"== {os.path.relpath(db, path)}")
        if "kernels" in views:
            rows = con.execute("select name, grid_x, duration from kernels order by start").fetchall()
            # One group per consecutive run of a kernel among the GEMM kernels
            # (the same kernel at two shapes, e.g. K=8192 and the headline K,
            # gives two groups, the later one suffixed #2).  The split-K
            # reduction, launched after every split-K launch, does not end a run.
            groups, runs, last = {}, {}, None
            for name, grid, dur in rows:
                key = (name, grid)
                if name.startswith("g9_") and "splitk_reduce" not in name and key != last:
                    runs[key] = runs.get(key, 0) + 1
                    last = key
                n = runs.get(key, 1)
                gname = name if n == 1 else f"{name}#{n}"
                groups.setdefault((gname, grid), []).append(dur / 1e3)
            if groups:
                print(f"{'kernel':48s} {'grid':>8s} {'calls':>6s} {'mean_us':>9s} {'median_us':>9s} "
                      f"{'min_us':>8s} {'max_us':>8s} {'last100_mean_us':>15s}")
            for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
                print(f"{name[:48]:48s} {grid:8d} {len(d):6d} {st.mean(d):9.2f} {st.median(d):9.2f} "
                      f"{min(d):8.2f} {max(d):8.2f} {st.mean(d[-100:]):15.2f}")
        if "counters_collection" in views:
            cols = {r[1] for r in con.execute("pragma table_info(counters_collection)")}
            order = next((c for c in ("dispatch_id", "start", "start_time") if c in cols), None)
            disp = order if order else "0"
            rows = con.execute(f"select kernel_name, grid_size, counter_name, value, duration, {disp} "
                               "from counters_collection" + (f" order by {order}" if order else "")).fetchall()
            # Consecutive runs of a GEMM kernel (one per shape) are grouped
            # separately, as for the kernel trace: the later ones get #2, #3...
            groups, runs, last = {}, {}, None
            for name, grid, cn, val, dur, _ in rows:
                key = (name, grid)
                if name.startswith("g9_") and "splitk_reduce" not in name and key != last:
                    runs[key] = runs.get(key, 0) + 1
                    last = key
                n = runs.get(key, 1)
                gname = name if n == 1 else f"{name}#{n}"
                g = groups.setdefault((gname, grid), {"dur": []})
                g.setdefault(cn, []).append(val)
                g["dur"].append(dur / 1e3)
            for (name, grid), g in sorted(groups.items(), key=lambda kv: -sum(kv[1]["dur"])):
                n = len(g["dur"]) // max(1, len(g) - 1)
                vals = "  ".join(f"{cn}={st.median(v):.6g}" for cn, v in sorted(g.items()) if cn != "dur")
                print(f"{name[:48]:48s} grid={grid} dispatches={n} median_us={st.median(g['dur']):.2f}  {vals}")


def _runs(rows):
    """Groups (name, grid, payload) rows in dispatch order by kernel and grid,
    one group per consecutive run of a GEMM kernel (the same kernel at two
    shapes gives two groups, the later one suffixed #2; the split-K
    reduction, launched after every split-K launch, does not end a run)."""
    groups, runs, last = {}, {}, None
    for name, grid, payload in rows:
        key = (name, grid)
        if name.startswith("g9_") and "splitk_reduce" not in name and key != last:
            runs[key] = runs.get(key, 0) + 1
            last = key
        n = runs.get(key, 1)
        groups.setdefault((name if n == 1 else f"{name}#{n}", grid), []).append(payload)
    return groups


def summarize_csv(f: str, root: str) -> None:
    """The same summary from rocprofv3's CSV output (``--output-format csv``
    / ``-f csv``, as the reference's protocol runs it): a kernel trace
    (``*_kernel_trace.csv``: durations) or a counter collection
    (``*_counter_collection.csv``: per-dispatch counter medians)."""
    import csv
    import statistics as st

    with open(f, newline="") as fh:
        rows = list(csv.DictReader(fh))
    print(f"== {os.path.relpath(f, root)}")
    if not rows:
        return

    def grid(r):
        return int(r.get("Grid_Size") or r.get("Grid_Size_X") or 0) * int(r.get("Grid_Size_Y") or 1) * \
            int(r.get("Grid_Size_Z") or 1)

    def order(r):
        return int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0), int(r.get("Start_Timestamp") or 0)

    rows.sort(key=order)
    if "Counter_Name" not in rows[0]:
        groups = _runs((r["Kernel_Name"], grid(r), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                       for r in rows)
        print(f"{'kernel':48s} {'grid':>8s} {'calls':>6s} {'mean_us':>9s} {'median_us':>9s} "
              f"{'min_us':>8s} {'max_us':>8s} {'last100_mean_us':>15s}")
        for (name, g), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            print(f"{name[:48]:48s} {g:8d} {len(d):6d} {st.mean(d):9.2f} {st.median(d):9.2f} "
                  f"{min(d):8.2f} {max(d):8.2f} {st.mean(d[-100:]):15.2f}")
        return
    groups = _runs((r["Kernel_Name"], grid(r), r) for r in rows)
    for (name, g), rs in sorted(groups.items(), key=lambda kv: -len(kv[1])):
        by_counter, durs = {}, {}
        for r in rs:
            by_counter.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            durs[r.get("Dispatch_Id") or r["Start_Timestamp"]] = (int(r["End_Timestamp"]) -
                                                                 int(r["Start_Timestamp"])) / 1e3
        vals = "  ".join(f"{cn}={st.median(v):.6g}" for cn, v in sorted(by_counter.items()))
        print(f"{name[:48]:48s} grid={g} dispatches={len(durs)} median_us={st.median(durs.values()):.2f}  {vals}")


def streamk_fixups(tiles: int, stages: int, ctas: int) -> int:
    """Partial tiles handed from one stream-K workgroup to the next: the CTA
    range boundaries (c*base + min(c, rem)) that fall inside a tile."""
    total = tiles * stages
    base, rem = divmod(total, ctas)
    return sum(1 for c in range(1, ctas) if (c * base + min(c, rem)) % stages)


# Grouped (MoE) GEMM benchmark: 32 experts, 32768 routed tokens (1024 per expert
# on average, Dirichlet(5)-skewed), N = 4096 (a fused gate/up projection), K = 7168.
MOE_SHAPE = {"E": 32, "T": 32768, "N": 4096, "K": 7168}


def moe_counts(E: int, T: int, seed: int = 7):
    """Tokens per expert: a seeded multinomial draw from Dirichlet(5) shares."""
    import numpy as np

    rng = np.random.default_rng(seed)
    return rng.multinomial(T, rng.dirichlet([5.0] * E))


def make_moe_case(dtype: str, dev, nsets: int, seed: int = 8):
    """Returns (launch(i), counts): the grouped GEMM on operand set i.  The
    operands are generated on the device (seeded) to keep set-up short."""
    import numpy as np
    import torch

    from gfx950_gluon_tutorials_amd import quant
    from gfx950_gluon_tutorials_amd.gemm.moe import moe_matmul, moe_matmul_a4w4, moe_matmul_a8w8

    E, T, N, K = (MOE_SHAPE[k] for k in ("E", "T", "N", "K"))
    counts = moe_counts(E, T)
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(seed)
    sets = []
    for _ in range(nsets):
        a = torch.randn(T, K, generator=gen, device=dev)
        if dtype == "fp16":
            b = torch.randn(E, N, K, generator=gen, device=dev, dtype=torch.float16)
            sets.append((a.half(), b, torch.empty(T, N, dtype=torch.float16, device=dev)))
        elif dtype == "bf8":
            qa, sa = quant.quantize_e5m2(a)
            qb = torch.empty(E, N, K, dtype=torch.float8_e5m2, device=dev)
            sb = torch.empty(E, dtype=torch.float32, device=dev)
            for e in range(E):
                qb[e], sb[e] = quant.quantize_e5m2(torch.randn(N, K, generator=gen, device=dev))
            sets.append((qa, qb, sa, sb, torch.empty(T, N, dtype=torch.bfloat16, device=dev)))
        else:
            pa, sa = quant.quantize_mxfp4(a)
            pb = torch.empty(E, N, K // 2, dtype=torch.uint8, device=dev)
            sb = torch.empty(E, N, K // 32, dtype=torch.uint8, device=dev)
            for e in range(E):
                pb[e], sb[e] = quant.quantize_mxfp4(torch.randn(N, K, generator=gen, device=dev))
            sets.append((pa, pb, sa, sb, torch.empty(T, N, dtype=torch.bfloat16, device=dev)))
        del a

    def launch(i, schedule="dp"):
        x = sets[i % nsets]
        if dtype == "fp16":
            moe_matmul(x[0], x[1], off, x[2])
        elif dtype == "bf8":
            moe_matmul_a8w8(x[0], x[1], off, x[4], a_scale=x[2], b_scales=x[3])
        else:
            moe_matmul_a4w4(x[0], x[1], x[2], x[3], off, x[4])

    return launch, counts


# K sweep of the reference benches (kernels/gemm/intra_wave/a16w16/bench.py:85-95, a8w8/bench.py:73-82,
# a4w4/bench.py:167-177) and the reference's published TFLOPS at M=N=4096 (4-wave, 8-wave):
# kernels/gemm/inter_wave/a16w16/README.md:120-122, inter_wave/a8w8/README.md:61-63,
# inter_wave/a4w4/v0_sliceMN/README.md:60-62 (4-wave) and inter_wave/a4w4/README.md:13-21 (8-wave, v2).
KSWEEP = {
    "fp16": [512, 1024, 2048, 3072, 4096, 8192, 16384, 32768],
    "bf8": [1024, 2048, 3072, 4096, 8192, 16384, 32768],
    "mxfp4": [1024, 2048, 3072, 4096, 8192, 16384, 32768, 65536],
}
KSWEEP_REF = {
    "fp16": {8192: (1608, 1478), 16384: (1651, 1529), 32768: (1432, 1328)},
    "bf8": {8192: (3215, 2949), 16384: (3476, 3131), 32768: (3090, 3202)},
    "mxfp4": {8192: (4986, 4479), 16384: (5550, 4900), 32768: (5804, 5196)},
}


def ksweep(args, dev) -> dict:
    import torch

    seeds = {"fp16": 1, "bf8": 2, "mxfp4": 3}
    out = {}
    for dt, ks in KSWEEP.items():
        for kk in ks:
            for w in (4, 8):
                rotate = args.rotate_mb if kk < 16384 else max(args.rotate_mb, 2048)
                nsets = max(2, -(-rotate * 2**20 // set_bytes(dt, 4096, 4096, kk)))
                launch = make_case(dt, 4096, 4096, kk, seeds[dt], dev, nsets, w)
                ms = time_case(launch, max(20, args.steps // 2), args.warmup // 2, settle_s=args.settle_ms / 2e3)
                tf = 2.0 * 4096 * 4096 * kk / (ms * 1e-3) / 1e12
                ref = KSWEEP_REF[dt].get(kk, (None, None))[0 if w == 4 else 1]
                out[f"{dt}_k{kk}_{w}w"] = {"tflops": round(tf, 2), "ms": round(ms, 5), "reference_tflops": ref}
                print(f"# ksweep {dt:5s} K={kk:<6d} {w}w: {ms * 1e3:8.1f} us  {tf:7.1f} TFLOPS"
                      + (f"  | reference {ref}" if ref else ""), flush=True)
                del launch
                torch.cuda.empty_cache()
    return out


def make_vendor_case(dtype: str, M: int, N: int, K: int, seed: int, dev, nsets: int):
    """launch(i) running ROCm's library GEMM (hipBLASLt through torch) on the
    same kind of operands as make_case: torch.matmul for fp16/bf16,
    torch._scaled_mm (e5m2 x e5m2 -> bf16, per-tensor scales) for bf8, and
    torch._scaled_mm on float4_e2m1fn_x2 operands with float8_e8m0fnu per-32
    scales (-> bf16) for mxfp4."""
    import torch

    from gfx950_gluon_tutorials_amd import quant

    gen = torch.Generator().manual_seed(seed)
    sets = []
    for _ in range(nsets):
        if dtype in ("fp16", "bf16"):
            tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
            a = (torch.randn(M, K, generator=gen) * 0.1).to(tdt).to(dev)
            b = (torch.randn(N, K, generator=gen) * 0.1).to(tdt).to(dev)
            sets.append((a, b, torch.empty(M, N, dtype=tdt, device=dev)))
        elif dtype == "bf8":
            qa, sa = quant.quantize_e5m2(torch.randn(M, K, generator=gen).to(dev))
            qb, sb = quant.quantize_e5m2(torch.randn(N, K, generator=gen).to(dev))
            sets.append((qa, qb, sa.reshape(()).float(), sb.reshape(()).float()))
        else:
            pa, sa = quant.quantize_mxfp4(torch.randn(M, K, generator=gen).to(dev))
            pb, sb = quant.quantize_mxfp4(torch.randn(N, K, generator=gen).to(dev))
            sets.append((pa.view(torch.float4_e2m1fn_x2), pb.view(torch.float4_e2m1fn_x2),
                         sa.view(torch.float8_e8m0fnu).flatten(), sb.view(torch.float8_e8m0fnu).flatten()))

    def launch(i, schedule="dp"):
        x = sets[i % nsets]
        if dtype in ("fp16", "bf16"):
            torch.matmul(x[0], x[1].T, out=x[2])
        else:
            torch._scaled_mm(x[0], x[1].T, scale_a=x[2], scale_b=x[3], out_dtype=torch.bfloat16)

    launch(0)  # raises here if the library has no kernel for this case
    torch.cuda.synchronize()
    return launch


def fmha_bench(args, dev) -> dict:
    """Flash-attention forward (g9_fmha_fwd through run_gluon_attention), bhsd,
    non-causal, fmha_v4 (lazy rescale) and fmha_v3 (eager), bf16 and fp16, at
    FMHA_SHAPE.  One (q, k, v, o) set is 2 GiB, far beyond the caches, so no
    rotation (the reference's rotating_set_count gives 1 for this shape,
    kernels/attention/bench.py:186-199).  FLOPs: 4 B H S^2 D
    (kernels/attention/common.py:177-184)."""
    import torch

    from gfx950_gluon_tutorials_amd.attention import MetaData, compute_flops, fmha_v3, fmha_v4

    B, H, S, D = (FMHA_SHAPE[k] for k in ("B", "H", "S", "D"))
    flop = compute_flops(B, H, S, S, D, False)
    out = {}
    for dt, tdt in (("bf16", torch.bfloat16), ("fp16", torch.float16)):
        g = torch.Generator(device=dev).manual_seed(20)
        q, k, v = (torch.randn(B, H, S, D, device=dev, dtype=tdt, generator=g) for _ in range(3))
        o = torch.empty_like(q)
        md = MetaData(sm_scale=D**-0.5)
        md.max_seqlens_q = md.max_seqlens_k = S
        md.layout = "bhsd"
        for variant, fn in ((4, fmha_v4.run_gluon_attention), (3, fmha_v3.run_gluon_attention)):
            def launch(i, schedule="dp", fn=fn):
                fn(q, k, v, o, md)

            if args.fmha_only:
                ms = time_case(launch, args.steps, args.warmup, settle_s=args.settle_ms / 1e3)
            else:
                ms = time_case(launch, max(10, args.steps // 10), max(3, args.warmup // 20), settle_s=args.settle_ms / 2e3)
            tf = flop / (ms * 1e-3) / 1e12
            ref = FMHA_REFERENCE_TFLOPS.get((dt, variant))
            key = f"{dt}_v{variant}"
            out[key] = {"tflops": round(tf, 2), "ms": round(ms, 5), "frac_of_peak": round(tf / PEAK[dt], 4),
                        "reference_tflops": ref, "vs_reference": round(tf / ref, 4) if ref else None}
            print(f"# fmha_v{variant} {dt} B={B} H={H} S={S} D={D}: {ms * 1e3:.1f} us  {tf:.1f} TFLOPS  "
                  f"{100 * tf / PEAK[dt]:.1f}% of peak" + (f"  | reference {ref:.0f}" if ref else ""), flush=True)
        del q, k, v, o
        torch.cuda.empty_cache()
    out["shape"] = dict(FMHA_SHAPE, layout="bhsd", causal=False)
    return out


def fmha_sweep(args, dev) -> dict:
    """The reference attention bench's sequence-length sweep (B=1, HQ=HK=64,
    bhsd, non-causal, bf16) for head dims 128 and 64, fmha_v4 and fmha_v3:
    HIP-event time of back-to-back launches over enough rotating (q, k, v, o)
    sets to exceed 512 MiB, as the reference's rotating_set_count does
    (kernels/attention/bench.py:186-199)."""
    import torch

    from gfx950_gluon_tutorials_amd.attention import MetaData, compute_flops, fmha_v3, fmha_v4

    B, H = FMHA_SWEEP_SHAPE["B"], FMHA_SWEEP_SHAPE["H"]
    out = {}
    for D in (128, 64):
        for S in FMHA_SWEEP_SEQLENS:
            per_set = 4 * B * H * S * D * 2
            nsets = max(1, -(-(512 << 20) // per_set))
            g = torch.Generator(device=dev).manual_seed(S + D)
            sets = []
            for _ in range(nsets):
                q, k, v = (torch.randn(B, H, S, D, device=dev, dtype=torch.bfloat16, generator=g) for _ in range(3))
                sets.append((q, k, v, torch.empty_like(q)))
            md = MetaData(sm_scale=D**-0.5)
            md.max_seqlens_q = md.max_seqlens_k = S
            md.layout = "bhsd"
            flop = compute_flops(B, H, S, S, D, False)
            for variant, fn in ((4, fmha_v4.run_gluon_attention), (3, fmha_v3.run_gluon_attention)):
                def launch(i, schedule="dp", fn=fn):
                    fn(*sets[i % nsets], md)

                ms = time_case(launch, args.steps, args.warmup, settle_s=args.settle_ms / 1e3)
                tf = flop / (ms * 1e-3) / 1e12
                out[f"d{D}_s{S}_v{variant}"] = {"tflops": round(tf, 2), "ms": round(ms, 5), "sets": nsets}
                print(f"# fmha_v{variant} bf16 B={B} H={H} S={S} D={D}: {ms * 1e3:.1f} us  {tf:.1f} TFLOPS "
                      f"({nsets} set(s))", flush=True)
            del sets
            torch.cuda.empty_cache()
    out["shape"] = dict(FMHA_SWEEP_SHAPE, layout="bhsd", causal=False, dtype="bf16")
    return out


def energy_study(args, dev) -> dict:
    """Energy per 4096x4096x8192 launch of our 4-wave data-parallel kernel and
    of hipBLASLt's (torch.matmul) for fp16 and bf16, on one box: each side runs
    back to back for args.energy seconds while amd-smi samples board power and
    GFX clock (telemetry), in two interleaved rounds; energy = median power x
    median launch time over the second half of each window."""
    import statistics as st

    import torch

    M = N = 4096
    K = 8192
    out = {}
    for dt in ("fp16", "bf16"):
        nsets = max(2, -(-args.rotate_mb * 2**20 // set_bytes(dt, M, N, K)))
        sides = {"ours": make_case(dt, M, N, K, 1, dev, nsets, 4), "hipblaslt": make_vendor_case(dt, M, N, K, 1, dev, nsets)}
        runs = {k: [] for k in sides}
        for _ in range(2):
            for name, launch in sides.items():
                tel = telemetry(launch, args.energy)
                if tel:
                    tel["energy_mj"] = round(tel["power_w"] * tel["launch_us"] * 1e-3, 2)
                    runs[name].append(tel)
                    print(f"# energy {dt} {name}: {tel['launch_us']:.1f} us at {tel['power_w']:.0f} W, "
                          f"{tel['gfx_clock_mhz']} MHz -> {tel['energy_mj']:.1f} mJ per launch", flush=True)
        out[dt] = {k: {"runs": v, "energy_mj": round(st.median(r["energy_mj"] for r in v), 2) if v else None,
                       "launch_us": round(st.median(r["launch_us"] for r in v), 2) if v else None}
                   for k, v in runs.items()}
        del sides
        torch.cuda.empty_cache()
    return out


def moe_set_bytes(dtype: str) -> int:
    E, T, N, K = (MOE_SHAPE[k] for k in ("E", "T", "N", "K"))
    if dtype == "fp16":
        return 2 * (T * K + E * N * K + T * N)
    if dtype == "bf8":
        return T * K + E * N * K + 2 * T * N
    return (T * K + E * N * K) // 2 + (T + E * N) * K // 32 + 2 * T * N


def load_traffic(key: str):
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def main():
    args = parse_args()
    if args.summarize:
        summarize_rocpd(args.summarize)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(the GEMM shards over output rows with no communication; one GPU's share "
                                   "is what --gpus 1 measures; nothing multi-GPU is launched)"}))
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    M = N = 4096
    K = 8192
    if args.ksweep:
        print(json.dumps({"ksweep": ksweep(args, dev)}))
        return
    if args.pair:
        dt = args.only or "fp16"
        seed = {"fp16": 1, "bf16": 1, "bf8": 2}[dt]
        ours, lib = make_case(dt, M, N, K, seed, dev, 4, 4), make_vendor_case(dt, M, N, K, seed, dev, 4)
        for i in range(args.pair):
            ours(i, "dp")
        torch.cuda.synchronize()
        for i in range(args.pair):
            lib(i)
        torch.cuda.synchronize()
        print(f"# pair: {args.pair} launches each of ours and hipBLASLt ({dt})", flush=True)
        return
    if args.fmha_only:
        print(json.dumps({"fmha": fmha_bench(args, dev)}), flush=True)
        return
    if args.fmha_sweep:
        print(json.dumps({"fmha_sweep": fmha_sweep(args, dev)}), flush=True)
        return
    if args.energy:
        print(json.dumps({"energy": energy_study(args, dev)}), flush=True)
        return
    dtypes = [d for d in args.dtypes.split(",") if d]
    if args.only:
        dtypes = [args.only]
    seeds = {"fp16": 1, "bf16": 1, "bf8": 2, "mxfp4": 3, "mxfp4ps": 3, "mxfp4km": 3}
    results = {}
    waves = [int(w) for w in args.waves.split(",") if w]
    cases = [(dt, K, w, REFERENCE_TFLOPS.get(dt) if w == 4 else REFERENCE_TFLOPS_8W.get(dt), args.rotate_mb)
             for dt in dtypes for w in waves if not (dt in FOUR_WAVE_ONLY and w == 8)]
    if args.headline_k and not args.only:
        for dt, (kk, r4, r8) in HEADLINE_K.items():
            if dt in dtypes:
                cases += [(dt, kk, w, r4 if w == 4 else r8, max(args.rotate_mb, 2048)) for w in waves
                          if not (dt in FOUR_WAVE_ONLY and w == 8)]
    for dt, kk, w, ref, rotate_mb in cases:
        nsets = max(2, -(-rotate_mb * 2**20 // set_bytes(dt, M, N, kk)))
        launch = make_case(dt, M, N, kk, seeds[dt], dev, nsets, w, prepared=bool(args.prepared))
        ms = time_case(launch, args.steps, args.warmup, settle_s=args.settle_ms / 1e3)
        tf = 2.0 * M * N * kk / (ms * 1e-3) / 1e12
        key = dt + ("" if kk == K else f"_k{kk}") + ("" if w == 4 else "_8w")
        results[key] = {"tflops": round(tf, 2), "ms": round(ms, 5), "frac_of_peak": round(tf / PEAK[dt], 4),
                        "reference_tflops": ref, "K": kk, "rotating_sets": nsets, "waves": w,
                        "launch": "prepared" if args.prepared else "matmul"}
        if dt in SCALE_LAYOUTS:
            results[key]["scales"] = SCALE_LAYOUTS[dt]
        msg = f"# {key}: {ms * 1e3:.1f} us  {tf:.1f} TFLOPS  {100 * tf / PEAK[dt]:.1f}% of peak"
        if args.serialized:
            ms_s = time_serialized(launch)
            tf_s = 2.0 * M * N * kk / (ms_s * 1e-3) / 1e12
            results[key]["serialized_tflops"] = round(tf_s, 2)
            results[key]["serialized_ms"] = round(ms_s, 5)
            msg += f"  | serialized, event-timed {ms_s * 1e3:.1f} us {tf_s:.1f} TFLOPS"
        if ref:
            msg += f"  | reference {ref:.0f}"
        print(msg, flush=True)
        if args.telemetry_s > 0 and not args.only and kk == K and w == 4:
            tel = telemetry(launch, args.telemetry_s)
            if tel:
                tel["tflops"] = round(2.0 * M * N * kk / tel["launch_us"] / 1e6, 1)
                results[key]["telemetry"] = tel
                print(f"#   steady state {tel['launch_us']:.1f} us ({tel['tflops']:.0f} TFLOPS) at "
                      f"{tel['power_w']:.0f} W, GFX clock {tel['gfx_clock_mhz']} MHz (amd-smi, {tel['samples']} samples)",
                      flush=True)
        if args.vendor and not args.only and kk == K and w == 4 and dt in ("fp16", "bf16", "bf8", "mxfp4", "mxfp4ps",
                                                                          "mxfp4km"):
            try:
                vlaunch = make_vendor_case("mxfp4" if dt in FOUR_WAVE_ONLY else dt, M, N, kk, seeds[dt], dev, nsets)
            except Exception as e:  # no library kernel for this type on this build
                results[key]["vendor"] = {"library": "hipBLASLt via torch", "error": str(e).splitlines()[0][:120]}
            else:
                # interleaved, three rounds each, so board drift hits both equally
                t_ours, t_lib = [], []
                for _ in range(3):
                    t_ours.append(time_case(launch, max(20, args.steps // 2), 20, settle_s=0.3))
                    t_lib.append(time_case(vlaunch, max(20, args.steps // 2), 20, settle_s=0.3))
                mo, ml = sorted(t_ours)[1], sorted(t_lib)[1]
                tf_o, tf_l = 2.0 * M * N * kk / (mo * 1e-3) / 1e12, 2.0 * M * N * kk / (ml * 1e-3) / 1e12
                results[key]["vendor"] = {"library": "hipBLASLt via torch." + ("matmul" if dt in ("fp16", "bf16") else "_scaled_mm"),
                                          "tflops": round(tf_l, 2), "ours_interleaved_tflops": round(tf_o, 2),
                                          "ours_over_library": round(tf_o / tf_l, 4)}
                print(f"#   same box, interleaved: ours {tf_o:.1f} vs hipBLASLt {tf_l:.1f} TFLOPS ({tf_o / tf_l:.3f}x)",
                      flush=True)
                del vlaunch
        del launch
        torch.cuda.empty_cache()
    sk = {}
    if args.streamk and not args.only:
        # The BASELINE shapes (fewer tiles than CUs), then two with more: 272 and 400 tiles.
        for (m, n, k) in [(3840, 3840, 16384), (8192, 1280, 8192), (4352, 4096, 8192), (5120, 5120, 8192)]:
            launch = make_case("fp16", m, n, k, 4, dev, max(2, -(-args.rotate_mb * 2**20 // set_bytes("fp16", m, n, k))))
            ms_dp = time_case(launch, max(10, args.steps // 2), args.warmup, "dp", args.settle_ms / 2e3)
            ms_sk = time_case(launch, max(10, args.steps // 2), args.warmup, "streamk", args.settle_ms / 2e3)
            # Stream-K over 256x128 tiles (twice the tiles; bit-identical as well).
            ms_skh = time_case(launch, max(10, args.steps // 2), args.warmup, "streamk_half", args.settle_ms / 2e3)
            flop = 2.0 * m * n * k
            from gfx950_gluon_tutorials_amd import _lib

            tiles, stages = -(-m // 256) * -(-n // 256), k // 64
            ctas = min(tiles * stages, _lib.load().g9_streamk_workgroups())
            fix = streamk_fixups(tiles, stages, ctas)
            tiles_h = -(-m // 256) * -(-n // 128)
            ctas_h = min(tiles_h * stages, _lib.load().g9_streamk_workgroups())
            fix_h = streamk_fixups(tiles_h, stages, ctas_h)
            sk[f"{m}x{n}x{k}"] = {"dp_tflops": round(flop / ms_dp / 1e9, 2), "sk_tflops": round(flop / ms_sk / 1e9, 2),
                                  "sk_half_tflops": round(flop / ms_skh / 1e9, 2),
                                  "dp_ms": round(ms_dp, 5), "sk_ms": round(ms_sk, 5), "sk_half_ms": round(ms_skh, 5),
                                  "sk_workgroups": ctas, "fixups": fix, "fixup_bytes": fix * 2 * 256 * 256 * 4,
                                  "sk_half_tiles": tiles_h, "sk_half_fixups": fix_h,
                                  "sk_half_fixup_bytes": fix_h * 2 * 256 * 128 * 4}
            print(f"# stream-K {m}x{n}x{k}: dp {flop / ms_dp / 1e9:.1f}  sk {flop / ms_sk / 1e9:.1f}  "
                  f"sk 256x128 {flop / ms_skh / 1e9:.1f} TFLOPS  ({ctas} workgroups, {fix} partial-tile handoffs = "
                  f"{fix * 0.5:.0f} MiB fp32 written+read; 256x128: {tiles_h} tiles, {fix_h} handoffs)",
                  flush=True)
            del launch
            torch.cuda.empty_cache()
    splitk = {}
    if args.splitk and not args.only:
        from gfx950_gluon_tutorials_amd import _lib

        lib = _lib.load()
        codes = {"fp16": _lib.G9_F16, "bf8": _lib.G9_BF8, "mxfp4": _lib.G9_FP4}
        stage_k = {"fp16": 64, "bf8": 128, "mxfp4": 256}
        # Few-row GEMMs and one GPU's shard of a row-sharded 4096 x 4096 x 8192
        # GEMM (512 rows = 1/8): 16-128 tiles, so data-parallel leaves CUs idle.
        for (dt, m, n, k) in [("fp16", 256, 4096, 8192), ("fp16", 512, 4096, 8192), ("fp16", 1024, 4096, 8192),
                              ("fp16", 2048, 4096, 8192), ("bf8", 512, 4096, 8192), ("mxfp4", 512, 4096, 8192)]:
            launch = make_case(dt, m, n, k, 5, dev, max(2, -(-args.rotate_mb * 2**20 // set_bytes(dt, m, n, k))))
            ms_dp = time_case(launch, max(20, args.steps // 2), 20, "dp", 0.3)
            ms_sp = time_case(launch, max(20, args.steps // 2), 20, "splitk", 0.3)
            flop = 2.0 * m * n * k
            tiles = -(-m // 256) * -(-n // 256)
            S = lib.g9_splitk_factor(tiles, k // stage_k[dt], lib.g9_streamk_workgroups())
            ws = lib.g9_workspace_size(codes[dt], m, n, k, _lib.G9_SCHED_SPLITK, 4)
            splitk[f"{dt}_{m}x{n}x{k}"] = {"dp_tflops": round(flop / ms_dp / 1e9, 2),
                                           "splitk_tflops": round(flop / ms_sp / 1e9, 2), "dp_ms": round(ms_dp, 5),
                                           "splitk_ms": round(ms_sp, 5), "tiles": tiles, "split": S,
                                           "workspace_bytes": ws}
            print(f"# split-K {dt} {m}x{n}x{k} ({tiles} tiles, {S} segments): dp {flop / ms_dp / 1e9:.1f}  "
                  f"splitk {flop / ms_sp / 1e9:.1f} TFLOPS ({ms_dp / ms_sp:.2f}x)", flush=True)
            del launch
            torch.cuda.empty_cache()
    moe = {}
    if args.moe and not args.only:
        E, T, N, K_ = (MOE_SHAPE[k] for k in ("E", "T", "N", "K"))
        for dt in ("mxfp4", "bf8", "fp16"):
            nsets = max(2, -(-args.rotate_mb * 2**20 // moe_set_bytes(dt)))
            launch, counts = make_moe_case(dt, dev, nsets)
            ms = time_case(launch, max(20, args.steps // 4), args.warmup // 4, settle_s=args.settle_ms / 2e3)
            flop = 2.0 * T * N * K_
            padded = sum(-(-int(c) // 256) * 256 for c in counts)
            tf = flop / (ms * 1e-3) / 1e12
            moe[dt] = {"tflops": round(tf, 2), "ms": round(ms, 5), "frac_of_peak": round(tf / PEAK[dt], 4),
                       "experts": E, "tokens": T, "N": N, "K": K_, "rotating_sets": nsets,
                       "min_max_tokens": [int(counts.min()), int(counts.max())],
                       "row_utilization": round(T / padded, 4)}
            print(f"# moe {dt}: E={E} T={T} N={N} K={K_} (tokens/expert {counts.min()}-{counts.max()}): "
                  f"{ms * 1e3:.1f} us  {tf:.1f} TFLOPS  {100 * tf / PEAK[dt]:.1f}% of peak  "
                  f"(256-row tiles {100 * T / padded:.1f}% filled)", flush=True)
            del launch
            torch.cuda.empty_cache()
    fmha = fmha_bench(args, dev) if args.fmha and not args.only else {}
    overhead = {}
    if args.launch_overhead and not args.only:
        try:  # an auxiliary figure: a failure here must not cost the headline line
            overhead = launch_overhead(dev)
        except Exception as e:  # noqa: BLE001 (reported in the JSON line instead)
            overhead = {"error": f"{type(e).__name__}: {e}"}
            print(f"# launch overhead not measured: {overhead['error']}", flush=True)
    if args.copy_mb:
        copy_calibration(args.copy_mb, dev)
    head = "fp16" if "fp16" in results else next(iter(results))
    r = results[head]
    line = {
        "metric": "TFLOPS & % of MFMA peak, 4096x4096x8192 fp16/bf8/mxfp4, 1xMI355X",
        "value": r["tflops"],
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": r["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(r["tflops"] / REFERENCE_TFLOPS[head], 4) if head in REFERENCE_TFLOPS else None,
        "dtype": head.split("_")[0],
        "data": "synthetic",
        "config": {"workload": f"{head} NT GEMM C=A.B^T, M=N=4096, K=8192, 256x256 tiles, data-parallel, 4-wave; "
                               f"operands rotate over {r['rotating_sets']} resident sets",
                   "M": M, "N": N, "K": K},
        "roofline": {"bound": "mfma", "achieved": r["tflops"], "peak": PEAK[head.split("_")[0]], "unit": "TFLOP/s",
                     "frac": r["frac_of_peak"], "traffic": load_traffic(f"{head}_{M}x{N}x{K}")},
        "per_dtype": results,
        "streamk": sk,
        "splitk": splitk,
        "moe": moe,
        "fmha": fmha,
        "launch_overhead": overhead,
    }
    if args.cpu_baseline and not args.only:
        line["cpu_baseline"] = cpu_baseline(M, N, K, dev, seeds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
