"""Per-family GEMM bench: the command-line surface of the reference's
kernels/gemm/{intra,inter}_wave/{a16w16,a8w8,a4w4}/bench.py on this library.

    python -m gfx950_gluon_tutorials_amd.gemm.intra_wave.a16w16.bench [--K 8192] [--dtype fp16 bf16]
    python -m gfx950_gluon_tutorials_amd.gemm.inter_wave.a4w4.bench --K 32768 --rocprof

Like the reference (a16w16/bench.py:85-166, 244-303; a8w8/bench.py:73-142;
a4w4/bench.py:115-240) it first checks every selected M x N x K (M = N = 4096,
the reference's K list) against torch's fp32 product of the reference's
inputs (a16w16 and a8w8: ``rand - 0.5``; a4w4: random nibbles with E8M0
scales in [124, 128) in the transposed K-major view the reference builds)
with the reference's ``atol=0.1`` plus half an ulp of the output type as
``rtol`` (the reference compares with torch's own 16-bit output, whose
rounding can differ from a correct result by an ulp), printing match /
differ; then either prints
TFLOPS per size and dtype (median of timed back-to-back launches), or, with
``--rocprof``, issues ``--iters`` launches over rotating operand sets of at
least ``--rotating-buffer-size`` MiB for an external ``rocprofv3
--kernel-trace``, through prepared launches as the reference's
scripts/benchmark_prepared.py does.  There is one kernel per family here, so
the reference's ``--version`` is accepted only as its final version.
"""

from __future__ import annotations

import argparse

import torch

from ... import quant

K_LISTS = {
    "a16w16": (512, 1024, 2048, 3072, 4096, 8192, 16384, 32768),
    "a8w8": (1024, 2048, 3072, 4096, 8192, 16384, 32768),
    "a4w4": (1024, 2048, 3072, 4096, 8192, 16384, 32768, 65536),
}
DTYPES = {"a16w16": ("fp16", "bf16"), "a8w8": ("f8",), "a4w4": ("mxfp4",)}
M_N = 4096


def gemm_sizes(family: str, k: int | None = None) -> list[tuple[int, int, int]]:
    sizes = [(M_N, M_N, kk) for kk in K_LISTS[family]]
    if k is None:
        return sizes
    picked = [s for s in sizes if s[2] == k]
    if not picked:
        raise ValueError(f"No GEMM size found with K={k}. Available K values: {list(K_LISTS[family])}")
    return picked


def parse_args(family: str, argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=f"{family} GEMM benchmark (gfx950)")
    p.add_argument("--K", type=int, default=None, help="select the GEMM size with this K")
    if family == "a16w16":
        p.add_argument("--dtype", nargs="+", choices=["fp16", "bf16"], default=None,
                       help="data type(s) to benchmark (default: fp16 bf16)")
    p.add_argument("--version", type=int, default=None,
                   help="accepted for the reference's command lines; this library has one kernel per family")
    p.add_argument("--rocprof", action="store_true",
                   help="issue --iters launches over rotating operand sets for rocprofv3 --kernel-trace")
    p.add_argument("--rotating-buffer-size", type=int, default=512,
                   help="total MiB of the rotating operand sets in --rocprof mode (default 512)")
    p.add_argument("--iters", type=int, default=1000, help="launches per size in --rocprof mode")
    return p.parse_args(argv)


def _inputs(family: str, dtype: str, M: int, N: int, K: int, dev, gen: torch.Generator):
    """Operands as the reference's benches build them, and the fp32 torch
    product of the same values to compare with."""
    if family == "a16w16":
        tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
        a = (torch.rand(M, K, generator=gen) - 0.5).to(tdt).to(dev)
        b = (torch.rand(N, K, generator=gen) - 0.5).to(tdt).to(dev)
        return (a, b.T), a.float() @ b.float().T
    if family == "a8w8":
        a = (torch.rand(M, K, generator=gen) - 0.5).half().to(torch.float8_e5m2).to(dev)
        b = (torch.rand(N, K, generator=gen) - 0.5).half().to(torch.float8_e5m2).to(dev)
        return (a, b.T), a.float() @ b.float().T
    a = (torch.randint(0, 16, (M, K // 2), generator=gen, dtype=torch.uint8)
         | (torch.randint(0, 16, (M, K // 2), generator=gen, dtype=torch.uint8) << 4)).to(dev)
    b = (torch.randint(0, 16, (N, K // 2), generator=gen, dtype=torch.uint8)
         | (torch.randint(0, 16, (N, K // 2), generator=gen, dtype=torch.uint8) << 4)).to(dev)
    sa = torch.randint(124, 128, (K // 32, M), generator=gen, dtype=torch.uint8).to(dev).T
    sb = torch.randint(124, 128, (K // 32, N), generator=gen, dtype=torch.uint8).to(dev).T
    return (a, b, sa, sb), quant.dequantize_mxfp4(a, sa) @ quant.dequantize_mxfp4(b, sb).T


def check(family: str, matmul, dtypes, sizes, dev) -> bool:
    ok = True
    gen = torch.Generator().manual_seed(42)
    for dtype in dtypes:
        for M, N, K in sizes:
            args, want = _inputs(family, dtype, M, N, K, dev, gen)
            got = matmul(*args).float()
            # The reference's atol, plus half an ulp of the output type: the
            # rounding of a correct result never reads as a difference.
            rtol = 2.0**-11 if family != "a4w4" and dtype != "bf16" else 2.0**-8
            match = torch.allclose(got, want, atol=1e-1, rtol=rtol)
            ok &= match
            tag = "match" if match else f"differ (max_diff={(got - want).abs().max().item():.4f})"
            print(f"[{family}] M={M} N={N} K={K} dtype={dtype}: gfx950 and torch {tag}", flush=True)
    return ok


def _rotating(family, dtype, M, N, K, dev, mb):
    one = {"a16w16": (M * K + N * K + M * N) * 2, "a8w8": M * K + N * K + 2 * M * N,
           "a4w4": (M * K + N * K) // 2 + (M + N) * K // 32 + 2 * M * N}[family]
    gen = torch.Generator().manual_seed(0)
    return [_inputs(family, dtype, M, N, K, dev, gen)[0] for _ in range(max(2, -(-mb * 2**20 // one)))]


def _prepared(family, dtype, sets, waves):
    from ..prepared import PreparedGemm

    M = sets[0][0].shape[0]
    N = sets[0][1].shape[0] if family == "a4w4" else sets[0][1].shape[1]
    if family == "a16w16":
        tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
        return PreparedGemm.a16w16([(a, b, torch.empty(M, N, dtype=tdt, device=a.device)) for a, b in sets],
                                   waves=waves)
    if family == "a8w8":
        return PreparedGemm.a8w8([(a, b, torch.empty(M, N, dtype=torch.float16, device=a.device), None, None)
                                  for a, b in sets], waves=waves)
    # The 8-wave kernels read row-major scales: the K-major views are copied
    # once here, outside the launches (the matmul wrapper does it per call).
    return PreparedGemm.a4w4([(a, b, sa if waves == 4 else sa.contiguous(), sb if waves == 4 else sb.contiguous(),
                               torch.empty(M, N, dtype=torch.bfloat16, device=a.device)) for a, b, sa, sb in sets],
                             waves=waves)


def timed_tflops(matmul, args, M, N, K, reps: int = 100) -> float:
    """Median over `reps` event-timed launches (after 25 warm-up launches) of
    2*M*N*K / t, as triton.testing.do_bench's median feeds the reference's
    perf report."""
    for _ in range(25):
        matmul(*args)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        matmul(*args)
        e1.record()
        times.append((e0, e1))
    torch.cuda.synchronize()
    ms = sorted(e0.elapsed_time(e1) for e0, e1 in times)[len(times) // 2]
    return 2.0 * M * N * K / (ms * 1e-3) / 1e12


def main(family: str, matmul, waves: int, argv=None) -> int:
    args = parse_args(family, argv)
    dev = torch.device("cuda", torch.cuda.current_device())
    sizes = gemm_sizes(family, args.K)
    dtypes = (args.dtype or list(DTYPES[family])) if family == "a16w16" else list(DTYPES[family])
    ok = check(family, matmul, dtypes, sizes, dev)
    if args.rocprof:
        for dtype in dtypes:
            for M, N, K in sizes:
                sets = _rotating(family, dtype, M, N, K, dev, args.rotating_buffer_size)
                prepared = _prepared(family, dtype, sets, waves)
                for i in range(args.iters):
                    prepared(i)
                torch.cuda.synchronize()
                print(f"[{family}] M={M} N={N} K={K} dtype={dtype}: {args.iters} iterations done", flush=True)
                del prepared, sets
        return 0 if ok else 1
    print(f"\n{family} ({waves}-wave):")
    print("M N K " + " ".join(dtypes))
    gen = torch.Generator().manual_seed(1)
    for M, N, K in sizes:
        row = []
        for dtype in dtypes:
            a, _ = _inputs(family, dtype, M, N, K, dev, gen)
            row.append(f"{timed_tflops(matmul, a, M, N, K):.1f}")
        print(f"{M} {N} {K} " + " ".join(row), flush=True)
    return 0 if ok else 1
