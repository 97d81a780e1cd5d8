"""Flash-attention forward bench with the command line of the reference's
kernels/attention/bench.py (options at :102-152, the sequence-length sweep at
:99, correctness at :163-186, rotating sets at :189-203, rocprof mode at
:206-219)::

    python -m gfx950_gluon_tutorials_amd.attention.bench [--dtype bf16] [--layout bhsd] [--batch 1]
        [--hq 64] [--hk 64] [--d 128] [--seqlen 8192 | --sweep] [--variant 4]
        [--rocprof [--n-iters 1000] [--rotating-sets 0] [--rotating-buffer-size 512]]

It checks the kernel against an fp32 softmax(Q K^T * sm_scale) V of the same
inputs (the reference's seeded ``input_helper``) on sampled query rows of
every head, with the reference's acceptance rule (rtol 1e-3, atol max(1e-3,
2 ulp of the output type x max|o_ref|); kernels/attention/common.py:142-171),
then prints TFLOPS (median of event-timed launches) or, with ``--rocprof``,
issues ``--n-iters`` launches over rotating (q, k, v, o) sets for an external
``rocprofv3 --kernel-trace``.  ``--prepared`` and ``--n-warmup`` are accepted:
a launch here is already one C call with the arguments resolved, so both
paths are the same.  ``--variant`` picks fmha_v4 (lazy rescale, default) or
fmha_v3, the reference's two kernels.
"""

from __future__ import annotations

import argparse
import sys

import torch

from . import fmha_v3, fmha_v4
from .common import compute_flops, input_helper

SEQLENS = [1024, 2048, 4096, 8192, 16384]
_DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="gfx950 flash-attention forward benchmark")
    p.add_argument("--dtype", choices=["fp16", "bf16"], default="bf16")
    p.add_argument("--layout", choices=["bhsd", "bshd"], default="bhsd")
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--hq", type=int, default=64, help="number of query heads")
    p.add_argument("--hk", type=int, default=64, help="number of kv heads (hq %% hk == 0; hq == hk is MHA)")
    p.add_argument("--d", type=int, default=128, help="head dimension (128 or 64)")
    p.add_argument("--seqlen", type=int, default=8192, help="sequence length (default: 8192)")
    p.add_argument("--sweep", action="store_true", help="sweep all sequence lengths instead of one")
    p.add_argument("--variant", type=int, choices=[3, 4], default=4, help="fmha_v4 (default) or fmha_v3")
    p.add_argument("--rocprof", action="store_true",
                   help="run the kernel --n-iters times for rocprofv3 --kernel-trace")
    p.add_argument("--n-iters", type=int, default=1000)
    p.add_argument("--prepared", action="store_true", help="accepted; launches are already prepared C calls")
    p.add_argument("--n-warmup", type=int, default=10, help="unmeasured launches before the --rocprof loop")
    p.add_argument("--rotating-sets", type=int, default=0,
                   help="(q, k, v, o) sets cycled in --rocprof mode; 0 derives it from --rotating-buffer-size")
    p.add_argument("--scale-on-q", type=int, default=1, choices=[0, 1],
                   help="1 (default) folds sm_scale into Q before the loop; 0 scales each score")
    p.add_argument("--rotating-buffer-size", type=int, default=512,
                   help="--rocprof mode: MiB the rotating sets should span (default 512)")
    p.add_argument("--check-rows", type=int, default=64, help="query rows checked per head")
    return p.parse_args(argv)


def _run(args):
    return (fmha_v4 if args.variant == 4 else fmha_v3).run_gluon_attention


def make_inputs(args, n_ctx):
    q, k, v, md = input_helper(args.batch, args.hq, args.hk, n_ctx, n_ctx, args.d, _DTYPES[args.dtype],
                               args.layout)
    return q, k, v, torch.empty_like(q), md


def _bhsd(t, layout):
    return t if layout == "bhsd" else t.transpose(1, 2)


def check(args, n_ctx) -> bool:
    """Sampled rows of every head against the fp32 softmax attention of the
    same inputs, with the reference's acceptance rule."""
    q, k, v, o, md = make_inputs(args, n_ctx)
    _run(args)(q, k, v, o, md, bool(args.scale_on_q))
    rows = torch.linspace(0, n_ctx - 1, min(args.check_rows, n_ctx), device=q.device).round().long()
    qb, kb, vb, ob = (_bhsd(t, args.layout) for t in (q, k, v, o))
    group = args.hq // args.hk
    kb = kb.repeat_interleave(group, dim=1).float()
    vb = vb.repeat_interleave(group, dim=1).float()
    scores = torch.matmul(qb[:, :, rows].float(), kb.transpose(-1, -2).contiguous()) * md.sm_scale
    ref = torch.matmul(torch.softmax(scores, dim=-1), vb)
    got = ob[:, :, rows].float()
    eps = torch.finfo(_DTYPES[args.dtype]).eps
    atol = max(1e-3, 2 * eps * ref.abs().max().item())
    diff = (got - ref).abs()
    ok = bool((diff <= atol + 1e-3 * ref.abs()).all()) and not torch.isnan(got).any().item()
    tag = "match" if ok else "MISMATCH"
    print(f"[FMHA] B={args.batch} HQ={args.hq} HK={args.hk} N={n_ctx} D={args.d} non-causal {args.layout} "
          f"{q.dtype}: {tag}  (max={diff.max().item():.2e} mean={diff.mean().item():.2e}, {rows.numel()} rows "
          f"per head)", flush=True)
    return ok


def rotating_set_count(args, n_ctx) -> int:
    """(q, k, v, o) sets whose total exceeds --rotating-buffer-size (one set
    when a single one already does), as the reference derives it."""
    if args.rotating_sets > 0:
        return args.rotating_sets
    per_set = (2 * args.hq + 2 * args.hk) * args.batch * n_ctx * args.d * _DTYPES[args.dtype].itemsize
    return max(1, -(-args.rotating_buffer_size * 2**20 // max(1, per_set)))


def timed_tflops(args, n_ctx, reps: int = 20) -> float:
    q, k, v, o, md = make_inputs(args, n_ctx)
    run = _run(args)
    for _ in range(5):
        run(q, k, v, o, md, bool(args.scale_on_q))
    torch.cuda.synchronize()
    events = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run(q, k, v, o, md, bool(args.scale_on_q))
        e1.record()
        events.append((e0, e1))
    torch.cuda.synchronize()
    ms = sorted(e0.elapsed_time(e1) for e0, e1 in events)[reps // 2]
    return compute_flops(args.batch, args.hq, n_ctx, n_ctx, args.d, False) / (ms * 1e-3) / 1e12


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.hq % args.hk:
        raise ValueError(f"--hq {args.hq} must be a multiple of --hk {args.hk}")
    seqlens = SEQLENS if args.sweep else [args.seqlen]
    ok = all([check(args, n) for n in seqlens])
    run = _run(args)
    if args.rocprof:
        for n in seqlens:
            sets = [make_inputs(args, n) for _ in range(rotating_set_count(args, n))]
            for i in range(args.n_warmup):
                q, k, v, o, md = sets[i % len(sets)]
                run(q, k, v, o, md, bool(args.scale_on_q))
            torch.cuda.synchronize()
            for i in range(args.n_iters):
                q, k, v, o, md = sets[i % len(sets)]
                run(q, k, v, o, md, bool(args.scale_on_q))
            torch.cuda.synchronize()
            print(f"[FMHA] N={n}: {args.n_iters} iterations done ({len(sets)} rotating set(s))", flush=True)
            del sets
        return 0 if ok else 1
    print(f"\nfmha_v{args.variant} {args.dtype} {args.layout} B={args.batch} HQ={args.hq} HK={args.hk} D={args.d}:")
    print("N_CTX TFLOPS")
    for n in seqlens:
        print(f"{n} {timed_tflops(args, n):.1f}", flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
