"""CPU oracle for the gfx950 GEMM path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker (or the timed CPU baseline).
The product (``gfx950_gluon_tutorials_amd``) never imports it.

It restates, in numpy, the reference's correctness path for this GEMM:

* a16w16: ``torch.matmul(a, b)`` with fp32 accumulation
  (kernels/gemm/intra_wave/a16w16/bench.py:167-187);
* a8w8: ``torch.matmul(a.to(fp16), b.to(fp16))`` on the e5m2 operands
  (kernels/gemm/intra_wave/a8w8/bench.py:129-142), extended by the per-tensor
  fp32 scales and bf16 output of the BF8 configuration;
* a4w4: ``torch_reference`` = fp32 mm of the dequantized MXFP4 operands, cast
  to bf16 (kernels/gemm/intra_wave/a4w4/bench.py:77-164);
* the data-parallel tile map ``get_pids`` (kernels/gemm/utils/common.py:38-83);
* the per-tensor e5m2 and OCP-MX MXFP4 quantizers, the stream-K work
  partition and the grouped (MoE) GEMM, which have no counterpart in the reference (they are defined by
  the BASELINE configurations and the OCP Microscaling Formats v1.0 spec).

How each function is pinned (golden fixtures made with exact rational
arithmetic, closed forms, torch's own float8 cast, brute force) is listed in
tests/test_oracle.py.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Element formats
# ---------------------------------------------------------------------------

# e2m1 code -> value; codes 8..15 are the negatives (code 8 is -0.0).
# kernels/gemm/intra_wave/a4w4/bench.py:86-103.
E2M1_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)
SCALE_GROUP = 32  # K values per E8M0 scale (OCP MX block size)
E5M2_MAX = 57344.0


def unpack_fp4(packed: np.ndarray) -> np.ndarray:
    """(R, K/2) uint8 -> (R, K) uint8 codes; the low nibble is the even k.
    kernels/gemm/intra_wave/a4w4/bench.py:80-85."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty((packed.shape[0], packed.shape[1] * 2), dtype=np.uint8)
    out[:, 0::2] = packed & 0xF
    out[:, 1::2] = packed >> 4
    return out


def pack_fp4(codes: np.ndarray) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint8)
    return (codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)


def mxfp4_to_f32(packed: np.ndarray) -> np.ndarray:
    """kernels/gemm/intra_wave/a4w4/bench.py:80-104."""
    return E2M1_VALUES[unpack_fp4(packed)]


def e8m0_to_f32(codes: np.ndarray) -> np.ndarray:
    """2^(x-127), 255 = NaN.  kernels/gemm/intra_wave/a4w4/bench.py:107-112."""
    codes = np.asarray(codes, dtype=np.uint8)
    out = np.ldexp(1.0, codes.astype(np.int64) - 127)  # float64: 2^128 is finite here
    out[codes == 255] = np.nan
    out = out.astype(np.float32)
    return out


def e5m2_to_f32(codes: np.ndarray) -> np.ndarray:
    """OCP fp8 e5m2 -> fp32.  e5m2 is the high byte of an IEEE binary16, so the
    decode is exact through float16."""
    codes = np.asarray(codes, dtype=np.uint8)
    return (codes.astype(np.uint16) << 8).view(np.float16).astype(np.float32)


def f32_to_e5m2(x: np.ndarray) -> np.ndarray:
    """fp32 -> OCP e5m2 codes with one rounding to nearest even (no detour
    through fp16, which would round twice).  Magnitudes from the overflow
    midpoint 61440 up become +-inf and NaN maps to 0x7F (code 0xFF for a
    negative NaN), the behaviour of torch's ``.to(torch.float8_e5m2)``."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        return _f32_to_e5m2(x)


def _f32_to_e5m2(x: np.ndarray) -> np.ndarray:
    a = np.abs(x).astype(np.float64)
    _, ex = np.frexp(a)
    e = ex.astype(np.int64) - 1  # floor(log2 a) for a > 0
    normal = a >= 2.0**-14
    step = np.where(normal, np.ldexp(1.0, e - 2), 2.0**-16)
    q = a / step  # exact: a power-of-two division
    r = np.floor(q)
    f = q - r
    r = r + ((f > 0.5) | ((f == 0.5) & (np.mod(r, 2) == 1)))
    val = r * step
    _, ex2 = np.frexp(val)
    e2 = ex2.astype(np.int64) - 1
    is_norm = val >= 2.0**-14
    mant_n = np.rint(val / np.ldexp(1.0, e2) * 4 - 4).astype(np.int64)
    mant_s = np.rint(val / 2.0**-16).astype(np.int64)
    code = np.where(is_norm, ((e2 + 15) << 2) | mant_n, mant_s)
    code = np.where(a >= 61440.0, 0x7C, code)
    sign = ((x.view(np.uint32) >> 31) & 1).astype(np.int64) << 7
    code = np.where(np.isnan(x), 0x7F, code) | sign
    return code.astype(np.uint8)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bf16, returned as fp32 values."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    out[np.isnan(x)] = np.nan
    return out


def round_to(x: np.ndarray, out_dtype: str) -> np.ndarray:
    """fp32 result -> output dtype ("f16" or "bf16") values as fp32."""
    if out_dtype == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if out_dtype == "bf16":
        return round_to_bf16(x)
    raise ValueError(out_dtype)


# ---------------------------------------------------------------------------
# Quantizers (BASELINE input contracts)
# ---------------------------------------------------------------------------


def quant_e5m2_per_tensor(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """Per-tensor e5m2: scale = absmax / 57344 so that absmax lands on the
    largest finite e5m2 value; codes = RNE(x / scale)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.float32(np.max(np.abs(x)))
    scale = np.float32(amax / np.float32(E5M2_MAX)) if amax > 0 else np.float32(1.0)
    y = np.clip(x / scale, -E5M2_MAX, E5M2_MAX).astype(np.float32)
    return f32_to_e5m2(y), scale


def _e2m1_round(m: np.ndarray) -> np.ndarray:
    """Magnitude (already divided by the block scale) -> e2m1 magnitude code
    0..7, round to nearest with ties to the even code, saturating at 6."""
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    idx = np.searchsorted(mids, m, side="left")  # m <= mids[i] -> i
    on_mid = np.isin(m, mids)
    # At a midpoint between codes i and i+1 pick the even one.
    tie_idx = np.searchsorted(mids, m, side="left")
    idx = np.where(on_mid, np.where(tie_idx % 2 == 0, tie_idx, tie_idx + 1), idx)
    return np.minimum(idx, 7).astype(np.uint8)


def quant_mxfp4(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """OCP MX v1.0 MXFP4 along the last axis: for each group of 32 values,
    E = floor(log2(amax)) - 2 (2 = emax of e2m1), E8M0 code = E + 127
    (clamped to [0, 254]; an all-zero group gets code 0), elements
    RNE(x / 2^E) saturated to +-6, sign kept (so small negatives give -0).
    Returns (packed (R, K/2) uint8, scales (R, K/32) uint8)."""
    x = np.asarray(x, dtype=np.float32)
    R, K = x.shape
    g = x.reshape(R, K // SCALE_GROUP, SCALE_GROUP)
    amax = np.abs(g).max(axis=-1)
    _, ex = np.frexp(amax)  # amax = m * 2^ex, m in [0.5, 1)
    E = ex.astype(np.int64) - 1 - 2
    E = np.where(amax > 0, E, -127)
    E = np.clip(E, -127, 127)
    scales = (E + 127).astype(np.uint8)
    y = g.astype(np.float64) / np.ldexp(1.0, E)[..., None]
    mag = _e2m1_round(np.abs(y))
    codes = mag | np.where(y < 0, 8, 0).astype(np.uint8)
    return pack_fp4(codes.reshape(R, K)), scales


# ---------------------------------------------------------------------------
# GEMM references
# ---------------------------------------------------------------------------


def preshuffle_e8m0(scales: np.ndarray) -> np.ndarray:
    """Restates, with explicit loops over the index definition, the preshuffled
    MXFP4 scale layout of g9_gemm_a4w4_preshuffled (no counterpart in the
    reference, whose ROADMAP.md lists preshuffled scales as planned): out[c, r,
    8j + 2s + h] = scales[r, 32c + 8s + 4h + g] with g = j ^ ((r >> 2) & 3);
    groups past the end read 127."""
    R, G = scales.shape
    chunks = -(-G // 32)
    out = np.full((chunks, R, 32), 127, dtype=np.uint8)
    for r in range(R):
        for c in range(chunks):
            for j in range(4):
                g = j ^ ((r >> 2) & 3)
                for s in range(4):
                    for h in range(2):
                        grp = 32 * c + 8 * s + 4 * h + g
                        if grp < G:
                            out[c, r, 8 * j + 2 * s + h] = scales[r, grp]
    return out


def torch_matmul_f32(a: np.ndarray, b_nk: np.ndarray):
    """The reference's CPU correctness path as BASELINE names it: torch.matmul
    in fp32 of the (dequantized) operands, C = A . B_nk^T
    (kernels/gemm/intra_wave/a4w4/bench.py:149-164 torch_reference; the fp16
    and bf8 benches' torch.matmul, a16w16/bench.py:167-187, a8w8/bench.py:129-142,
    run here in fp32 on the CPU).  Returns a torch fp32 tensor."""
    import torch

    at = torch.as_tensor(np.ascontiguousarray(a, dtype=np.float32))
    bt = torch.as_tensor(np.ascontiguousarray(b_nk, dtype=np.float32))
    return torch.matmul(at, bt.T)


def gemm_f32(a: np.ndarray, b_nk: np.ndarray) -> np.ndarray:
    """C = A . B^T in fp32 (numpy/BLAS), A (M, K), B (N, K)."""
    return np.asarray(a, dtype=np.float32) @ np.asarray(b_nk, dtype=np.float32).T


def a16w16_ref(a: np.ndarray, b_nk: np.ndarray, out_dtype: str = "f16") -> np.ndarray:
    """kernels/gemm/intra_wave/a16w16/bench.py:183 (fp32 accumulate, output in
    the operand dtype)."""
    return round_to(gemm_f32(a, b_nk), out_dtype)


def a8w8_ref(a_codes: np.ndarray, b_codes: np.ndarray, a_scale=1.0, b_scale=1.0,
             out_dtype: str = "f16") -> np.ndarray:
    """fp32 mm of the dequantized e5m2 operands (kernels/gemm/intra_wave/a8w8/bench.py:138),
    times the per-tensor scales, in the output dtype."""
    a = e5m2_to_f32(a_codes) * np.float32(a_scale)
    b = e5m2_to_f32(b_codes) * np.float32(b_scale)
    return round_to(gemm_f32(a, b), out_dtype)


def a8w8_ref_f32(a_codes, b_codes, a_scale=1.0, b_scale=1.0) -> np.ndarray:
    a = e5m2_to_f32(a_codes) * np.float32(a_scale)
    b = e5m2_to_f32(b_codes) * np.float32(b_scale)
    return gemm_f32(a, b)


def mxfp4_dequant(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """kernels/gemm/intra_wave/a4w4/bench.py:149-160: values x repeat_interleave(32) scales."""
    v = mxfp4_to_f32(packed)
    s = np.repeat(e8m0_to_f32(scales), SCALE_GROUP, axis=1)
    return v * s


def a4w4_ref(a: np.ndarray, b: np.ndarray, a_scales: np.ndarray, b_scales: np.ndarray,
             out_dtype: str = "bf16") -> np.ndarray:
    """``torch_reference`` of kernels/gemm/intra_wave/a4w4/bench.py:149-164."""
    return round_to(gemm_f32(mxfp4_dequant(a, a_scales), mxfp4_dequant(b, b_scales)), out_dtype)


def a4w4_ref_f32(a, b, a_scales, b_scales) -> np.ndarray:
    return gemm_f32(mxfp4_dequant(a, a_scales), mxfp4_dequant(b, b_scales))


def moe_ref(dense, a_rows, b_experts, offsets, *row_args, expert_args=()):
    """Grouped GEMM (no counterpart in the reference): expert e applies
    ``dense`` to rows [offsets[e], offsets[e+1]) of each row operand (a_rows and
    row_args, e.g. A's scales) and its own slice of each expert operand
    (b_experts and expert_args, e.g. B's scales).  Rows no expert owns are NaN."""
    offsets = np.asarray(offsets, dtype=np.int64)
    E = len(offsets) - 1
    out = None
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi <= lo:
            continue
        r = dense(a_rows[lo:hi], b_experts[e], *[x[lo:hi] for x in row_args], *[x[e] for x in expert_args])
        if out is None:
            out = np.full((a_rows.shape[0], r.shape[1]), np.nan, dtype=r.dtype)
        out[lo:hi] = r
    if out is None:
        out = np.full((a_rows.shape[0], b_experts.shape[1]), np.nan, dtype=np.float32)
    return out


def rel_frobenius(x: np.ndarray, ref: np.ndarray) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-300))


# ---------------------------------------------------------------------------
# Tile schedules
# ---------------------------------------------------------------------------


def get_pids(pid: int, M: int, N: int, BM: int, BN: int, GRID_MN: int, NUM_XCDS: int, GROUP_SIZE_M: int):
    """kernels/gemm/utils/common.py:38-83, restated by construction: build each
    XCD's contiguous block of new ids, then walk GROUP_SIZE_M-row groups."""
    tiles_m = -(-M // BM)
    tiles_n = -(-N // BN)
    # Round-robin dispatch: XCD x receives pids x, x+NUM_XCDS, ...; it owns
    # the next len(own) ids of the contiguous renumbering.
    new_id = {}
    nxt = 0
    for x in range(NUM_XCDS):
        own = list(range(x, GRID_MN, NUM_XCDS))
        for local, p in enumerate(own):
            new_id[p] = nxt + local
        nxt += len(own)
    q = new_id[pid]
    # Groups of GROUP_SIZE_M tile rows, column-major inside a group.
    per_group = GROUP_SIZE_M * tiles_n
    g = q // per_group
    rows = min(tiles_m - g * GROUP_SIZE_M, GROUP_SIZE_M)
    r = q - g * per_group
    return g * GROUP_SIZE_M + r % rows, r // rows


def streamk_segments(tiles: int, stages: int, ctas: int):
    """Stream-K partition: the tile-major (tile, stage) space split into `ctas`
    contiguous ranges (the first total % ctas ranges one unit longer).  Returns,
    per CTA, its segments (tile, first stage, end stage) in processing order
    (last tile first)."""
    total = tiles * stages
    base, rem = divmod(total, ctas)
    out = []
    for c in range(ctas):
        u0 = c * base + min(c, rem)
        u1 = u0 + base + (1 if c < rem else 0)
        segs = []
        while u1 > u0:
            t = (u1 - 1) // stages
            t0 = t * stages
            sb = max(u0, t0) - t0
            segs.append((t, sb, u1 - t0))
            u1 = t0 + sb
        out.append(segs)
    return out


def simulate_streamk(tiles: int, stages: int, ctas: int):
    """Runs the K-ordered chain protocol with every CTA resident and advancing
    one stage per step; a segment with sb > 0 may start only once the tile's
    flag equals sb.  Returns (makespan in stage-steps, per-tile final flag).
    Raises if the protocol deadlocks or a stage is covered twice."""
    segs = streamk_segments(tiles, stages, ctas)
    flag = [0] * tiles
    done = [[False] * stages for _ in range(tiles)]
    pos = [0] * ctas  # segment index per CTA
    prog = [0] * ctas  # stages done inside the current segment
    step = 0
    while any(pos[c] < len(segs[c]) for c in range(ctas)):
        moved = False
        advance = []
        for c in range(ctas):
            if pos[c] >= len(segs[c]):
                continue
            t, sb, se = segs[c][pos[c]]
            if prog[c] == 0 and sb > 0 and flag[t] != sb:
                continue  # waiting for the predecessor's partial
            advance.append(c)
        for c in advance:
            t, sb, se = segs[c][pos[c]]
            s = sb + prog[c]
            if done[t][s]:
                raise AssertionError(f"stage {s} of tile {t} covered twice")
            done[t][s] = True
            prog[c] += 1
            moved = True
            if sb + prog[c] == se:
                flag[t] = se
                pos[c] += 1
                prog[c] = 0
        step += 1
        if not moved:
            raise AssertionError("stream-K chain deadlocked")
    if not all(all(r) for r in done):
        raise AssertionError("some (tile, stage) never computed")
    return step, flag


def streamk_cta_of_block(block: int, ctas: int, num_xcds: int = 8) -> int:
    """The stream-K range a workgroup takes: gemm_sk renumbers blockIdx with
    the XCD remap of get_pids (one contiguous run of ranges per XCD, group size
    1), so block b, dispatched to XCD b % num_xcds, owns range new_id[b]."""
    if num_xcds == 1:
        return block
    pid_m, _ = get_pids(block, ctas, 1, 1, 1, ctas, num_xcds, 1)
    return pid_m


def simulate_streamk_dispatch(tiles: int, stages: int, ctas: int, resident, num_xcds: int = 8,
                              cta_of_block=None):
    """The stream-K chain protocol under partial residency (other kernels
    holding CUs): workgroup b goes to XCD b % num_xcds, each XCD starts its
    workgroups in increasing b as slots free up, at most resident[x] of them
    at once (resident[x] >= 1), and a workgroup holds its slot while it waits
    for a predecessor's flag.  Each step, every resident workgroup whose
    current segment may run advances one stage; a finished workgroup frees its
    slot.  Returns the makespan in stage-steps; raises AssertionError if the
    workgroups deadlock or a stage is covered twice or never.

    cta_of_block maps a workgroup to its range (default: gemm_sk's XCD remap)."""
    if cta_of_block is None:
        cta_of_block = lambda b: streamk_cta_of_block(b, ctas, num_xcds)  # noqa: E731
    segs = streamk_segments(tiles, stages, ctas)
    queues = [[b for b in range(x, ctas, num_xcds)] for x in range(num_xcds)]
    running: list[list[int]] = [[] for _ in range(num_xcds)]
    flag = [0] * tiles
    done = [[False] * stages for _ in range(tiles)]
    pos = {}
    prog = {}
    step = 0
    finished = 0
    while finished < ctas:
        for x in range(num_xcds):  # dispatch in block order into free slots
            while queues[x] and len(running[x]) < resident[x]:
                b = queues[x].pop(0)
                c = cta_of_block(b)
                running[x].append(c)
                pos[c], prog[c] = 0, 0
        moved = False
        advance = []
        for x in range(num_xcds):
            for c in running[x]:
                if pos[c] >= len(segs[c]):
                    continue
                t, sb, se = segs[c][pos[c]]
                if prog[c] == 0 and sb > 0 and flag[t] != sb:
                    continue
                advance.append(c)
        for c in advance:
            t, sb, se = segs[c][pos[c]]
            s = sb + prog[c]
            if done[t][s]:
                raise AssertionError(f"stage {s} of tile {t} covered twice")
            done[t][s] = True
            prog[c] += 1
            moved = True
            if sb + prog[c] == se:
                flag[t] = se
                pos[c] += 1
                prog[c] = 0
        for x in range(num_xcds):
            left = [c for c in running[x] if pos[c] < len(segs[c])]
            finished += len(running[x]) - len(left)
            moved = moved or len(left) != len(running[x])
            running[x] = left
        step += 1
        if not moved:
            raise AssertionError("stream-K workgroups deadlocked")
    if not all(all(r) for r in done):
        raise AssertionError("some (tile, stage) never computed")
    return step
