"""CPU model of the 4-wave main loop's LDS schedule (csrc/g9_gemm.hpp).

Restates, per region, what the kernel issues -- the operand sub-buffer it
reads (stage()'s table), the sub-buffer it refills and with which stage, the
scale-chunk DMAs (Shape::sc_part), the chunk-scale reads and the row-major
chunk transposes (xform_step) -- together with the waits (Shape::vm_wait /
vm_wait_hb) and barriers of both barrier patterns, and the prologue of
mainloop().  It then replays the program order of one wave, which every wave
of the workgroup shares, and checks what a race needs to be impossible
whatever the waves' relative timing between barriers:

* every LDS read sees the stage (or chunk) it expects: the last DMA into its
  sub-buffer carried that stage;
* read after DMA: that DMA had completed (a vmcnt wait whose count leaves it
  out of the outstanding ones) before a barrier that precedes the read, so it
  completed for every wave;
* DMA after read: the last read of the sub-buffer's previous contents
  precedes a barrier (every region and prologue wait also waits for the
  wave's LDS reads) that precedes the refill;
* a chunk transpose reads its own wave's chunk DMA only after a wait that
  covers it, and its writes reach a barrier before any wave reads the chunk.

Plausible mistakes (refilling the sub-buffer read in the previous region under
half barriers, waiting for one region's DMAs too few) fail the checks.  The
8-wave ping-pong (region_pp) is replayed the same way, phase by phase, and
so is the 256x128 stream-K tile's three-slot schedule (mainloop_h).
"""

import pytest

D = 4           # operand DMAs per sub-buffer per wave (G::kDmaPerSub, 4 waves)
SP = 4          # scale-chunk parts per wave (G::kScParts, 4 waves)
CHUNK = 4       # stages per scale chunk (kScChunk)
A0, A1, B0, B1 = 0, 1, 2, 3


def body_regions(scaled):
    return 4 * (2 * CHUNK if scaled else 2)


def sc_part(pos, scaled):
    """Shape::sc_part: the scale-chunk part issued at body position pos."""
    if not scaled:
        return -1
    q = pos % 16
    if q == 14:
        return 0
    if q % 2 == 0 and q // 2 + 1 < SP:
        return q // 2 + 1
    return -1


def dmas(pos, scaled):
    return D + (1 if sc_part(pos, scaled) >= 0 else 0)


def vm_wait(pos, scaled, back=6):
    R = body_regions(scaled)
    return sum(dmas((pos - q) % R, scaled) for q in range(1, back + 1))


def stage_table(k, half, refill_prev=False):
    """stage(): per region q of stage k, (read sub-buffer, read stage, refill
    sub-buffer, refill stage)."""
    if half and not refill_prev:
        return [(B1, k, A0, k + 2), (A1, k, B0, k + 2), (A0, k + 1, B1, k + 2), (B0, k + 1, A1, k + 2)]
    return [(B1, k, B0, k + 2), (A1, k, B1, k + 2), (A0, k + 1, A1, k + 2), (B0, k + 1, A0, k + 3)]


class Wave:
    """Program order of one wave: DMAs, reads, transposes and sync points."""

    def __init__(self):
        self.dmas = []      # (key, content)
        self.content = {}   # key -> (content, dma index)
        self.reads = {}     # key -> list of program points since its last DMA
        self.point = 0
        self.syncs = []     # (point, frontier, barrier)
        self.errors = []

    def tick(self):
        self.point += 1
        return self.point

    def dma(self, key, content, n=1):
        """n DMA instructions (vmcnt counts each) fill sub-buffer `key`."""
        p = self.tick()
        last_reads = self.reads.get(key, [])
        if last_reads:
            t = max(last_reads)
            if not any(b and t < y < p for y, _, b in self.syncs):
                self.errors.append(f"refill of {key} with {content} races the read at point {t}")
        self.dmas.extend([(key, content)] * n)
        self.content[key] = (content, len(self.dmas) - 1)
        self.reads[key] = []

    def sync(self, vm_count, barrier):
        p = self.tick()
        frontier = len(self.dmas) - vm_count if vm_count is not None else None
        if frontier is None:
            frontier = max((f for _, f, _ in self.syncs), default=0)
        else:
            frontier = max(frontier, max((f for _, f, _ in self.syncs), default=0))
        self.syncs.append((p, frontier, barrier))

    def _landed(self, idx, p, need_barrier):
        return any(f > idx and (b or not need_barrier) and y < p for y, f, b in self.syncs)

    def read(self, key, want, own=False):
        p = self.tick()
        got = self.content.get(key)
        if got is None or got[0] != want:
            self.errors.append(f"read of {key} at point {p} wants {want}, holds {got and got[0]}")
            return p
        if not self._landed(got[1], p, need_barrier=not own):
            self.errors.append(f"read of {key} ({want}) at point {p} before its DMA landed for every wave")
        self.reads.setdefault(key, []).append(p)
        return p


def run(nst, scaled, half, xform=False, refill_prev=False, hb_back=4, fb_back=6, write_shift=0):
    """Replays mainloop() for stages [0, nst); returns the violations."""
    w = Wave()
    R = body_regions(scaled)
    written = {}  # chunk -> program point of its last transpose write

    def chunk_dma(c, part):
        w.dma(("C", c % 2, part), c)

    first_read = {}  # chunk -> program point of its first read

    def chunk_read(c):
        for part in range(SP):
            p = w.read(("C", c % 2, part), c)
            first_read.setdefault(c, p)
            if xform and c in written and not any(b and written[c] < y < p for y, _, b in w.syncs):
                w.errors.append(f"chunk {c} read at point {p} before its transpose reached a barrier")

    def transpose_write(c):
        written[c] = w.tick()
        if c in first_read:
            w.errors.append(f"chunk {c} read at point {first_read[c]} before its transpose reached a barrier")

    # Prologue.
    if scaled:
        for part in range(SP):
            chunk_dma(0, part)
    for s in (0, 1):
        for x in (A0, B0, B1, A1):
            w.dma(("S", x, s % 2), s, D)
    if scaled:
        chunk_dma(1, 0)
    first = 6 * D + (1 if scaled else 0)
    w.sync(first, barrier=False)
    if xform:
        for part in range(SP):
            w.read(("C", 0, part), 0, own=True)
        transpose_write(0)
    w.sync(None, barrier=True)
    w.read(("S", A0, 0), 0)
    w.read(("S", B0, 0), 0)
    if scaled:
        chunk_read(0)
    w.sync(first, barrier=True)
    if not half:
        w.dma(("S", A0, 0), 2, D)
    # Loop (a partial body runs the same table).
    for r in range(4 * nst):
        k, q, pos = r // 4, r % 4, r % R
        bar = not half or pos % 2 == 0
        if not half:
            w.sync(vm_wait(pos, scaled, back=fb_back), True)
        elif bar:
            w.sync(vm_wait(pos, scaled, back=hb_back), True)
        else:
            w.sync(None, False)
        rx, rs, dx, ds = stage_table(k, half, refill_prev)[q]
        if rs < nst:
            w.read(("S", rx, rs % 2), rs)
            if scaled and rs % CHUNK == 0:
                chunk_read(rs // CHUNK)
        w.dma(("S", dx, ds % 2), ds, D)
        part = sc_part(pos, scaled)
        if part >= 0:
            h = 2 * (r // R) + pos // 16
            chunk_dma(h + (2 if part == 0 else 1), part)
        if xform:
            h = 2 * (r // R) + pos // 16
            p16 = pos % 16
            rj = {5: 0, 8: 1, 10: 2, 12: 3}.get(p16, -1)
            wj = {6 + write_shift: 0, 9 + write_shift: 1, 11 + write_shift: 2, 13 + write_shift: 3}.get(p16, -1)
            if 0 <= rj < SP and 4 * (h + 1) < nst:
                w.read(("C", (h + 1) % 2, rj), h + 1, own=True)
            if 0 <= wj < SP and 4 * (h + 1) < nst:
                transpose_write(h + 1)
    return w.errors


@pytest.mark.parametrize("nst", list(range(1, 19)) + [24, 33])
@pytest.mark.parametrize("half", [True, False])
def test_unscaled_schedules_are_race_free(nst, half):
    assert run(nst, scaled=False, half=half) == []


@pytest.mark.parametrize("nst", list(range(1, 19)) + [24, 33])
@pytest.mark.parametrize("half", [True, False])
@pytest.mark.parametrize("xform", [False, True])
def test_scaled_schedules_are_race_free(nst, half, xform):
    assert run(nst, scaled=True, half=half, xform=xform) == []


@pytest.mark.parametrize("scaled", [False, True])
def test_refilling_the_previous_region_under_half_barriers_races(scaled):
    # Planted in the model: with barriers in even regions only, refilling the
    # sub-buffer read in the previous region (the per-region pattern) lets a
    # fast wave overwrite it while a slow one still reads it.
    errors = run(12, scaled=scaled, half=True, refill_prev=True)
    assert any("races the read" in e for e in errors)


@pytest.mark.parametrize("scaled", [False, True])
def test_waiting_one_region_short_is_caught(scaled):
    # Planted: an even region that leaves the DMAs of 5 regions outstanding
    # instead of 4 publishes a sub-buffer before its last DMA landed.
    errors = run(12, scaled=scaled, half=True, hb_back=5)
    assert any("before its DMA landed" in e for e in errors)


def test_per_region_barriers_need_the_seven_region_lead():
    # Planted: with a barrier per region, leaving the DMAs of 7 regions
    # outstanding instead of 6 publishes a sub-buffer one region early.
    assert run(12, scaled=False, half=False) == []
    errors = run(12, scaled=False, half=False, fb_back=7)
    assert any("before its DMA landed" in e for e in errors)


@pytest.mark.parametrize("half", [True, False])
def test_a_late_transpose_write_is_caught(half):
    # Planted: each transpose write one region later puts the last one in the
    # region that first reads the chunk, after that region's barrier.
    errors = run(12, scaled=True, half=half, xform=True, write_shift=1)
    assert any("before its transpose reached a barrier" in e for e in errors)


# ---------------------------------------------------------------------------
# 8-wave ping-pong (region_pp): waves 0-3 (group 0) and 4-7 (group 1) run the
# same clusters one barrier apart, so between two barriers exactly one group
# runs a memory cluster (its LDS reads, its half of every DMA, then lgkmcnt(0)
# and vmcnt(vm_wait_pp)) while the other runs MFMAs.  Phase p >= 1 holds
# group 0's memory cluster of region (p - 1) / 2 (p odd) or group 1's of
# region (p - 2) / 2 (p even); phase 0 holds both groups' prologue refill.
# A sub-buffer's contents are complete only once both groups' DMAs of it have
# landed, each followed by a barrier; a refill by either group must come in a
# later phase than every read of the previous contents.
# ---------------------------------------------------------------------------
D8 = 2   # operand DMAs per sub-buffer per wave (8 waves)
SP8 = 2  # scale-chunk parts per wave (8 waves)


def sc_part8(pos, scaled):
    if not scaled:
        return -1
    q = pos % 16
    if q == 14:
        return 0
    if q % 2 == 0 and q // 2 + 1 < SP8:
        return q // 2 + 1
    return -1


def vm_wait_pp(pos, scaled, back=5):
    R = body_regions(scaled)
    return sum(D8 + (1 if sc_part8((pos - q) % R, scaled) >= 0 else 0) for q in range(0, back + 1))


def run_pingpong(nst, scaled, back=5):
    """Replays the 8-wave mainloop() for stages [0, nst); returns the violations."""
    R = body_regions(scaled)
    errors = []
    issued = [[], []]          # per group: list of DMA keys (one entry per instruction)
    frontier = [[], []]        # per group: (phase after which, DMAs complete)
    content = {}               # key -> (content, {group: last instruction index})
    reads = {}                 # key -> phases of reads of the current contents

    def dma(g, phase, key, c, n):
        if any(p >= phase for p in reads.get(key, [])):
            errors.append(f"group {g} refills {key} with {c} in phase {phase} before a read of it ended")
        issued[g].extend([key] * n)
        old = content.get(key)
        idx = dict(old[1]) if old and old[0] == c else {}
        idx[g] = len(issued[g]) - 1
        content[key] = (c, idx)
        if not old or old[0] != c:
            reads[key] = []

    def wait(g, phase, count):
        frontier[g].append((phase, len(issued[g]) - count))

    def read(g, phase, key, c):
        got = content.get(key)
        if got is None or got[0] != c or set(got[1]) != {0, 1}:
            errors.append(f"group {g} reads {key} in phase {phase} wanting {c}, holds {got and got[0]}")
            return
        for h, idx in got[1].items():
            if not any(f > idx and p < phase for p, f in frontier[h]):
                errors.append(f"group {g} reads {key} ({c}) in phase {phase} before group {h}'s DMA landed")
        reads[key].append(phase)

    def both_dma(phase, key, c, n):
        for g in (0, 1):
            dma(g, phase, key, c, n)

    # Prologue (both groups in lockstep, phases -3 .. 0).
    if scaled:
        for part in range(SP8):
            both_dma(-3, ("C", 0, part), 0, 1)
    for s in (0, 1):
        for x in (A0, B0, B1, A1):
            both_dma(-3, ("S", x, s % 2), s, D8)
    if scaled:
        both_dma(-3, ("C", 1, 0), 1, 1)
    first = 5 * D8 + (1 if scaled else 0)
    for g in (0, 1):
        wait(g, -3, first)                       # then a barrier
    for g in (0, 1):
        read(g, -2, ("S", A0, 0), 0)
        read(g, -2, ("S", B0, 0), 0)
        if scaled:
            for part in range(SP8):
                read(g, -2, ("C", 0, part), 0)
        wait(g, -2, first)                       # then a barrier
    both_dma(0, ("S", A0, 0), 2, D8)             # before group 1's extra barrier
    for r in range(4 * nst):
        k, q, pos = r // 4, r % 4, r % R
        rx, rs, dx, ds = stage_table(k, half=False)[q]
        for g in (0, 1):
            phase = 2 * r + 1 + g
            if rs < nst:
                read(g, phase, ("S", rx, rs % 2), rs)
                if scaled:
                    for part in range(SP8):
                        read(g, phase, ("C", (rs // CHUNK) % 2, part), rs // CHUNK)
            dma(g, phase, ("S", dx, ds % 2), ds, D8)
            part = sc_part8(pos, scaled)
            if part >= 0:
                h = 2 * (r // R) + pos // 16
                c = h + (2 if part == 0 else 1)
                dma(g, phase, ("C", c % 2, part), c, 1)
            wait(g, phase, vm_wait_pp(pos, scaled, back))
    return errors


@pytest.mark.parametrize("nst", list(range(1, 19)) + [24, 33])
@pytest.mark.parametrize("scaled", [False, True])
def test_pingpong_schedule_is_race_free(nst, scaled):
    assert run_pingpong(nst, scaled) == []


@pytest.mark.parametrize("scaled", [False, True])
def test_pingpong_waiting_one_region_short_is_caught(scaled):
    # Planted: a memory cluster leaving its DMAs of 7 regions outstanding
    # instead of 6 lets the leading group read a sub-buffer the lagging
    # group's DMAs have not filled yet.
    errors = run_pingpong(12, scaled, back=6)
    assert any("DMA landed" in e for e in errors)


# ---------------------------------------------------------------------------
# 256x128 stream-K tiles (mainloop_h): sub-buffers A0, A1, B0 in three slots
# (stage s in slot s % 3), two regions per stage with a barrier each.  Region
# 0 of stage s reads A1(s) and B0(s + 1) and refills B0 and the first half of
# A0's rows of slot s % 3 with stage s + 3; region 1 reads A0(s + 1) and
# B0(s + 1) and refills the other half of A0 and A1.  Each region waits for
# all but the DMAs of the three regions before it (kHnVmWait).
# ---------------------------------------------------------------------------
def run_hn(nst, back=3):
    w = Wave()
    for s in (0, 1, 2):
        w.dma(("B0", s), s, D)
        w.dma(("A0lo", s), s, 2)
        w.dma(("A0hi", s), s, 2)
        w.dma(("A1", s), s, D)
    w.sync(7 * D, barrier=True)
    for key in ("A0lo", "A0hi", "B0"):
        w.read((key, 0), 0)
    for r in range(2 * nst):
        s, half = r // 2, r % 2
        w.sync(back * 6, barrier=True)
        if half == 0:
            reads = [(("A1", s % 3), s), (("B0", (s + 1) % 3), s + 1)]
            refills = [("B0", D), ("A0lo", 2)]
        else:
            reads = [(("A0lo", (s + 1) % 3), s + 1), (("A0hi", (s + 1) % 3), s + 1), (("B0", (s + 1) % 3), s + 1)]
            refills = [("A0hi", 2), ("A1", D)]
        for key, want in reads:
            if want < nst:
                w.read(key, want)
        for x, n in refills:
            w.dma((x, s % 3), s + 3, n)
    return w.errors


@pytest.mark.parametrize("nst", list(range(1, 20)) + [25, 36])
def test_half_tile_streamk_schedule_is_race_free(nst):
    assert run_hn(nst) == []


def test_half_tile_waiting_one_region_short_is_caught():
    errors = run_hn(12, back=4)
    assert any("before its DMA landed" in e for e in errors)
