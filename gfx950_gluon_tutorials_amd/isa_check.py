"""Static check of the library's gfx950 assembly for MFMA data hazards.

The kernels issue their MFMAs as inline assembly (to keep each accumulator
tied to its AGPRs), and the compiler's hazard recognizer does not look inside
inline assembly.  It therefore inserts no wait states when its own code --
register copies, spills, epilogue conversions, stores -- touches an MFMA's
destination registers right after the MFMA, or when a VALU instruction writes
an MFMA source just before it.  The kernels add the wait states themselves
where their own code does this; this check proves that nothing else does, by
scanning the device assembly of the built library:

* MFMA write -> non-MFMA access of any of its destination registers: at least
  ``READ_AFTER_MFMA[kind]`` wait states in between (the counts the compiler
  itself uses for the same MFMAs written as builtins).  A following MFMA that
  accumulates into exactly the same registers needs none.
* VALU (including ``v_accvgpr_write``) write -> MFMA read of the register as
  any source: at least ``MFMA_AFTER_VALU`` wait states.

Each instruction counts one wait state, ``s_nop N`` counts N + 1.  The scan is
a fixed-point over the basic blocks (labels and branches), so hazards that
cross a branch or a loop back edge are seen.

A second scan covers LDS reads the compiler does not track (the transpose
reads of the MXFP4 scale chunks are inline assembly): a VGPR written by a
``ds_*`` read is pending until an ``s_waitcnt lgkmcnt(k)`` with at least k DS
instructions issued after that read (DS operations complete in order), and
no instruction may read or write it while it is pending.  Compiler-generated
LDS reads satisfy this by construction; the scan proves it for the inline
ones.

Usage: ``python -m gfx950_gluon_tutorials_amd.isa_check file.s`` (exit status 1
on violations), or ``check_text(asm) -> list of violations``.
"""

from __future__ import annotations

import re
import sys
from dataclasses import dataclass, field

# Wait states between an MFMA and the first non-MFMA access of its result, by
# MFMA shape and operand format.
READ_AFTER_MFMA = {
    "16x16x32_f16": 8,
    "16x16x32_bf16": 8,
    "16x16x128_f8f6f4": 12,
    "scale_16x16x128_f8f6f4": 8,
    "32x32x16_f16": 12,
    "32x32x16_bf16": 12,
    "32x32x64_f8f6f4": 20,
    "scale_32x32x64_f8f6f4": 12,
}
DEFAULT_READ_AFTER_MFMA = 20
MFMA_AFTER_VALU = 2

_REG = re.compile(r"\b([vas])(?:\[(\d+):(\d+)\]|(\d+)\b)")
_LABEL = re.compile(r"^([.\w]+):")
_BRANCH = re.compile(r"^\s*s_(cbranch_\w+|branch)\s+([.\w]+)")


def _regs(text: str, kinds="va") -> set[tuple[str, int]]:
    out = set()
    for m in _REG.finditer(text):
        k = m.group(1)
        if k not in kinds:
            continue
        if m.group(4) is not None:
            out.add((k, int(m.group(4))))
        else:
            out.update((k, r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def _mfma_kind(mnemonic: str) -> str:
    name = mnemonic[len("v_mfma_"):]
    if name.startswith("scale_f32_"):
        return "scale_" + name[len("scale_f32_"):]
    if name.startswith("f32_"):
        return name[len("f32_"):]
    return name


@dataclass
class Instr:
    line: int
    text: str
    mnemonic: str
    dst: set = field(default_factory=set)
    src: set = field(default_factory=set)
    waits: int = 1


def _parse_instr(lineno: int, raw: str) -> Instr | None:
    text = raw.split(";", 1)[0].strip()
    if not text or text.startswith(".") or text.endswith(":"):
        return None
    parts = text.split(None, 1)
    mn = parts[0]
    ops = parts[1] if len(parts) > 1 else ""
    ins = Instr(lineno, text, mn)
    if mn == "s_nop":
        ins.waits = int(ops.strip(), 0) + 1
        return ins
    if not (mn.startswith("v_") or mn.startswith(("global_", "buffer_", "scratch_", "flat_", "ds_"))):
        return ins
    operands = [o.strip() for o in ops.split(",")]
    is_store = mn.startswith(("global_store", "buffer_store", "scratch_store", "flat_store", "ds_write")) or (
        "atomic" in mn and "_rtn" not in mn
    )
    if is_store or mn.startswith("ds_write"):
        ins.src = _regs(ops)
    elif operands:
        ins.dst = _regs(operands[0])
        ins.src = _regs(",".join(operands[1:]))
    return ins


def _blocks(lines: list[str]):
    """Splits one function into basic blocks: (label, [Instr], successors)."""
    blocks = []
    cur_label, cur = "<entry>", []
    succ_of = {}

    def close(next_label, fallthrough=True):
        nonlocal cur_label, cur
        blocks.append([cur_label, cur, []])
        succ_of[len(blocks) - 1] = fallthrough
        cur_label, cur = next_label, []

    pending_targets = {}
    for i, raw in enumerate(lines):
        m = _LABEL.match(raw)
        if m and not raw.startswith("\t"):
            close(m.group(1))
            continue
        ins = _parse_instr(i, raw)
        if ins is None:
            continue
        cur.append(ins)
        b = _BRANCH.match(raw)
        if b:
            pending_targets.setdefault(len(blocks), []).append(b.group(2))
            close(f"<after {i}>", fallthrough=b.group(1) != "branch")
        elif ins.mnemonic in ("s_endpgm", "s_setpc_b64"):
            close(f"<after {i}>", fallthrough=False)
    close("<end>", fallthrough=False)
    index = {b[0]: k for k, b in enumerate(blocks)}
    for k, b in enumerate(blocks):
        if succ_of.get(k) and k + 1 < len(blocks):
            b[2].append(k + 1)
        for t in pending_targets.get(k, []):
            if t in index:
                b[2].append(index[t])
    return blocks


def _step(state: dict, ins: Instr, violations: list, func: str):
    """Advances the pending-hazard state over one instruction (one message per
    offending instruction).

    state maps a register to (remaining wait states, origin line, written by
    an MFMA)."""
    is_mfma = ins.mnemonic.startswith("v_mfma")
    msg = None
    if is_mfma:
        for r in sorted(ins.src | ins.dst):
            ent = state.get(r)
            if ent and not ent[2]:
                msg = f"{ins.mnemonic} reads {r[0]}{r[1]} {ent[0]} wait state(s) too soon after the VALU write at line {ent[1] + 1}"
                break
            # Accumulating into exactly the previous MFMA's destination is
            # fine; reading part of a pending MFMA result any other way is not.
            if ent and ent[2] and r not in ins.dst:
                msg = f"{ins.mnemonic} reads {r[0]}{r[1]} as a source {ent[0]} wait state(s) too soon after the MFMA at line {ent[1] + 1}"
                break
    else:
        for r in sorted(ins.dst | ins.src):
            ent = state.get(r)
            if ent and ent[2]:
                msg = f"'{ins.text}' touches {r[0]}{r[1]} {ent[0]} wait state(s) too soon after the MFMA at line {ent[1] + 1}"
                break
    if msg:
        violations.append(f"{func}: line {ins.line + 1}: {msg}")
    # Time passes.
    for r in list(state):
        rem = state[r][0] - ins.waits
        if rem <= 0:
            del state[r]
        else:
            state[r] = (rem,) + state[r][1:]
    # New hazards.
    if is_mfma:
        need = READ_AFTER_MFMA.get(_mfma_kind(ins.mnemonic), DEFAULT_READ_AFTER_MFMA)
        for r in ins.dst:
            state[r] = (need, ins.line, True)
    elif ins.mnemonic.startswith("v_") and ins.dst:
        for r in ins.dst:
            state[r] = (MFMA_AFTER_VALU, ins.line, False)


_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


def _lgkm_wait(ins: Instr) -> int | None:
    """The lgkmcnt limit of an s_waitcnt (None if it does not constrain it)."""
    if ins.mnemonic != "s_waitcnt":
        return None
    ops = ins.text.split(None, 1)[1] if " " in ins.text else ""
    m = _LGKM.search(ops)
    if m:
        return int(m.group(1))
    try:
        v = int(ops.strip(), 0)  # raw gfx9 encoding: lgkmcnt in bits 11:8
    except ValueError:
        return None
    k = (v >> 8) & 15
    return None if k == 15 else k


def _lds_step(state: dict, ins: Instr, violations: list, func: str):
    """Advances the pending-LDS-result state over one instruction.

    state maps a VGPR to (DS instructions issued since the read, read line)."""
    for r in sorted(ins.dst | ins.src):
        ent = state.get(r)
        if ent:
            violations.append(
                f"{func}: line {ins.line + 1}: '{ins.text}' touches {r[0]}{r[1]} before the LDS read at line "
                f"{ent[1] + 1} is waited for"
            )
            break
    k = _lgkm_wait(ins)
    if k is not None:
        for r in [r for r, ent in state.items() if ent[0] >= k]:
            del state[r]
    if ins.mnemonic.startswith("ds_"):
        for r in list(state):
            state[r] = (state[r][0] + 1, state[r][1])
        if not ins.mnemonic.startswith("ds_write"):
            for r in ins.dst:
                state[r] = (0, ins.line)


def _merge_lds(a: dict, b: dict) -> dict:
    out = dict(a)
    for r, ent in b.items():
        if r not in out or out[r][0] > ent[0]:
            out[r] = ent
    return out


def _merge(a: dict, b: dict) -> dict:
    out = dict(a)
    for r, ent in b.items():
        if r not in out or out[r][0] < ent[0]:
            out[r] = ent
    return out


def _fixpoint(name: str, blocks, step, merge) -> list[str]:
    entry_state = [None] * len(blocks)
    entry_state[0] = {}
    work = [0]
    seen_violations: dict[str, None] = {}
    rounds = 0
    while work and rounds < 100000:
        rounds += 1
        k = work.pop()
        state = dict(entry_state[k])
        v: list[str] = []
        for ins in blocks[k][1]:
            step(state, ins, v, name)
        for msg in v:
            seen_violations.setdefault(msg, None)
        for s in blocks[k][2]:
            new = state if entry_state[s] is None else merge(entry_state[s], state)
            if new != entry_state[s]:
                entry_state[s] = new
                work.append(s)
    return list(seen_violations)


def check_function(name: str, lines: list[str]) -> list[str]:
    blocks = _blocks(lines)
    return _fixpoint(name, blocks, _step, _merge) + _fixpoint(name, blocks, _lds_step, _merge_lds)


def check_text(asm: str) -> list[str]:
    """Checks every kernel function in an assembly listing."""
    violations = []
    lines = asm.split("\n")
    starts = [(i, m.group(1)) for i, l in enumerate(lines) if (m := re.match(r"^([A-Za-z_]\w*):", l))]
    for n, (i, name) in enumerate(starts):
        end = starts[n + 1][0] if n + 1 < len(starts) else len(lines)
        body = lines[i + 1:end]
        for j, l in enumerate(body):
            if l.strip().startswith("s_endpgm"):
                body = body[: j + 1]
                break
        violations += check_function(name, body)
    return violations


def resource_table(asm: str) -> list[dict]:
    """Per-kernel register, scratch and LDS use from the code-object metadata
    of an assembly listing (the figures the reference reads from its own
    builds: VGPR, AGPR and spill counts)."""
    rows = []
    for blk in asm.split("  - .agpr_count:")[1:]:
        def field(name, cast=int):
            m = re.search(rf"\.{name}:\s+(\S+)", blk)
            return cast(m.group(1)) if m else None

        name = field("name", str)
        if name is None or name.startswith("_Z"):
            continue
        rows.append({
            "kernel": name,
            "agpr": int(re.match(r"\s*(\d+)", blk).group(1)),
            "vgpr_total": field("vgpr_count"),
            "sgpr": field("sgpr_count"),
            "vgpr_spill": field("vgpr_spill_count"),
            "sgpr_spill": field("sgpr_spill_count"),
            "scratch_bytes": field("private_segment_fixed_size"),
            "lds_bytes": field("group_segment_fixed_size"),
        })
    return sorted(rows, key=lambda r: r["kernel"])


def main(argv: list[str]) -> int:
    bad = []
    for path in argv:
        with open(path) as f:
            bad += check_text(f.read())
    for msg in bad:
        print(msg)
    print(f"{len(bad)} hazard(s)")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
