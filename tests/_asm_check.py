"""Static check of the gfx950 kernels' hand-scheduled LDS reads.

The K loops issue their LDS fragment reads from inline asm, so the compiler
does not know that a read's destination registers are written when the data
returns, after the statement.  If the compiler copies such a register, or
gives it to another value, before the wave has waited for the read, the copy
holds stale data or the late return overwrites the new value.  This module
scans the device assembly for exactly that: an instruction that reads or
writes a register of an asm ds_read still in flight, by the wave's
lgkmcnt rules (an s_waitcnt lgkmcnt(N) retires all but the last N LDS and
scalar-memory operations issued; a wave never has more than 15 outstanding,
so the 16th issued retires the oldest).  Reads retire in issue order.

The asm MFMAs are invisible to the compiler's hazard recognizer in the
same way: their results arrive passes after the statement.  The scan also
flags any instruction other than an MFMA that touches an asm MFMA's
destination within MFMA_WAIT_STATES of it (each instruction counts one
wait state, s_nop N counts N + 1; 18 covers a 16-pass MFMA's result
latency for a VALU or memory reader).

The scan follows the text order of each function."""

from __future__ import annotations

import re

_VRANGE = re.compile(r"v\[(\d+):(\d+)\]")
_VREG = re.compile(r"v(\d+)$")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


def _regs(spec: str) -> set[int]:
    m = _VRANGE.match(spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = _VREG.match(spec)
    return {int(m.group(1))} if m else set()


def _operands(line: str) -> tuple[str, list[str]]:
    parts = line.split(None, 1)
    if len(parts) < 2:
        return (parts[0] if parts else ""), []
    return parts[0], [o.strip().split()[0] for o in parts[1].split(",") if o.strip()]


def _dst(op: str, ops: list[str], line: str) -> set[int]:
    if not ops or op.startswith(("s_", "ds_write", "buffer_store", "global_store", "scratch_store", "v_cmp")):
        return set()
    if op.startswith("buffer_load") and " lds" in line:
        return set()  # LDS-DMA: no register destination
    return _regs(ops[0])


def _srcs(op: str, ops: list[str]) -> set[int]:
    if op.startswith(("s_", "ds_")) or not ops:
        return set()
    if op.startswith(("buffer_store", "global_store", "scratch_store")):
        cand = ops
    else:
        cand = ops[1:]
    out: set[int] = set()
    for o in cand:
        out |= _regs(o)
    return out


MFMA_WAIT_STATES = 18
_AREG = re.compile(r"a\[(\d+):(\d+)\]")
_NOP = re.compile(r"s_nop\s+(\d+)")


def _mfma_regs(spec: str) -> set[int]:
    """VGPRs (as v) or AGPRs (as 1000 + a) of an MFMA destination."""
    m = _AREG.match(spec)
    if m:
        return set(range(1000 + int(m.group(1)), 1001 + int(m.group(2))))
    return _regs(spec)


def _touched(op: str, ops: list[str], line: str) -> set[int]:
    out = _srcs(op, ops) | _dst(op, ops, line)
    for o in ops:
        out |= {r for r in _mfma_regs(o) if r >= 1000}
    return out


def inflight_lds_hazards(asm: str) -> list[str]:
    """Lines that touch a register of an asm ds_read still in flight, or of
    an asm MFMA's result within MFMA_WAIT_STATES of it."""
    found = []
    fn = "?"
    queue: list[tuple[bool, set[int], int]] = []  # (asm read, registers, line)
    mfma: list[tuple[set[int], int, int]] = []    # (destination, wait states since, line)
    in_asm = False
    for no, raw in enumerate(asm.splitlines(), 1):
        s = raw.strip()
        if re.match(r"^_Z\S+:", s):
            fn, queue, mfma = s.split(":")[0], [], []
            continue
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith((";", ".")):
            continue
        nop = _NOP.match(s)
        ws = int(nop.group(1)) + 1 if nop else 1
        op0, ops0 = _operands(s)
        if op0.startswith("v_mfma"):
            # an MFMA may take another MFMA's result as its accumulator
            if in_asm:
                mfma.append((_mfma_regs(ops0[0]), 0, no))
            mfma = [(r, w + ws, l) for r, w, l in mfma]
            mfma = [x for x in mfma if x[1] < MFMA_WAIT_STATES + 1]
        else:
            pending = [x for x in mfma if x[1] < MFMA_WAIT_STATES]
            if pending and not s.startswith("s_"):
                t = _touched(op0, ops0, s)
                for r, w, l in pending:
                    if r & t:
                        found.append(f"{fn}: line {no} '{s}' touches the asm MFMA result of line {l} "
                                     f"after {w} wait states")
                        break
            mfma = [(r, w + ws, l) for r, w, l in mfma if w + ws < MFMA_WAIT_STATES]
        m = _LGKM.search(s)
        if s.startswith("s_waitcnt") and m:
            n = int(m.group(1))
            queue = queue[len(queue) - n:] if 0 < n < len(queue) else ([] if n == 0 else queue)
            continue
        op, ops = _operands(s)
        live: set[int] = set()
        for is_asm, regs, _ in queue:
            if is_asm:
                live |= regs
        if live and not op.startswith("ds_"):
            touched = (_srcs(op, ops) | _dst(op, ops, s)) & live
            if touched:
                src = min(q[2] for q in queue if q[0] and q[1] & touched)
                found.append(f"{fn}: line {no} '{s}' touches v{sorted(touched)} of the asm ds_read at line {src}")
        if op.startswith(("ds_", "s_load", "s_buffer_load")):
            queue.append((in_asm and op.startswith("ds_read"), _dst(op, ops, s) if op.startswith("ds_read") else set(),
                          no))
            queue = queue[-15:]
    return found
