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
so the 16th issued retires the oldest).  Reads retire in issue order.  The
scan follows the text order of each function."""

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


def inflight_lds_hazards(asm: str) -> list[str]:
    """Lines that touch a register of an asm ds_read still in flight."""
    found = []
    fn = "?"
    queue: list[tuple[bool, set[int], int]] = []  # (asm read, registers, line)
    in_asm = False
    for no, raw in enumerate(asm.splitlines(), 1):
        s = raw.strip()
        if re.match(r"^_Z\S+:", s):
            fn, queue = s.split(":")[0], []
            continue
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith((";", ".")):
            continue
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
