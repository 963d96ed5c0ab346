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
so the 16th issued retires the oldest).  LDS operations retire in issue
order, but scalar-memory (and flat) loads may return out of order: while one
is pending, only lgkmcnt(0) proves that an older LDS read has landed, and the
15-outstanding rule proves nothing.  An LDS instruction's own VGPR operands
(address, write data, destination) are checked like any other's.

The asm MFMAs are invisible to the compiler's hazard recognizer in the
same way: their results arrive passes after the statement.  The scan also
flags any instruction other than an MFMA that touches an asm MFMA's
destination within MFMA_WAIT_STATES of it (each instruction counts one
wait state, s_nop N counts N + 1; 18 covers a 16-pass MFMA's result
latency for a VALU or memory reader).

Each function is split into basic blocks (labels start one; branches and
s_endpgm end one) and the in-flight state is propagated along the control
flow to a fixed point: a read or MFMA result counts as pending at a block's
entry if it is pending at the end of any predecessor, with the fewest
retiring operations or wait states of those paths.  So a loop that the
compiler lays out rotated (its latch blocks placed before its header) is
judged by its real paths, and every path is covered."""

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
    if op.startswith("s_") or not ops:
        return set()
    if op.startswith(("buffer_store", "global_store", "scratch_store", "ds_write", "ds_store")):
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


_LABEL = re.compile(r"^(\.LBB\w+):")
_BRANCH = re.compile(r"^s_(c?branch\w*)\s+(\.LBB\w+)")
LGKM_MAX = 15  # outstanding LDS/SMEM operations a wave can have
# lgkmcnt operations that may return out of order with LDS ones
_SMEM = ("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "flat_")


def _blocks(lines: list[tuple[int, str, bool]]):
    """Basic blocks of one function: (label or None, [(line no, text, in asm)], successor labels, falls through)."""
    blocks, cur, label = [], [], None

    def close(succ, falls):
        nonlocal cur, label
        blocks.append((label, cur, succ, falls))
        cur, label = [], None

    for no, s, in_asm in lines:
        m = _LABEL.match(s)
        if m:
            if cur or label is not None:
                close([], True)
            label = m.group(1)
            continue
        cur.append((no, s, in_asm))
        b = _BRANCH.match(s)
        if b:
            close([b.group(2)], b.group(1) != "branch")
        elif s.startswith(("s_endpgm", "s_setpc", "s_trap")):
            close([], False)
    if cur or label is not None:
        close([], False)
    return blocks


def _step(state, no, s, in_asm, fn, found):
    """Advances (reads, mfmas) over one instruction, recording hazards in found (if not None)."""
    # reads: {line: (asm ds_read, regs, ops issued after, out-of-order kind)}; mfma: {line: (regs, wait states)}
    reads, mfma = state
    nop = _NOP.match(s)
    ws = int(nop.group(1)) + 1 if nop else 1
    op0, ops0 = _operands(s)
    if op0.startswith("v_mfma"):
        mfma = {l: (r, w + ws) for l, (r, w) in mfma.items() if w + ws < MFMA_WAIT_STATES + 1}
        if in_asm:
            mfma[no] = (_mfma_regs(ops0[0]), 0)
    else:
        if not s.startswith("s_") and found is not None:
            t = _touched(op0, ops0, s)
            for l, (r, w) in sorted(mfma.items()):
                if w < MFMA_WAIT_STATES and r & t:
                    found.append(f"{fn}: line {no} '{s}' touches the asm MFMA result of line {l} "
                                 f"after {w} wait states")
                    break
        mfma = {l: (r, w + ws) for l, (r, w) in mfma.items() if w + ws < MFMA_WAIT_STATES}
    m = _LGKM.search(s)
    if s.startswith("s_waitcnt") and m:
        n = int(m.group(1))
        if n == 0:
            return {}, mfma
        if any(x[3] for x in reads.values()):  # an out-of-order return may be what the count saw
            return reads, mfma
        return {l: x for l, x in reads.items() if x[2] < n}, mfma
    op, ops = _operands(s)
    if found is not None:
        live = {}
        for l, (is_asm, regs, _, _) in reads.items():
            if is_asm and l != no:  # (a loop's earlier instance of this same read is not a conflict)
                for r in regs:
                    live.setdefault(r, l)
        if live:
            touched = (_srcs(op, ops) | _dst(op, ops, s)) & set(live)
            if touched:
                found.append(f"{fn}: line {no} '{s}' touches v{sorted(touched)} of the asm ds_read at line "
                             f"{min(live[r] for r in touched)}")
    if op.startswith(("ds_",) + _SMEM):
        unordered = any(x[3] for x in reads.values())
        reads = {l: (a, r, c + 1, u) for l, (a, r, c, u) in reads.items() if unordered or c + 1 < LGKM_MAX}
        reads[no] = (in_asm and op.startswith("ds_read"), _dst(op, ops, s) if op.startswith("ds_read") else set(), 0,
                     op.startswith(_SMEM))
    return reads, mfma


def _merge(a, b):
    if a is None:
        return b
    reads = dict(a[0])
    for l, (x, r, c, u) in b[0].items():
        reads[l] = (x, r, min(c, reads[l][2]), u) if l in reads else (x, r, c, u)
    mfma = dict(a[1])
    for l, (r, w) in b[1].items():
        mfma[l] = (r, min(w, mfma[l][1])) if l in mfma else (r, w)
    return reads, mfma


def _function_hazards(fn: str, lines: list[tuple[int, str, bool]]) -> list[str]:
    blocks = _blocks(lines)
    index = {lab: i for i, (lab, _, _, _) in enumerate(blocks) if lab is not None}
    succ = []
    for i, (_, _, targets, falls) in enumerate(blocks):
        out = [index[t] for t in targets if t in index]
        if falls and i + 1 < len(blocks):
            out.append(i + 1)
        succ.append(out)
    entry = [None] * len(blocks)
    entry[0] = ({}, {})
    work = [0]
    while work:
        i = work.pop()
        st = entry[i]
        for no, s, in_asm in blocks[i][1]:
            st = _step(st, no, s, in_asm, fn, None)
        for j in succ[i]:
            merged = _merge(entry[j], st)
            if merged != entry[j]:
                entry[j] = merged
                work.append(j)
    found: list[str] = []
    for i, blk in enumerate(blocks):
        if entry[i] is None:
            continue
        st = entry[i]
        for no, s, in_asm in blk[1]:
            st = _step(st, no, s, in_asm, fn, found)
    return found


def inflight_lds_hazards(asm: str) -> list[str]:
    """Lines that touch a register of an asm ds_read still in flight, or of
    an asm MFMA's result within MFMA_WAIT_STATES of it, on some path."""
    found: list[str] = []
    fn, lines, in_asm = None, [], False
    for no, raw in enumerate(asm.splitlines(), 1):
        s = raw.strip()
        if re.match(r"^_Z\S+:", s):
            if fn is not None:
                found += _function_hazards(fn, lines)
            fn, lines, in_asm = s.split(":")[0], [], False
            continue
        if fn is None:
            continue
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith(";") or (s.startswith(".") and not _LABEL.match(s)):
            continue
        lines.append((no, s, in_asm))
    if fn is not None:
        found += _function_hazards(fn, lines)
    return found


# ---------------------------------------------------------------------------
# SGPR operands of asm vector-memory instructions.  A VALU instruction that
# writes an SGPR (v_readlane_b32 / v_readfirstlane_b32 reloading a spilled
# scalar, a v_cmp mask) needs VALU_SGPR_VMEM_WAIT_STATES before a VMEM
# instruction reads that SGPR as its resource, offset or (LDS-DMA) M0.  The
# compiler inserts them for its own VMEM instructions but cannot see the
# operands of inline asm, so an asm load must carry them itself.

VALU_SGPR_VMEM_WAIT_STATES = 5
_SRANGE = re.compile(r"s\[(\d+):(\d+)\]$")
_SREG = re.compile(r"s(\d+)$")
_VCC = {106, 107}
_M0 = 124


def _sgprs(spec: str) -> set[int]:
    m = _SRANGE.match(spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = _SREG.match(spec)
    if m:
        return {int(m.group(1))}
    if spec in ("vcc", "vcc_lo", "vcc_hi"):
        return set(_VCC)
    if spec == "m0":
        return {_M0}
    return set()


def _valu_sgpr_writes(op: str, ops: list[str]) -> set[int]:
    if not op.startswith("v_") or not ops:
        return set()
    out = _sgprs(ops[0])
    if "_co_" in op and len(ops) > 1:
        out |= _sgprs(ops[1])
    if op.endswith("_e32") and (op.startswith("v_cmp") or "_co_" in op):
        out |= _VCC
    return out


def _vmem_sgpr_reads(op: str, ops: list[str], line: str) -> set[int]:
    if not op.startswith(("buffer_", "global_", "scratch_")):
        return set()
    out: set[int] = set()
    for o in ops:
        out |= _sgprs(o)
    if " lds" in line:
        out.add(_M0)
    return out


def _sgpr_function_hazards(fn: str, lines: list[tuple[int, str, bool]]) -> list[str]:
    blocks = _blocks(lines)
    index = {lab: i for i, (lab, _, _, _) in enumerate(blocks) if lab is not None}
    succ = []
    for i, (_, _, targets, falls) in enumerate(blocks):
        out = [index[t] for t in targets if t in index]
        if falls and i + 1 < len(blocks):
            out.append(i + 1)
        succ.append(out)

    def step(state, no, s, in_asm, found):
        op, ops = _operands(s)
        if found is not None and in_asm:
            for r in sorted(_vmem_sgpr_reads(op, ops, s)):
                if r in state and state[r][1] < VALU_SGPR_VMEM_WAIT_STATES:
                    found.append(f"{fn}: line {no} '{s}' reads s{r} {state[r][1]} wait states after the VALU "
                                 f"write at line {state[r][0]}")
                    break
        nop = _NOP.match(s)
        ws = int(nop.group(1)) + 1 if nop else 1
        state = {r: (l, w + ws) for r, (l, w) in state.items() if w + ws < VALU_SGPR_VMEM_WAIT_STATES}
        for r in _valu_sgpr_writes(op, ops):
            state[r] = (no, 0)
        return state

    entry: list[dict | None] = [None] * len(blocks)
    entry[0] = {}
    work = [0]
    while work:
        i = work.pop()
        st = entry[i]
        for no, s, in_asm in blocks[i][1]:
            st = step(st, no, s, in_asm, None)
        for j in succ[i]:
            merged = dict(entry[j] or {})
            for r, (l, w) in st.items():
                if r not in merged or w < merged[r][1]:
                    merged[r] = (l, w)
            if entry[j] is None or merged != entry[j]:
                entry[j] = merged
                work.append(j)
    found: list[str] = []
    for i, blk in enumerate(blocks):
        if entry[i] is None:
            continue
        st = entry[i]
        for no, s, in_asm in blk[1]:
            st = step(st, no, s, in_asm, found)
    return found


def sgpr_vmem_hazards(asm: str) -> list[str]:
    """Asm vector-memory instructions that read an SGPR (or M0) fewer than
    VALU_SGPR_VMEM_WAIT_STATES after a VALU instruction wrote it, on some
    path."""
    found: list[str] = []
    fn, lines, in_asm = None, [], False
    for no, raw in enumerate(asm.splitlines(), 1):
        s = raw.strip()
        if re.match(r"^_Z\S+:", s):
            if fn is not None:
                found += _sgpr_function_hazards(fn, lines)
            fn, lines, in_asm = s.split(":")[0], [], False
            continue
        if fn is None:
            continue
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith(";") or (s.startswith(".") and not _LABEL.match(s)):
            continue
        lines.append((no, s, in_asm))
    if fn is not None:
        found += _sgpr_function_hazards(fn, lines)
    return found
