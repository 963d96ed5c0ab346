"""numpy restatement of the reference's torch semantics (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module.  bf16 tensors are represented as uint16 bit patterns.  Paths in
citations are relative to the reference repository root.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

LAYOUTS = ("nn", "nt", "tn", "tt")

# ---------------------------------------------------------------------------
# bf16


def bf16_round(x) -> np.ndarray:
    """fp32 -> bf16 bits, round-to-nearest-even; NaN -> 0x7FC0.

    This is the conversion behind torch's ``.to(torch.bfloat16)`` used at the
    end of reference_mm (api.py:292-293).
    """
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_from_f32(x) -> np.ndarray:
    """Rounds float values to bf16 and returns the bits (for building scales)."""
    return bf16_round(x)


def bf16_ulp_diff(a_bits, b_bits) -> np.ndarray:
    """Distance in bf16 units in the last place between two bit arrays.

    Maps the sign-magnitude bit patterns onto a monotone integer line so that
    +0 and -0 coincide and adjacent representable values differ by 1.
    """

    def line(bits):
        v = np.asarray(bits, dtype=np.uint16).astype(np.int64)
        mag = v & 0x7FFF
        return np.where(v & 0x8000, -mag, mag)

    return np.abs(line(a_bits) - line(b_bits))


# ---------------------------------------------------------------------------
# Quantization and packing (quant.py)


def fake_quant_int(x, *, bits: int, scale: float) -> np.ndarray:
    """clamp(round(x / scale), qmin, qmax) as int8 (quant.py:14-29).

    ``round`` is round-half-to-even, as torch.round.  ``x`` is taken as
    float32 (the reference calls ``x.float()``).
    """
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    if isinstance(scale, bool) or not isinstance(scale, (int, float)):
        raise TypeError("scale must be a positive Python int or float scalar")
    if scale <= 0:
        raise ValueError("scale must be positive")
    qmin = -(1 << (bits - 1))
    qmax = (1 << (bits - 1)) - 1
    q = np.round(np.asarray(x, dtype=np.float32) / np.float32(scale))
    return np.clip(q, qmin, qmax).astype(np.int8)


def fake_quant_int_device(x, *, bits: int, scale: float) -> np.ndarray:
    """fake_quant_int (quant.py:14-29) as torch evaluates it on a GPU.

    There ``x.float() / scale`` with a Python scalar multiplies by the
    reciprocal of the scale, rounded once from double to float32 (measured on
    MI355X, torch 2.10: bit-identical to ``x * float32(1.0 / scale)`` for
    every value and scale tried, where ``x / float32(scale)`` and
    ``x * (1 / float32(scale))`` both differ); then round half to even and
    clamp as on the CPU, and NaN converts to the code 0.
    """
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    if isinstance(scale, bool) or not isinstance(scale, (int, float)) or scale <= 0:
        raise ValueError("scale must be a positive Python int or float scalar")
    qmin = -(1 << (bits - 1))
    qmax = (1 << (bits - 1)) - 1
    with np.errstate(invalid="ignore", over="ignore"):
        q = np.rint(np.asarray(x, dtype=np.float32) * np.float32(1.0 / scale))
        q = np.clip(q, qmin, qmax)
    return np.where(np.isnan(q), 0, q).astype(np.int8)


def pack_int4_k_major(x) -> np.ndarray:
    """Packs pairs along the last axis: byte = (odd << 4) | (even & 0xF),
    zero-padding an odd length (quant.py:32-38)."""
    x = np.asarray(x, dtype=np.int8)
    if x.shape[-1] % 2:
        pad = [(0, 0)] * (x.ndim - 1) + [(0, 1)]
        x = np.pad(x, pad)
    even = x[..., 0::2].astype(np.int16) & 0xF
    odd = x[..., 1::2].astype(np.int16) & 0xF
    return np.ascontiguousarray(((odd << 4) | even).astype(np.uint8))


def unpack_int4_k_major(p) -> np.ndarray:
    """Inverse of pack_int4_k_major with sign extension of each nibble
    (quant.py:41-51)."""
    p = np.asarray(p, dtype=np.uint8)
    lo = (p & 0xF).astype(np.int8)
    hi = ((p >> 4) & 0xF).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo).astype(np.int8)
    hi = np.where(hi >= 8, hi - 16, hi).astype(np.int8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def pack_rhs_subchannel_scales(b_scale) -> np.ndarray:
    """(..., N, S) -> (..., S, N) (quant.py:54-65)."""
    b = np.asarray(b_scale)
    if b.ndim < 2:
        raise ValueError("b_scale must have at least 2 dimensions to pack RHS subchannel scales")
    return np.ascontiguousarray(np.swapaxes(b, -2, -1))


# ---------------------------------------------------------------------------
# Exact integer matmul


def int_matmul(a, b) -> np.ndarray:
    """Exact int32 result of torch.matmul on int32 operands (api.py:304, :319).

    Computed in int64 and checked to fit int32 (the reference accumulates in
    int32 and never overflows for these operand ranges).
    """
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape[-1] * b.shape[-1] * (a.shape[-2] if a.ndim > 1 else 1) > 64 * 1024 * 1024:
        from . import native  # noqa: PLC0415 - optional accelerated path

        if native.available() and a.ndim == 2 and b.ndim == 2:
            return native.matmul_i8(a.astype(np.int8), b.astype(np.int8))
    r = np.matmul(a.astype(np.int64), b.astype(np.int64))
    if r.size and (r.max() > np.iinfo(np.int32).max or r.min() < np.iinfo(np.int32).min):
        raise OverflowError("int32 accumulator overflow")
    return r.astype(np.int32)


# ---------------------------------------------------------------------------
# Dense reference (api.py:257-325)


def logical_operands(a_arg, b_arg, *, bits: int, layout: str):
    """Unpacks and transposes the physical operands to logical A[M,K], B[K,N]
    (api.py:267-281)."""
    layout = layout.lower()
    a = np.asarray(a_arg)
    b = np.asarray(b_arg)
    if bits == 4:
        if layout in ("tn", "tt"):
            a = unpack_int4_k_major(a.T).T
        else:
            a = unpack_int4_k_major(a)
        if layout in ("nt", "tt"):
            b = unpack_int4_k_major(b)
        else:
            b = unpack_int4_k_major(b.T).T
    else:
        a = a.astype(np.int8)
        b = b.astype(np.int8)
    if layout in ("tn", "tt"):
        a = a.T
    if layout in ("nt", "tt"):
        b = b.T
    return np.ascontiguousarray(a), np.ascontiguousarray(b)


def scaled_mm(a_q, b_q, a_scale_bits, b_scale_bits, *, subchannel: int | None) -> np.ndarray:
    """fp32 result of _scaled_reference_mm (api.py:299-325).

    Per-channel: (float(A@B) * a_scale[:, None]) * b_scale[None, :].
    Subchannel S: zeros, then for each K group g in order:
    out += (float(A_g@B_g) * a_scale[:, g, None]) * b_scale[g, None, :].
    Scales are bf16 bits (None = no scaling, as the reference allows).
    """
    sa = None if a_scale_bits is None else bf16_to_f32(a_scale_bits)
    sb = None if b_scale_bits is None else bf16_to_f32(b_scale_bits)
    if not subchannel:
        out = int_matmul(a_q, b_q).astype(np.float32)
        if sa is not None:
            out = (out * sa[:, None]).astype(np.float32)
        if sb is not None:
            out = (out * sb[None, :]).astype(np.float32)
        return out
    k = a_q.shape[1]
    out = np.zeros((a_q.shape[0], b_q.shape[1]), dtype=np.float32)
    for g, k0 in enumerate(range(0, k, subchannel)):
        k1 = min(k0 + subchannel, k)
        part = int_matmul(a_q[:, k0:k1], b_q[k0:k1, :]).astype(np.float32)
        if sa is not None:
            part = (part * sa[:, g, None]).astype(np.float32)
        if sb is not None:
            part = (part * sb[g, :][None, :]).astype(np.float32)
        out = (out + part).astype(np.float32)
    return out


def relu2(x) -> np.ndarray:
    """torch.relu(x).square() (api.py:290-291)."""
    r = np.maximum(np.asarray(x, dtype=np.float32), np.float32(0.0))
    return (r * r).astype(np.float32)


def swiglu(x) -> np.ndarray:
    """up * (gate / (1 + exp(-gate))) with x = [up | gate] (api.py:283-289).

    numpy's float32 exp may differ from torch's by an ulp; results are
    compared within the bf16 tolerance, never bit for bit.
    """
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1] // 2
    up = x[..., :d]
    gate = x[..., d:]
    # exp(-gate) overflows to inf for gates below about -88: the quotient is
    # then -0 or 0, as torch gives, so the overflow warning is expected
    with np.errstate(over="ignore"):
        den = (np.float32(1.0) + np.exp(-gate).astype(np.float32)).astype(np.float32)
    return (up * (gate / den).astype(np.float32)).astype(np.float32)


def reference_gemm(a_arg, b_arg, *, bits: int, layout: str = "nn", a_scale=None, b_scale=None,
                   subchannel: int | None = None, epilogue: str = "none") -> np.ndarray:
    """fp32 output of reference_mm before the output cast (api.py:257-291)."""
    a_q, b_q = logical_operands(a_arg, b_arg, bits=bits, layout=layout)
    out = scaled_mm(a_q, b_q, a_scale, b_scale, subchannel=subchannel)
    if epilogue == "swiglu":
        out = swiglu(out)
    elif epilogue == "relu2":
        out = relu2(out)
    return out


def reference_gemm_bf16(*args, **kwargs) -> np.ndarray:
    """reference_gemm cast to bf16 bits (api.py:292-293)."""
    return bf16_round(reference_gemm(*args, **kwargs))


# ---------------------------------------------------------------------------
# Ragged task list (ragged.py:201-323, torch branch :307-323)


@dataclass
class GroupInfo:
    group_id: np.ndarray
    block_start: np.ndarray
    actual_start: np.ndarray
    actual_end: np.ndarray
    start_within_block: np.ndarray
    actual_size: np.ndarray
    num_tasks: int


def calculate_group_info(group_sizes, tile: int, *, tid_size: int | None = None, align_tile: int = 8) -> GroupInfo:
    """Row-block task list of calculate_group_info (ragged.py:201-323)."""
    sizes = np.asarray(group_sizes)
    if sizes.ndim != 1:
        raise ValueError(f"group_sizes must be 1D; got shape {tuple(sizes.shape)}")
    if tile <= 0:
        raise ValueError("tile must be positive")
    if align_tile <= 0:
        raise ValueError("align_tile must be positive")
    if tile % align_tile != 0:
        raise ValueError("tile must be a multiple of align_tile")
    if tid_size is not None and tid_size < 0:
        raise ValueError("tid_size must be non-negative")
    sizes = np.clip(sizes.astype(np.int64), 0, None)
    groups = sizes.shape[0]

    def empty(cap, num):
        z = np.zeros((cap,), dtype=np.int64)
        return GroupInfo(z.copy(), z.copy(), z.copy(), z.copy(), z.copy(), z.copy(), num)

    if groups == 0:
        return empty(tid_size or 0, 0)
    starts = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    gstart = starts[:-1]
    aligned = (gstart // align_tile) * align_tile
    gend = gstart + sizes
    blocks = np.where(sizes == 0, 0, (gend - aligned + tile - 1) // tile)
    task_start = np.concatenate([[0], np.cumsum(blocks)]).astype(np.int64)
    num_tasks = int(task_start[-1])
    cap = num_tasks if tid_size is None else tid_size
    if cap < num_tasks:
        raise ValueError(f"tid_size must be at least {num_tasks}; got {cap}")
    info = empty(cap, num_tasks)
    for t in range(num_tasks):
        g = int(np.searchsorted(task_start[1:], t, side="right"))
        g = min(g, groups - 1)
        bs = aligned[g] + (t - task_start[g]) * tile
        a0 = max(bs, gstart[g])
        a1 = min(bs + tile, gend[g])
        info.group_id[t] = g
        info.block_start[t] = bs
        info.actual_start[t] = a0
        info.actual_end[t] = a1
        info.start_within_block[t] = a0 - bs
        info.actual_size[t] = max(a1 - a0, 0)
    return info


# ---------------------------------------------------------------------------
# Grouped ragged references (tests/test_ragged_dot.py:19-117)


def ragged_fwd_reference(a_q, b_q, group_sizes, a_scale_bits, b_scale_bits, *, subchannel: int | None = None):
    """fp32 out[rows of g] = scaled(a_q[rows] @ b_q[g]) (test_ragged_dot.py:19-51).

    a_q: int [M, K]; b_q: int [G, K, N]; per-channel scales a[M], b[G, N];
    subchannel S: a[M, ceil(K/S)], b[G, ceil(K/S), N].
    """
    a_q = np.asarray(a_q)
    b_q = np.asarray(b_q)
    sizes = [int(s) for s in np.asarray(group_sizes)]
    out = np.zeros((a_q.shape[0], b_q.shape[2]), dtype=np.float32)
    row = 0
    for g, sz in enumerate(sizes):
        nxt = row + sz
        if sz:
            sb = None if b_scale_bits is None else np.asarray(b_scale_bits)[g]
            out[row:nxt] = scaled_mm(a_q[row:nxt], b_q[g], None if a_scale_bits is None else np.asarray(a_scale_bits)[row:nxt],
                                     sb, subchannel=subchannel)
        row = nxt
    return out


def ragged_bwd_reference(a_q, b_q, group_sizes, a_scale_bits, b_scale_bits, *, subchannel: int | None = None):
    """fp32 out[g] = scaled(a_q[g][:, :gk] @ b_q[g][:gk]) (test_ragged_dot.py:84-117).

    a_q: int [G, M, Kcap]; b_q: int [G, Kcap, N]; per-channel scales a[G, M],
    b[G, N]; subchannel S: a[G, M, ceil(Kcap/S)], b[G, ceil(Kcap/S), N]; only
    the groups that start below group_sizes[g] contribute, the last one
    truncated at group_sizes[g].
    """
    a_q = np.asarray(a_q)
    b_q = np.asarray(b_q)
    groups, rows, kcap = a_q.shape
    cols = b_q.shape[2]
    out = np.zeros((groups, rows, cols), dtype=np.float32)
    for g, gk in enumerate(int(s) for s in np.asarray(group_sizes)):
        sa = np.asarray(a_scale_bits)[g]
        sb = np.asarray(b_scale_bits)[g]
        if not subchannel:
            out[g] = scaled_mm(a_q[g, :, :gk], b_q[g, :gk, :], sa, sb, subchannel=None)
            continue
        acc = np.zeros((rows, cols), dtype=np.float32)
        for si, k0 in enumerate(range(0, kcap, subchannel)):
            k1 = min(k0 + subchannel, gk)
            if k1 <= k0:
                continue
            part = int_matmul(a_q[g, :, k0:k1], b_q[g, k0:k1, :]).astype(np.float32)
            part = (part * bf16_to_f32(sa[:, si])[:, None]).astype(np.float32)
            part = (part * bf16_to_f32(sb[si, :])[None, :]).astype(np.float32)
            acc = (acc + part).astype(np.float32)
        out[g] = acc
    return out


# ---------------------------------------------------------------------------
# TOPS accounting (benchmarking.py:104-111; SwiGLU counts up + gate, autotune.py:971-976)


def gemm_ops(m: int, n: int, k: int) -> int:
    return 2 * int(m) * int(n) * int(k)


def tops_for_runtime(m: int, n: int, k: int, runtime_ms: float) -> float:
    return gemm_ops(m, n, k) / (runtime_ms * 1.0e-3) / 1.0e12


# ---------------------------------------------------------------------------
# Seeded inputs of the benchmark configs (C1-C5, scaled down
# where a test needs a small case)


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def uniform_bf16(r: np.random.Generator, shape, lo: float, hi: float) -> np.ndarray:
    return bf16_round(r.uniform(lo, hi, size=shape).astype(np.float32))


def randint4(r: np.random.Generator, shape) -> np.ndarray:
    return r.integers(-8, 8, size=shape, dtype=np.int8)


def randint8(r: np.random.Generator, shape) -> np.ndarray:
    return r.integers(-127, 128, size=shape, dtype=np.int8)


def randn_bf16_fake_quant(r: np.random.Generator, shape, *, bits: int, std: float = 0.1, scale: float = 0.1):
    """randn * std rounded to bf16, then fake-quantized (config C1's recipe)."""
    x = bf16_to_f32(bf16_round((r.standard_normal(shape) * std).astype(np.float32)))
    return fake_quant_int(x, bits=bits, scale=scale)


def pack_operands(a_q, b_q, *, bits: int, layout: str):
    """Physical operands of a layout from logical A[M,K], B[K,N]
    (tests/test_quant.py:112-129)."""
    layout = layout.lower()
    a_trans = layout in ("tn", "tt")
    b_trans = layout in ("nt", "tt")
    if bits == 4:
        a_arg = pack_int4_k_major(a_q)
        if a_trans:
            a_arg = np.ascontiguousarray(a_arg.T)
        b_arg = pack_int4_k_major(np.asarray(b_q).T)
        if not b_trans:
            b_arg = np.ascontiguousarray(b_arg.T)
        return a_arg, b_arg
    a_arg = np.ascontiguousarray(np.asarray(a_q).T) if a_trans else np.ascontiguousarray(a_q)
    b_arg = np.ascontiguousarray(np.asarray(b_q).T) if b_trans else np.ascontiguousarray(b_q)
    return a_arg, b_arg


def multinomial_group_sizes(r: np.random.Generator, rows: int, groups: int) -> np.ndarray:
    """Dirichlet(1) probabilities, multinomial counts, then at least one empty
    group: the smallest group's rows move to the largest group."""
    p = r.dirichlet(np.ones(groups))
    sizes = r.multinomial(rows, p).astype(np.int64)
    if not (sizes == 0).any():
        lo = int(np.argmin(sizes))
        hi = int(np.argmax(sizes))
        sizes[hi] += sizes[lo]
        sizes[lo] = 0
    return sizes
