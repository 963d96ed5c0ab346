"""Helpers shared by the GPU tests: numpy <-> torch transfers and case builders."""

from __future__ import annotations

import hashlib

import numpy as np

from oracle import ref


def stable_seed(*parts) -> int:
    """Process-independent seed (Python's hash() is salted per process)."""
    text = "|".join(str(p) for p in parts)
    return int.from_bytes(hashlib.sha256(text.encode()).digest()[:4], "little") & 0x7FFFFFFF


def to_dev(torch, arr, device):
    a = np.ascontiguousarray(arr)
    if a.dtype == np.uint16:  # bf16 bits
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)
    return torch.from_numpy(a).to(device)


def bf16_bits(torch, t) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def dense_case(seed: int, *, bits: int, layout: str, m: int, n: int, k: int, subchannel: int | None,
               swiglu: bool, scale_lo: float = 0.005, scale_hi: float = 0.02):
    """Random logical operands, physical operands for `layout`, and bf16 scales."""
    r = ref.rng(seed)
    b_cols = 2 * n if swiglu else n
    a_q = ref.randint4(r, (m, k)) if bits == 4 else ref.randint8(r, (m, k))
    b_q = ref.randint4(r, (k, b_cols)) if bits == 4 else ref.randint8(r, (k, b_cols))
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=bits, layout=layout)
    if subchannel:
        cols = -(-k // subchannel)
        sa = ref.uniform_bf16(r, (m, cols), scale_lo, scale_hi)
        sb = ref.uniform_bf16(r, (cols, b_cols), scale_lo, scale_hi)
    else:
        sa = ref.uniform_bf16(r, (m,), scale_lo, scale_hi)
        sb = ref.uniform_bf16(r, (b_cols,), scale_lo, scale_hi)
    return a_q, b_q, a_arg, b_arg, sa, sb


def max_ulp(a_bits, b_bits) -> int:
    return int(ref.bf16_ulp_diff(a_bits, b_bits).max()) if np.size(a_bits) else 0
