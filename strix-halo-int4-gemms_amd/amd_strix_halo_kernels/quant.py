"""Quantization and int4 packing helpers (torch), the wire format of the path.

Same functions and error messages as the reference's quant.py:14-81.  Packed
int4 stores two two's-complement nibbles per byte along the packed axis: the
even element in the low nibble, the odd element in the high nibble; an odd
length is padded with a zero element.
"""

from __future__ import annotations

from typing import Any


def _torch() -> Any:
    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("torch is required for quantization helpers") from exc
    return torch


def fake_quant_int(x: Any, *, bits: int, scale: float) -> Any:
    """Signed integer codes clamp(round(x / scale)) as int8 (quant.py:14-29).

    The result holds int4/int8 codes, not dequantized values; pack int4 codes
    with pack_int4_k_major(...).
    """
    torch = _torch()
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    if isinstance(scale, bool) or not isinstance(scale, (int, float)):
        raise TypeError("scale must be a positive Python int or float scalar")
    if scale <= 0:
        raise ValueError("scale must be positive")
    lo = -(1 << (bits - 1))
    hi = (1 << (bits - 1)) - 1
    return torch.clamp(torch.round(x.float() / scale), lo, hi).to(torch.int8)


def pack_int4_k_major(x: Any) -> Any:
    """Packs int4 codes pairwise along the last axis (quant.py:32-38)."""
    torch = _torch()
    if x.shape[-1] % 2:
        x = torch.nn.functional.pad(x, (0, 1))
    lo = x[..., 0::2].to(torch.int16) & 0xF
    hi = x[..., 1::2].to(torch.int16) & 0xF
    return (lo | (hi << 4)).to(torch.uint8).contiguous()


def unpack_int4_k_major(x_packed: Any) -> Any:
    """Sign-extending inverse of pack_int4_k_major (quant.py:41-51)."""
    torch = _torch()
    lo = (x_packed & 0xF).to(torch.int8)
    hi = (x_packed >> 4).to(torch.int8) & 0xF
    lo = torch.where(lo > 7, lo - 16, lo)
    hi = torch.where(hi > 7, hi - 16, hi)
    return torch.stack((lo, hi), dim=-1).reshape(*x_packed.shape[:-1], 2 * x_packed.shape[-1])


def pack_rhs_subchannel_scales(b_scale: Any) -> Any:
    """Logical RHS subchannel scales (..., N, scale_cols) -> the weight-matched
    physical layout (..., scale_cols, N) the kernels read (quant.py:54-65)."""
    if b_scale.ndim < 2:
        raise ValueError("b_scale must have at least 2 dimensions to pack RHS subchannel scales")
    return b_scale.transpose(-2, -1).contiguous()


def pack_ragged_rhs_subchannel_scales(b_scale: Any) -> Any:
    """Ragged RHS subchannel scales (G, N, S) -> (G, S, N) (quant.py:68-73)."""
    if b_scale.ndim != 3:
        raise ValueError("ragged b_scale must have shape (G, N, scale_cols)")
    return pack_rhs_subchannel_scales(b_scale)


def apply_scales(result: Any, a_scale: Any | None, b_scale: Any | None) -> Any:
    """result * a_scale[..., :, None] * b_scale[..., None, :] (quant.py:76-81)."""
    if a_scale is not None:
        result = result * a_scale[..., :, None]
    if b_scale is not None:
        result = result * b_scale[..., None, :]
    return result
