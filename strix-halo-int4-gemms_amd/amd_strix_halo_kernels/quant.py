"""Quantization and int4 packing helpers, the wire format of the path.

Same functions and error messages as the reference's quant.py:14-81.  Packed
int4 stores two two's-complement nibbles per byte along the packed axis: the
even element in the low nibble, the odd element in the high nibble; an odd
length is padded with a zero element.

CPU tensors run the reference's torch code.  CUDA tensors run the library's
one-pass HIP kernel (amd_strix_halo_kernels_quantize), which gives the bits
torch gives on the GPU: there ``x.float() / scale`` multiplies by the
reciprocal of the Python scale, rounded once to fp32 from double, and NaN
converts to the code 0.  ``quantize_pack_int4`` fuses fake_quant_int(bits=4)
with the packing along either of the last two axes.
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
    if _on_device(x):
        return _device_codes(torch, x, bits=bits, scale=scale)
    lo = -(1 << (bits - 1))
    hi = (1 << (bits - 1)) - 1
    return torch.clamp(torch.round(x.float() / scale), lo, hi).to(torch.int8)


def _on_device(x: Any) -> bool:
    return getattr(getattr(x, "device", None), "type", None) == "cuda"


def _rows(x: Any) -> Any:
    """x as a 2-D [prod(leading dims), last dim] tensor."""
    return x.reshape(1, 1) if x.dim() == 0 else x.reshape(-1, x.shape[-1])


def _device_codes(torch: Any, x: Any, *, bits: int, scale: float) -> Any:
    from . import kernel_table as kt
    from .native import quantize_device

    xf = x if x.dtype in (torch.float32, torch.float16, torch.bfloat16) else x.float()
    out = quantize_device(_rows(xf), mode=kt.QUANT_CODES, bits=bits, inv_scale=1.0 / scale)
    return out.reshape(x.shape)


def pack_int4_k_major(x: Any) -> Any:
    """Packs int4 codes pairwise along the last axis (quant.py:32-38)."""
    torch = _torch()
    if _on_device(x) and x.dim() > 0 and not x.dtype.is_floating_point and not x.dtype.is_complex:
        from . import kernel_table as kt
        from .native import quantize_device

        # narrowing to int8 keeps the low byte, so the low nibble packed is the same
        codes = x if x.dtype == torch.int8 else x.to(torch.int8)
        out = quantize_device(_rows(codes), mode=kt.QUANT_PACK_COLS, bits=4)
        return out.reshape(*x.shape[:-1], (x.shape[-1] + 1) // 2)
    if x.shape[-1] % 2:
        x = torch.nn.functional.pad(x, (0, 1))
    lo = x[..., 0::2].to(torch.int16) & 0xF
    hi = x[..., 1::2].to(torch.int16) & 0xF
    return (lo | (hi << 4)).to(torch.uint8).contiguous()


def quantize_pack_int4(x: Any, *, scale: float, axis: int = -1) -> Any:
    """pack_int4_k_major(fake_quant_int(x, bits=4, scale=scale)) along `axis`.

    axis=-1 packs pairs along the last axis (the K-major A operand, or any
    row-major activation); axis=-2 packs pairs of rows of the last two axes,
    ``pack_int4_k_major(q.transpose(-1, -2)).transpose(-1, -2)`` (the NN B
    operand [K/2, N], or activations packed along the rows for the K-ragged
    backward).  On CUDA tensors this is one pass over HBM: read x once,
    write the packed bytes once.
    """
    torch = _torch()
    if isinstance(scale, bool) or not isinstance(scale, (int, float)):
        raise TypeError("scale must be a positive Python int or float scalar")
    if scale <= 0:
        raise ValueError("scale must be positive")
    nd = x.dim()
    ax = axis + nd if axis < 0 else axis
    if ax < 0 or ax not in (nd - 1, nd - 2):
        raise ValueError("axis must be -1 (the last axis) or -2 (pairs of rows of the last two axes)")
    rows_axis = ax == nd - 2
    if not _on_device(x):
        q = fake_quant_int(x, bits=4, scale=scale)
        if rows_axis:
            return pack_int4_k_major(q.transpose(-1, -2)).transpose(-1, -2).contiguous()
        return pack_int4_k_major(q)
    from . import kernel_table as kt
    from .native import quantize_device

    xf = x if x.dtype in (torch.float32, torch.float16, torch.bfloat16) else x.float()
    inv = 1.0 / scale
    if not rows_axis:
        out = quantize_device(_rows(xf), mode=kt.QUANT_PACK_COLS, bits=4, inv_scale=inv)
        return out.reshape(*x.shape[:-1], (x.shape[-1] + 1) // 2)
    rows, cols = int(x.shape[-2]), int(x.shape[-1])
    lead = tuple(x.shape[:-2])
    if rows % 2 == 0 or not lead:
        # pairs never cross a matrix of the batch
        out = quantize_device(xf.reshape(-1, cols), mode=kt.QUANT_PACK_ROWS, bits=4, inv_scale=inv)
        return out.reshape(*lead, (rows + 1) // 2, cols)
    parts = [quantize_device(m, mode=kt.QUANT_PACK_ROWS, bits=4, inv_scale=inv) for m in xf.reshape(-1, rows, cols)]
    return torch.stack(parts).reshape(*lead, (rows + 1) // 2, cols)


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
