"""Launch-shape contract of a dense kernel (template_config.py:8-80).

Dense kernels run only on tile-multiple shapes; the rejection reasons and their
wording are the reference's, so callers that parse them keep working.
"""

from __future__ import annotations

from dataclasses import dataclass

from . import kernel_table
from .metadata import Epilogue, KernelMetadata, OperandDType, ScaleMode


@dataclass(frozen=True, slots=True)
class LaunchShape:
    m: int
    n: int
    k: int

    def validate_for(self, kernel: KernelMetadata) -> None:
        reasons = tile_multiple_rejection_reasons(kernel, self)
        if reasons:
            raise ValueError(f"{kernel.kernel_id} requires tile-multiple shape: " + "; ".join(reasons))


def tile_multiple_rejection_reasons(kernel: KernelMetadata, shape: LaunchShape) -> tuple[str, ...]:
    if shape.m <= 0 or shape.n <= 0 or shape.k <= 0:
        return (f"M, N, and K must be positive; got ({shape.m}, {shape.n}, {shape.k})",)
    tile = kernel.tile
    out: list[str] = []
    if shape.m % tile.block_m:
        out.append(f"M={shape.m} is not divisible by BLOCK_M={tile.block_m}")
    if shape.n % tile.block_n:
        out.append(f"N={shape.n} is not divisible by BLOCK_N={tile.block_n}")
    period = tile.block_k * tile.split_k
    if shape.k % period:
        out.append(f"K={shape.k} is not divisible by BLOCK_K*SPLIT_K={period}")
    sub = kernel.scale.subchannel_size
    if kernel.scale.mode is ScaleMode.SUBCHANNEL and sub is not None and shape.k % sub:
        out.append(f"K={shape.k} is not divisible by SUBCHANNEL={sub}")
    elif (kernel.scale.mode is ScaleMode.SUBCHANNEL and sub is not None and tile.split_k > 1
          and _slices_k(kernel) and (shape.k // tile.split_k) % sub):
        # each K slice of a split-K kernel starts at a scale group boundary
        out.append(f"K/SPLIT_K={shape.k // tile.split_k} is not divisible by SUBCHANNEL={sub}")
    return tuple(out)


def _slices_k(kernel: KernelMetadata) -> bool:
    """Whether a split-K kernel cuts K into SPLIT_K contiguous slices (the
    gfx950 split tiles); the skinny (STREAM) split tiles fold every scale
    group of the whole K in one workgroup and need no slice boundary."""
    if kernel.table_index is None:
        return True
    return kernel_table.TABLE[kernel.table_index].operand_format != kernel_table.OPERANDS_STREAM


def is_tile_multiple_shape(kernel: KernelMetadata, shape: LaunchShape) -> bool:
    return not tile_multiple_rejection_reasons(kernel, shape)


@dataclass(frozen=True, slots=True)
class TemplatePlan:
    kernel: KernelMetadata
    shape: LaunchShape
    needs_packed_int4: bool
    needs_subchannel_loop: bool
    needs_per_channel_epilogue_scale: bool
    needs_relu2_activation: bool
    needs_fused_swiglu_up_gate: bool
    even_k: bool
    split_k: int


def plan_template(kernel: KernelMetadata, shape: LaunchShape) -> TemplatePlan:
    shape.validate_for(kernel)
    return TemplatePlan(
        kernel=kernel,
        shape=shape,
        needs_packed_int4=kernel.a_dtype is OperandDType.INT4,
        needs_subchannel_loop=kernel.scale.mode is ScaleMode.SUBCHANNEL,
        needs_per_channel_epilogue_scale=kernel.scale.mode is ScaleMode.PER_CHANNEL,
        needs_relu2_activation=kernel.epilogue is Epilogue.RELU2,
        needs_fused_swiglu_up_gate=kernel.epilogue is Epilogue.SWIGLU,
        even_k=kernel.tile.even_k,
        split_k=kernel.tile.split_k,
    )


def representative_generation_shape(kernel: KernelMetadata) -> LaunchShape:
    """Smallest tile-multiple shape a kernel accepts (template_config.py:73-80)."""
    period = kernel.tile.block_k * kernel.tile.split_k
    k = period
    if kernel.scale.mode is ScaleMode.SUBCHANNEL:
        sub = kernel.scale.subchannel_size or period
        while k < sub or k % sub:
            k += period
    return LaunchShape(kernel.tile.block_m, kernel.tile.block_n, k)
