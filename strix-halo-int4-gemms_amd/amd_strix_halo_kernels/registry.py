"""Kernel registry over the gfx950 kernel table.

Same selection contract as the reference's KernelRegistry (registry.py:254-352):
candidates must match dtype, scale spec, epilogue, layout and schedule, be
even-K, obey the split rule, and (for ``select``) accept the shape as a tile
multiple; among them the one with the largest (measured_tops or 0,
BLOCK_M * BLOCK_N) wins, the first on ties (the skinny subchannel tiles'
figure counts up to kernel_table.SKINNY_SUB_MAX_M rows).  The entries come from the gfx950
kernel table (``kernel_table.TABLE``) instead of gfx1151 tile seeds: every
dense table entry is registered once per epilogue and subchannel size it
serves.
"""

from __future__ import annotations

from dataclasses import replace
from typing import Iterable

from . import kernel_table as kt
from .metadata import (
    ACC_DTYPE,
    ARCH,
    SCALE_DTYPE_BF16,
    SUPPORTED_SUBCHANNELS,
    Epilogue,
    GemmLayout,
    KernelMetadata,
    KernelSchedule,
    KernelStatus,
    OperandDType,
    ScaleMode,
    ScaleSpec,
    TileConfig,
    make_kernel_id,
    output_dtype_for_split_k,
)
from .template_config import LaunchShape, is_tile_multiple_shape

_LAYOUT_OF_CODE = {kt.LAYOUT_NN: GemmLayout.NN, kt.LAYOUT_NT: GemmLayout.NT, kt.LAYOUT_TN: GemmLayout.TN,
                   kt.LAYOUT_TT: GemmLayout.TT}


def _tile_of(desc: kt.KernelDesc) -> TileConfig:
    return TileConfig(
        block_m=desc.block_m,
        block_n=desc.block_n,
        block_k=desc.block_k,
        group_size_m=desc.group_size_m,
        num_warps=desc.num_waves,
        num_stages=desc.num_stages,
        waves_per_eu=max(1, desc.num_waves // 4),
        even_k=True,
        split_k=desc.split_k,
    )


def _scales_of(desc: kt.KernelDesc) -> tuple[ScaleSpec, ...]:
    if desc.scale_mode == kt.SCALE_PER_CHANNEL:
        return (ScaleSpec(ScaleMode.PER_CHANNEL),)
    return tuple(
        ScaleSpec(ScaleMode.SUBCHANNEL, s)
        for s in SUPPORTED_SUBCHANNELS
        if desc.min_subchannel <= s <= desc.max_subchannel
    )


def _epilogues_of(desc: kt.KernelDesc) -> tuple[Epilogue, ...]:
    if desc.epilogue_kind == kt.EPI_KIND_SWIGLU:
        return (Epilogue.SWIGLU,)
    if desc.schedule == kt.SCHEDULE_PERSISTENT or desc.split_k > 1:
        return (Epilogue.NONE,)  # the reference's persistent kernels (registry.py:230-251)
    return (Epilogue.NONE, Epilogue.RELU2)


def iter_supported_kernel_metadata() -> Iterable[KernelMetadata]:
    """One KernelMetadata per (dense table entry, epilogue, scale spec)."""
    for desc in kt.entries(kt.FAMILY_DENSE):
        dtype = OperandDType.INT4 if desc.dtype_bits == 4 else OperandDType.INT8
        tile = _tile_of(desc)
        layout = _LAYOUT_OF_CODE[desc.layout]
        for scale in _scales_of(desc):
            for epilogue in _epilogues_of(desc):
                schedule = (KernelSchedule.PERSISTENT if desc.schedule == kt.SCHEDULE_PERSISTENT
                            else KernelSchedule.STANDARD)
                kernel_id = make_kernel_id(dtype, scale, epilogue, tile, arch=ARCH, layout=layout, schedule=schedule)
                yield KernelMetadata(
                    kernel_id=kernel_id,
                    arch=ARCH,
                    a_dtype=dtype,
                    b_dtype=dtype,
                    acc_dtype=ACC_DTYPE,
                    output_dtype=output_dtype_for_split_k(tile.split_k),
                    scale_dtype=SCALE_DTYPE_BF16,
                    scale=scale,
                    epilogue=epilogue,
                    tile=tile,
                    triton_kernel_name=f"shk::dense_gemm_kernel#{desc.index}",
                    layout=layout,
                    schedule=schedule,
                    assembly_path=None,
                    status=KernelStatus.COMPILED,
                    table_index=desc.index,
                    measured_tops=kt.measured_tops(desc),
                )


def _selection_key(kernel: KernelMetadata, m: int) -> tuple[float, int]:
    tops = kernel.measured_tops
    if tops is not None and kernel.table_index is not None and m > kt.SKINNY_SUB_MAX_M:
        desc = kt.TABLE[kernel.table_index]
        if desc.operand_format == kt.OPERANDS_STREAM and desc.scale_mode == kt.SCALE_SUBCHANNEL:
            tops = None  # the skinny subchannel figure holds for few rows only (kernel_table.selection_tops)
    return (tops or 0.0, kernel.tile.block_m * kernel.tile.block_n)


def _matches(kernel: KernelMetadata, dtype, scale, epilogue, layout, schedule, split_k) -> bool:
    return (
        kernel.a_dtype is dtype
        and kernel.b_dtype is dtype
        and kernel.scale == scale
        and kernel.epilogue is epilogue
        and kernel.layout is layout
        and kernel.schedule is schedule
        and not (kernel.epilogue in {Epilogue.RELU2, Epilogue.SWIGLU} and kernel.tile.split_k != 1)
        and (split_k is None or kernel.tile.split_k == split_k)
        and kernel.tile.even_k
    )


def _runs_k(kernel: KernelMetadata, k: int) -> bool:
    """The library's K bound of the kernel's table entry (gfx950 accumulators
    and buffer offsets); kernels without a table entry have none."""
    if kernel.table_index is None:
        return True
    return kt.TABLE[kernel.table_index].supports_k(k)


class KernelRegistry:
    def __init__(self, kernels: Iterable[KernelMetadata] = ()) -> None:
        self._kernels: dict[str, KernelMetadata] = {}
        # Selections are memoized per request (mm() selects on every call, and
        # a scan of the table costs hundreds of microseconds); the candidates
        # are indexed by family.  register() clears both.
        self._families: dict[tuple, list[KernelMetadata]] | None = None
        self._selected: dict[tuple, KernelMetadata] = {}
        for kernel in kernels:
            self.register(kernel)

    def register(self, kernel: KernelMetadata) -> None:
        if kernel.kernel_id in self._kernels:
            raise ValueError(f"duplicate kernel id: {kernel.kernel_id}")
        self._kernels[kernel.kernel_id] = kernel
        self._families = None
        self._selected = {}

    def _family(self, dtype, scale, epilogue, layout, schedule) -> list[KernelMetadata]:
        families = self._families
        if families is None:
            families = {}
            for kern in self._kernels.values():
                if kern.a_dtype is kern.b_dtype:
                    key = (kern.a_dtype, kern.scale, kern.epilogue, kern.layout, kern.schedule)
                    families.setdefault(key, []).append(kern)
            self._families = families
        return families.get((dtype, scale, epilogue, layout, schedule), [])

    def get(self, kernel_id: str) -> KernelMetadata:
        return self._kernels[kernel_id]

    def all(self) -> tuple[KernelMetadata, ...]:
        return tuple(self._kernels.values())

    def select(
        self,
        *,
        dtype: OperandDType,
        scale: ScaleSpec,
        epilogue: Epilogue,
        m: int,
        n: int,
        k: int,
        layout: GemmLayout = GemmLayout.NN,
        split_k: int | None = None,
        schedule: KernelSchedule = KernelSchedule.STANDARD,
        require_compiled: bool = False,
    ) -> KernelMetadata:
        request = (dtype, scale, epilogue, m, n, k, layout, split_k, schedule, require_compiled)
        hit = self._selected.get(request)
        if hit is not None:
            return hit
        shape = LaunchShape(m, n, k)
        candidates = [
            kernel
            for kernel in self._family(dtype, scale, epilogue, layout, schedule)
            if _matches(kernel, dtype, scale, epilogue, layout, schedule, split_k)
            and is_tile_multiple_shape(kernel, shape)
            and _runs_k(kernel, k)
        ]
        if require_compiled:
            candidates = [c for c in candidates if c.status in {KernelStatus.COMPILED, KernelStatus.BENCHMARKED}]
        if not candidates:
            raise LookupError(
                f"no kernel for dtype={dtype.value}, scale={scale.label}, epilogue={epilogue.value}, "
                f"layout={layout.value}, schedule={schedule.value}, shape=({m}, {n}, {k})"
            )
        chosen = max(candidates, key=lambda kern: _selection_key(kern, m))
        if len(self._selected) >= 4096:  # bounded for callers that vary M call to call
            self._selected = {}
        self._selected[request] = chosen
        return chosen

    def select_reference(
        self,
        *,
        dtype: OperandDType,
        scale: ScaleSpec,
        epilogue: Epilogue,
        layout: GemmLayout = GemmLayout.NN,
        split_k: int | None = 1,
        schedule: KernelSchedule = KernelSchedule.STANDARD,
    ) -> KernelMetadata:
        candidates = [
            kernel
            for kernel in self._family(dtype, scale, epilogue, layout, schedule)
            if _matches(kernel, dtype, scale, epilogue, layout, schedule, split_k)
        ]
        if not candidates:
            raise LookupError(
                f"no reference kernel metadata for dtype={dtype.value}, scale={scale.label}, "
                f"epilogue={epilogue.value}, layout={layout.value}, schedule={schedule.value}"
            )
        # no shape: rank as for a large M (the skinny subchannel figure applies to few rows only)
        return max(candidates, key=lambda kern: _selection_key(kern, 1 << 30))

    def with_status(self, kernel_id: str, status: KernelStatus, **updates: object) -> "KernelRegistry":
        copied = KernelRegistry(self._kernels.values())
        copied._kernels[kernel_id] = replace(copied._kernels[kernel_id], status=status, **updates)
        return copied


default_registry = KernelRegistry(iter_supported_kernel_metadata())
