"""Shape support and kernel choice over the registry (reference heuristics.py:9-60).

``kernel_supports_shape`` is the reference's rule: the shape is a multiple
of the tile (and of the subchannel), the kernel has no K tail, and fused
RELU2 / SwiGLU epilogues never run split-K; K must also be within the
kernel's gfx950 bound.  ``estimate_kernel_score`` ranks
a kernel by a benchmark database record for the exact shape when there is
one, otherwise by the kernel's measured MI355X throughput divided by its
split-K factor.  The reference's extra weight for its 64x512x64 Triton tile
has no counterpart here: the scores of this kernel table are measured on
MI355X.
"""

from __future__ import annotations

from . import kernel_table as kt
from .benchmarking import BenchmarkDatabase, BenchmarkShape
from .metadata import Epilogue, GemmLayout, KernelMetadata, KernelSchedule, OperandDType, ScaleSpec
from .registry import KernelRegistry, default_registry
from .template_config import LaunchShape, is_tile_multiple_shape


def kernel_supports_shape(kernel: KernelMetadata, *, m: int, n: int, k: int) -> bool:
    """The reference's rule, plus the K bound of the kernel's gfx950 table
    entry (its int32 accumulators and buffer offsets)."""
    if kernel.epilogue in {Epilogue.RELU2, Epilogue.SWIGLU} and kernel.tile.split_k != 1:
        return False
    return (kernel.tile.even_k and is_tile_multiple_shape(kernel, LaunchShape(m, n, k))
            and (kernel.table_index is None or kt.TABLE[kernel.table_index].supports_k(k)))


def estimate_kernel_score(
    kernel: KernelMetadata,
    *,
    m: int,
    n: int,
    k: int,
    benchmark_db: BenchmarkDatabase | None = None,
) -> float:
    if not kernel_supports_shape(kernel, m=m, n=n, k=k):
        return float("-inf")
    if benchmark_db is not None:
        record = benchmark_db.best_record(kernel, BenchmarkShape(m, n, k))
        if record is not None:
            return record.tops
    return (kernel.measured_tops or 1.0) / kernel.tile.split_k


def choose_kernel(
    *,
    m: int,
    n: int,
    k: int,
    dtype: OperandDType,
    layout: GemmLayout = GemmLayout.NN,
    scale: ScaleSpec,
    epilogue: Epilogue,
    schedule: KernelSchedule = KernelSchedule.STANDARD,
    registry: KernelRegistry = default_registry,
    benchmark_db: BenchmarkDatabase | None = None,
) -> KernelMetadata:
    """The best-scoring registry kernel for the request and shape."""
    candidates = [
        kern for kern in registry.all()
        if kern.a_dtype is dtype and kern.b_dtype is dtype and kern.layout is layout and kern.scale == scale
        and kern.epilogue is epilogue and kern.schedule is schedule
        and kernel_supports_shape(kern, m=m, n=n, k=k)
    ]
    if not candidates:
        raise LookupError("no kernels match logical dtype/layout/scale/epilogue request and shape")
    return max(candidates, key=lambda kern: estimate_kernel_score(kern, m=m, n=n, k=k, benchmark_db=benchmark_db))
