"""Grouped ragged int4 dot: ragged_dot_int4, ragged_dot_int4_bwd, calculate_group_info.

Public signatures, validation order and messages follow the reference's
ragged.py (ragged.py:11-72, 201-366, 834-1402).  What differs is underneath:

* the row-block task list is built on the device by one HIP kernel and read
  by the forward kernel from device memory, so the forward issues no
  host synchronisation beyond the reference's own group-size validation
  (ragged.py:846-860);
* the kernels are the gfx950 table kernels; the Triton JIT fallback of the
  reference does not exist, and ``use_native=False`` (which asked for it) is
  rejected;
* per-channel calls with N a multiple of 8 (and a 16-byte aligned output,
  an 8-byte aligned b_scale) run the fp6 kernels, which convert both int4
  operands into a workspace and use the fp6 MFMA at twice the int8 rate; the
  forward's task tile is then 128 rows with align_tile 32;
* otherwise ``RaggedDotConfig.block_m`` / ``align_tile`` set the task tiling
  when the table has that block_m (16, 32, 64, 128), else 64 is used (block_m
  64, the default, and 256 leave the choice of the fp6 kernel to the
  library); block_n, block_k, num_warps and num_stages are Triton tuning
  knobs with no effect on the result, and the gfx950 kernels use their own;
* ``RaggedBwdDotConfig.split_k`` is honoured: per-channel splits add exact
  int32 partials (the result equals split_k=1), subchannel splits own whole
  scale groups and add fp32 partials (as the reference, atomically);
* missing scales are treated as ones (the reference's JIT path accepted them).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

from . import kernel_table as kt
from .metadata import GemmLayout, ScaleMode, ScaleSpec

RAGGED_FWD = "fwd"
RAGGED_BWD = "bwd"
RAGGED_EVEN_K = "evenk"
RAGGED_MASK_K = "maskk"


@dataclass(frozen=True, slots=True)
class RaggedDotConfig:
    """Launch configuration of the forward ragged dot (ragged.py:11-36)."""

    block_m: int = 64
    block_n: int = 256
    block_k: int = 64
    align_tile: int = 8
    group_size_tasks: int = 1
    enable_even_k_fast_path: bool = True
    num_warps: int = 8
    num_stages: int = 3

    def __post_init__(self) -> None:
        if self.block_m <= 0 or self.block_n <= 0 or self.block_k <= 0:
            raise ValueError("block_m, block_n, and block_k must be positive")
        if self.block_k % 2 != 0:
            raise ValueError("block_k must be even for packed int4 operands")
        if self.align_tile <= 0:
            raise ValueError("align_tile must be positive")
        if self.block_m % self.align_tile != 0:
            raise ValueError("block_m must be a multiple of align_tile")
        if self.group_size_tasks <= 0:
            raise ValueError("group_size_tasks must be positive")
        if self.num_warps <= 0 or self.num_stages <= 0:
            raise ValueError("num_warps and num_stages must be positive")


@dataclass(frozen=True, slots=True)
class RaggedBwdDotConfig:
    """Launch configuration of the K-ragged backward dot (ragged.py:39-59)."""

    block_m: int = 64
    block_n: int = 256
    block_k: int = 64
    split_k: int = 1
    num_warps: int = 8
    num_stages: int = 3
    enable_even_k_fast_path: bool = True

    def __post_init__(self) -> None:
        if self.block_m <= 0 or self.block_n <= 0 or self.block_k <= 0:
            raise ValueError("block_m, block_n, and block_k must be positive")
        if self.block_k % 2 != 0:
            raise ValueError("block_k must be even for packed int4 operands")
        if self.split_k <= 0:
            raise ValueError("split_k must be positive")
        if self.num_warps <= 0 or self.num_stages <= 0:
            raise ValueError("num_warps and num_stages must be positive")


@dataclass(frozen=True, slots=True)
class RaggedGroupInfo:
    """Compact row-block assignments for grouped ragged dot (ragged.py:62-72)."""

    group_id: Any
    block_start: Any
    actual_start: Any
    actual_end: Any
    start_within_block: Any
    actual_size: Any
    num_tasks: int


def _torch() -> Any:
    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("torch is required for ragged_dot_int4") from exc
    return torch


def _cdiv(x: int, y: int) -> int:
    return (x + y - 1) // y


def _is_integer_dtype(torch: Any, dtype: Any) -> bool:
    return dtype in {torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8}


def _check_layout(layout: GemmLayout) -> GemmLayout:
    if type(layout) is not GemmLayout:
        raise TypeError(f"layout must be a GemmLayout, got {type(layout).__name__}")
    return layout


# ---------------------------------------------------------------------------
# Task list


def _host_group_info(torch: Any, sizes: Any, tile: int, align_tile: int, tid_size: int | None) -> RaggedGroupInfo:
    """Task list computed with torch ops on the CPU (the contract of
    ragged.py:245-323 for CPU tensors)."""
    i64 = torch.int64
    groups = int(sizes.shape[0])
    if groups == 0:
        cap = tid_size or 0
        z = [torch.zeros((cap,), dtype=i64) for _ in range(6)]
        return RaggedGroupInfo(*z, num_tasks=0)
    ends = torch.cumsum(sizes, 0)
    starts = ends - sizes
    aligned = torch.div(starts, align_tile, rounding_mode="floor") * align_tile
    blocks = torch.where(sizes > 0, torch.div(ends - aligned + tile - 1, tile, rounding_mode="floor"),
                         torch.zeros_like(sizes))
    task_end = torch.cumsum(blocks, 0)
    num_tasks = int(task_end[-1].item()) if groups else 0
    cap = num_tasks if tid_size is None else tid_size
    if cap < num_tasks:
        raise ValueError(f"tid_size must be at least {num_tasks}; got {cap}")
    t = torch.arange(cap, dtype=i64)
    valid = t < num_tasks
    g = torch.clamp(torch.searchsorted(task_end, t, right=True), max=groups - 1)
    first_task = task_end[g] - blocks[g]
    bstart = aligned[g] + (t - first_task) * tile
    astart = torch.maximum(bstart, starts[g])
    aend = torch.minimum(bstart + tile, ends[g])
    zero = torch.zeros_like(t)
    fields = [g, bstart, astart, aend, astart - bstart, torch.clamp(aend - astart, min=0)]
    return RaggedGroupInfo(*[torch.where(valid, f, zero) for f in fields], num_tasks=num_tasks)


def calculate_group_info(
    group_sizes: Any,
    tile: int,
    *,
    tid_size: int | None = None,
    align_tile: int = 8,
    allow_triton: bool = True,
) -> RaggedGroupInfo:
    """Aligned row-block assignments (ragged.py:201-323).

    Group ``g`` owns rows ``[sum(group_sizes[:g]), sum(group_sizes[:g+1]))``;
    task ``t`` covers rows ``[block_start, block_start + tile)`` of one group,
    of which ``[actual_start, actual_end)`` belong to it.  Without ``tid_size``
    the arrays hold exactly ``num_tasks`` entries; with it they hold
    ``tid_size`` entries, the extra ones zero.  CUDA/HIP inputs are processed
    by the library's device kernel (``allow_triton`` is accepted for
    compatibility and has no effect); ``num_tasks`` is read back to the host.
    """
    torch = _torch()
    if not torch.is_tensor(group_sizes):
        raise TypeError("group_sizes must be a torch.Tensor")
    if group_sizes.ndim != 1:
        raise ValueError(f"group_sizes must be 1D; got shape {tuple(group_sizes.shape)}")
    if not _is_integer_dtype(torch, group_sizes.dtype):
        raise ValueError(f"group_sizes must have integer dtype; got {group_sizes.dtype}")
    if tile <= 0:
        raise ValueError("tile must be positive")
    if align_tile <= 0:
        raise ValueError("align_tile must be positive")
    if tile % align_tile != 0:
        raise ValueError("tile must be a multiple of align_tile")
    if tid_size is not None and tid_size < 0:
        raise ValueError("tid_size must be non-negative")
    sizes = torch.clamp(group_sizes.to(torch.int64), min=0)
    if not sizes.is_cuda:
        return _host_group_info(torch, sizes, tile, align_tile, tid_size)

    from .native import ragged_group_info_device, ragged_task_capacity

    groups = int(sizes.shape[0])
    rows_bound = int(sizes.sum().item()) if groups else 0
    bound = ragged_task_capacity(rows_bound, groups, tile, align_tile)
    capacity = max(bound, tid_size or 0)
    _, num, info = ragged_group_info_device(sizes.to(torch.int32).contiguous(), tile=tile, align_tile=align_tile,
                                            capacity=capacity, with_info=True)
    num_tasks = int(num.item())
    cap = num_tasks if tid_size is None else tid_size
    if cap < num_tasks:
        raise ValueError(f"tid_size must be at least {num_tasks}; got {cap}")
    fields = [info[i, :cap] for i in range(6)]
    return RaggedGroupInfo(*fields, num_tasks=num_tasks)


# ---------------------------------------------------------------------------
# Even-K eligibility (ragged.py:326-366): which K masks a launch needs.


def _can_use_even_k_fast_path(*, logical_k: int, scale: ScaleSpec, config: RaggedDotConfig) -> bool:
    if not config.enable_even_k_fast_path:
        return False
    if logical_k % config.block_k != 0:
        return False
    if scale.mode is ScaleMode.SUBCHANNEL:
        sub = scale.subchannel_size or 0
        if logical_k % sub != 0:
            return False
        if sub % config.block_k != 0 and config.block_k % sub != 0:
            return False
    return True


def _can_use_bwd_even_k_fast_path(torch: Any, *, group_sizes: Any, scale: ScaleSpec,
                                  config: RaggedBwdDotConfig) -> bool:
    if not config.enable_even_k_fast_path:
        return False
    sizes = group_sizes.detach().cpu()
    positive = sizes[sizes > 0]
    if int(positive.numel()) == 0:
        return True
    if bool((positive % config.block_k != 0).any()):
        return False
    if scale.mode is ScaleMode.SUBCHANNEL:
        sub = scale.subchannel_size or 0
        if sub <= 0 or bool((positive % sub != 0).any()):
            return False
        if sub % config.block_k != 0 and config.block_k % sub != 0:
            return False
    return True


# ---------------------------------------------------------------------------
# Validation (ragged.py:834-1005)


def _require_cuda_tensor(torch: Any, name: str, tensor: Any) -> None:
    if not torch.is_tensor(tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a CUDA/HIP tensor")


def _require_bfloat16_scale(torch: Any, name: str, tensor: Any | None) -> None:
    if tensor is not None and tensor.dtype != torch.bfloat16:
        raise ValueError(f"{name} must have dtype torch.bfloat16; got {tensor.dtype}")


def _check_group_sizes_tensor(torch: Any, group_sizes: Any, groups: int, what: str) -> Any:
    if not torch.is_tensor(group_sizes):
        raise TypeError("group_sizes must be a torch.Tensor")
    if group_sizes.ndim != 1:
        raise ValueError(f"group_sizes must be 1D; got shape {tuple(group_sizes.shape)}")
    if int(group_sizes.shape[0]) != groups:
        raise ValueError(f"group_sizes length must match {what} {groups}; got {int(group_sizes.shape[0])}")
    if not _is_integer_dtype(torch, group_sizes.dtype):
        raise ValueError(f"group_sizes must have integer dtype; got {group_sizes.dtype}")
    host = group_sizes.detach().cpu()
    if bool((host < 0).any()):
        raise ValueError("group_sizes must be non-negative")
    return host


def _validate_group_sizes(torch: Any, group_sizes: Any, *, groups: int, rows: int) -> None:
    host = _check_group_sizes_tensor(torch, group_sizes, groups, "rhs groups")
    total = int(host.sum().item())
    if total != rows:
        raise ValueError(f"sum(group_sizes) must equal lhs rows {rows}; got {total}")


def _validate_k_group_sizes(torch: Any, group_sizes: Any, *, groups: int, max_k: int) -> Any:
    host = _check_group_sizes_tensor(torch, group_sizes, groups, "operand groups")
    largest = int(host.max().item()) if groups else 0
    if largest > max_k:
        raise ValueError(f"group_sizes entries must be <= logical padded K {max_k}; got {largest}")
    return host


def _validate_scale_shapes(*, a_scale, b_scale, scale: ScaleSpec, groups: int, rows: int, cols: int,
                           scale_cols: int) -> None:
    if scale.mode is ScaleMode.PER_CHANNEL:
        if a_scale is not None and tuple(a_scale.shape) != (rows,):
            raise ValueError(f"a_scale must have shape ({rows},); got {tuple(a_scale.shape)}")
        if b_scale is not None and tuple(b_scale.shape) != (groups, cols):
            raise ValueError(f"b_scale must have shape ({groups}, {cols}); got {tuple(b_scale.shape)}")
        return
    if a_scale is not None and tuple(a_scale.shape) != (rows, scale_cols):
        raise ValueError(f"a_scale must have shape ({rows}, {scale_cols}); got {tuple(a_scale.shape)}")
    if b_scale is not None and tuple(b_scale.shape) != (groups, scale_cols, cols):
        raise ValueError(
            "subchannel b_scale must use weight-matched layout "
            f"({groups}, {scale_cols}, {cols}) == (groups, scale_cols, N); got {tuple(b_scale.shape)}. "
            "If you have logical layout "
            f"({groups}, {cols}, {scale_cols}) == (groups, N, scale_cols), "
            "call pack_ragged_rhs_subchannel_scales(...) first."
        )


def _validate_bwd_scale_shapes(*, a_scale, b_scale, scale: ScaleSpec, groups: int, rows: int, cols: int,
                               scale_cols: int) -> None:
    if scale.mode is ScaleMode.PER_CHANNEL:
        if a_scale is not None and tuple(a_scale.shape) != (groups, rows):
            raise ValueError(f"a_scale must have shape ({groups}, {rows}); got {tuple(a_scale.shape)}")
        if b_scale is not None and tuple(b_scale.shape) != (groups, cols):
            raise ValueError(f"b_scale must have shape ({groups}, {cols}); got {tuple(b_scale.shape)}")
        return
    if a_scale is not None and tuple(a_scale.shape) != (groups, rows, scale_cols):
        raise ValueError(f"a_scale must have shape ({groups}, {rows}, {scale_cols}); got {tuple(a_scale.shape)}")
    if b_scale is not None and tuple(b_scale.shape) != (groups, scale_cols, cols):
        raise ValueError(
            "subchannel b_scale must use weight-matched layout "
            f"({groups}, {scale_cols}, {cols}) == (groups, scale_cols, N); got {tuple(b_scale.shape)}"
        )


def _forward_logical_shape(lhs: Any, rhs: Any, layout: GemmLayout) -> tuple[int, int, int, int]:
    """(rows, cols, K_PACKED, groups) of a forward call (ragged.py:910-939)."""
    lhs_t = layout in {GemmLayout.TN, GemmLayout.TT}
    rhs_t = layout in {GemmLayout.NT, GemmLayout.TT}
    rows, k_packed = (int(lhs.shape[1]), int(lhs.shape[0])) if lhs_t else (int(lhs.shape[0]), int(lhs.shape[1]))
    groups = int(rhs.shape[0])
    cols, rhs_k = (int(rhs.shape[1]), int(rhs.shape[2])) if rhs_t else (int(rhs.shape[2]), int(rhs.shape[1]))
    if rhs_k != k_packed:
        raise ValueError(f"lhs and rhs packed K mismatch for layout={layout.value}: {k_packed} vs {rhs_k}")
    return rows, cols, k_packed, groups


def _bwd_logical_shape(lhs: Any, rhs: Any, layout: GemmLayout) -> tuple[int, int, int, int]:
    """(rows, cols, K_PACKED, groups) of a backward call (ragged.py:942-977)."""
    lhs_t = layout in {GemmLayout.TN, GemmLayout.TT}
    rhs_t = layout in {GemmLayout.NT, GemmLayout.TT}
    groups = int(lhs.shape[0])
    rows, k_packed = (int(lhs.shape[2]), int(lhs.shape[1])) if lhs_t else (int(lhs.shape[1]), int(lhs.shape[2]))
    rhs_groups = int(rhs.shape[0])
    cols, rhs_k = (int(rhs.shape[1]), int(rhs.shape[2])) if rhs_t else (int(rhs.shape[2]), int(rhs.shape[1]))
    if rhs_groups != groups:
        raise ValueError(f"lhs and rhs group mismatch for layout={layout.value}: {groups} vs {rhs_groups}")
    if rhs_k != k_packed:
        raise ValueError(f"lhs and rhs packed K mismatch for layout={layout.value}: {k_packed} vs {rhs_k}")
    return rows, cols, k_packed, groups


def _check_packed_operands(torch: Any, lhs: Any, rhs: Any, *, lhs_ndim: int) -> None:
    _require_cuda_tensor(torch, "lhs", lhs)
    _require_cuda_tensor(torch, "rhs", rhs)
    if lhs.dtype != torch.uint8:
        raise ValueError(f"lhs must be packed int4 torch.uint8; got {lhs.dtype}")
    if rhs.dtype != torch.uint8:
        raise ValueError(f"rhs must be packed int4 torch.uint8; got {rhs.dtype}")
    if lhs.ndim != lhs_ndim:
        if lhs_ndim == 2:
            raise ValueError(f"lhs must have shape (M, K/2); got {tuple(lhs.shape)}")
        raise ValueError(f"lhs must be a grouped packed tensor; got shape {tuple(lhs.shape)}")
    if rhs.ndim != 3:
        if lhs_ndim == 2:
            raise ValueError(f"rhs must have shape (G, K/2, N); got {tuple(rhs.shape)}")
        raise ValueError(f"rhs must be a grouped packed tensor; got shape {tuple(rhs.shape)}")
    if not lhs.is_contiguous():
        raise ValueError("lhs must be contiguous")
    if not rhs.is_contiguous():
        raise ValueError("rhs must be contiguous")


def _scales_or_ones(torch, a_scale, b_scale, a_shape, b_shape, device):
    if a_scale is None:
        a_scale = torch.ones(a_shape, device=device, dtype=torch.bfloat16)
    if b_scale is None:
        b_scale = torch.ones(b_shape, device=device, dtype=torch.bfloat16)
    return a_scale, b_scale


def _aligned(tensor: Any, nbytes: int) -> bool:
    return tensor.data_ptr() % nbytes == 0


def _fp6_buffers_ok(out: Any, b_scale: Any) -> bool:
    """Buffer alignment the fp6 ragged kernels need (k_f6ragged.hip)."""
    return _aligned(out, 16) and _aligned(b_scale, 8)


def _reject_jit(use_native: bool | None) -> None:
    if use_native is False:
        raise ValueError("use_native=False requests the Triton JIT path, which this gfx950 build does not have")


# ---------------------------------------------------------------------------
# Entry points


def ragged_dot_int4(
    lhs: Any,
    rhs: Any,
    group_sizes: Any,
    *,
    a_scale: Any | None = None,
    b_scale: Any | None = None,
    scale: ScaleSpec = ScaleSpec(ScaleMode.PER_CHANNEL),
    config: RaggedDotConfig = RaggedDotConfig(),
    layout: GemmLayout = GemmLayout.NN,
    out: Any | None = None,
    output_dtype: Any | None = None,
    use_native: bool | None = None,
    native_root: str | None = None,
    native_library_path: str | None = None,
) -> Any:
    """Forward grouped ragged int4 dot (ragged.py:1008-1229).

    NN: ``lhs[M, K/2]``, ``rhs[G, K/2, N]``; NT: ``rhs[G, N, K/2]``;
    TN: ``lhs[K/2, M]``; TT: both.  ``group_sizes[G]`` assigns contiguous row
    groups of ``lhs`` to experts; the output is ``(M, N)`` in bf16 (default)
    or fp32.  Scales: per-channel ``a_scale[M]``, ``b_scale[G, N]``;
    subchannel S ``a_scale[M, ceil(K/S)]``, ``b_scale[G, ceil(K/S), N]``.
    """
    layout = _check_layout(layout)
    torch = _torch()
    _reject_jit(use_native)
    _check_packed_operands(torch, lhs, rhs, lhs_ndim=2)
    rows, cols, k_packed, groups = _forward_logical_shape(lhs, rhs, layout)
    _validate_group_sizes(torch, group_sizes, groups=groups, rows=rows)
    _require_bfloat16_scale(torch, "a_scale", a_scale)
    _require_bfloat16_scale(torch, "b_scale", b_scale)
    if a_scale is not None:
        _require_cuda_tensor(torch, "a_scale", a_scale)
    if b_scale is not None:
        _require_cuda_tensor(torch, "b_scale", b_scale)
    subchannel = None
    logical_k = 2 * k_packed
    scale_cols = 1
    if scale.mode is ScaleMode.SUBCHANNEL:
        subchannel = scale.subchannel_size or 0
        if subchannel % 2 != 0:
            raise ValueError("subchannel_size must be even for packed int4 operands")
        scale_cols = _cdiv(logical_k, subchannel)
    _validate_scale_shapes(a_scale=a_scale, b_scale=b_scale, scale=scale, groups=groups, rows=rows, cols=cols,
                           scale_cols=scale_cols)
    if a_scale is not None and not a_scale.is_contiguous():
        raise ValueError("a_scale must be contiguous")
    if b_scale is not None and not b_scale.is_contiguous():
        raise ValueError("b_scale must be contiguous")
    if output_dtype is None:
        output_dtype = torch.bfloat16
    if output_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"output_dtype must be torch.bfloat16 or torch.float32; got {output_dtype}")
    if out is None:
        out = torch.empty((rows, cols), device=lhs.device, dtype=output_dtype)
    else:
        _require_cuda_tensor(torch, "out", out)
        if tuple(out.shape) != (rows, cols):
            raise ValueError(f"out must have shape ({rows}, {cols}); got {tuple(out.shape)}")
        if out.dtype != output_dtype:
            raise ValueError(f"out dtype {out.dtype} does not match output_dtype {output_dtype}")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")
    if rows == 0 or cols == 0 or groups == 0:
        return out
    a_shape = (rows,) if subchannel is None else (rows, scale_cols)
    b_shape = (groups, cols) if subchannel is None else (groups, scale_cols, cols)
    a_scale, b_scale = _scales_or_ones(torch, a_scale, b_scale, a_shape, b_shape, lhs.device)
    fp6 = (config.block_m in (64, kt.RAGGED_FP6_CONFIG_BLOCK_M)
            and kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_FWD, subchannel=subchannel, m=rows, n=cols, k_packed=k_packed)
           and _fp6_buffers_ok(out, b_scale))
    if fp6:
        block_m, align = kt.RAGGED_FP6_BLOCK_M, kt.RAGGED_FP6_ALIGN
    else:
        block_m = config.block_m if config.block_m in kt.RAGGED_FWD_BLOCK_M else 64
        align = config.align_tile if block_m % config.align_tile == 0 else 8
    from .native import launch_ragged_fwd

    gs = group_sizes.to(device=lhs.device, dtype=torch.int32).contiguous()
    return launch_ragged_fwd(
        lhs, rhs, gs, a_scale=a_scale, b_scale=b_scale, out=out, layout=layout, subchannel=subchannel,
        block_m=block_m, align_tile=align, rows=rows, cols=cols, k_packed=k_packed,
        out_mode=kt.OUT_BF16 if output_dtype == torch.bfloat16 else kt.OUT_F32, fp6=fp6,
        library_path=native_library_path if native_library_path is not None else (
            None if native_root is None else f"{native_root}/libamd_strix_halo_kernels_gfx950.so"),
    )


def ragged_dot_int4_bwd(
    lhs: Any,
    rhs: Any,
    group_sizes: Any,
    *,
    a_scale: Any | None = None,
    b_scale: Any | None = None,
    scale: ScaleSpec = ScaleSpec(ScaleMode.PER_CHANNEL),
    config: RaggedBwdDotConfig = RaggedBwdDotConfig(),
    layout: GemmLayout = GemmLayout.NN,
    out: Any | None = None,
    use_native: bool | None = None,
    native_root: str | None = None,
    native_library_path: str | None = None,
) -> Any:
    """Grouped K-ragged dot for backward reductions (ragged.py:1232-1402).

    ``out[g] = op(lhs[g]) @ op(rhs[g])`` over the first ``group_sizes[g]``
    logical K values; K beyond it (operand padding, which may hold anything)
    reads as zero.  NN: ``lhs[G, M, K/2]``, ``rhs[G, K/2, N]``; NT:
    ``rhs[G, N, K/2]``; TN: ``lhs[G, K/2, M]``; TT: both.  Output fp32
    ``(G, M, N)``.
    """
    layout = _check_layout(layout)
    torch = _torch()
    _reject_jit(use_native)
    _check_packed_operands(torch, lhs, rhs, lhs_ndim=3)
    rows, cols, k_packed, groups = _bwd_logical_shape(lhs, rhs, layout)
    k_capacity = 2 * k_packed
    _validate_k_group_sizes(torch, group_sizes, groups=groups, max_k=k_capacity)
    _require_bfloat16_scale(torch, "a_scale", a_scale)
    _require_bfloat16_scale(torch, "b_scale", b_scale)
    if a_scale is not None:
        _require_cuda_tensor(torch, "a_scale", a_scale)
    if b_scale is not None:
        _require_cuda_tensor(torch, "b_scale", b_scale)
    subchannel = None
    scale_cols = 1
    if scale.mode is ScaleMode.SUBCHANNEL:
        subchannel = scale.subchannel_size or 0
        if subchannel % 2 != 0:
            raise ValueError("subchannel_size must be even for packed int4 operands")
        scale_cols = _cdiv(k_capacity, subchannel)
    _validate_bwd_scale_shapes(a_scale=a_scale, b_scale=b_scale, scale=scale, groups=groups, rows=rows, cols=cols,
                               scale_cols=scale_cols)
    if a_scale is not None and not a_scale.is_contiguous():
        raise ValueError("a_scale must be contiguous")
    if b_scale is not None and not b_scale.is_contiguous():
        raise ValueError("b_scale must be contiguous")
    if out is None:
        out = torch.empty((groups, rows, cols), device=lhs.device, dtype=torch.float32)
    else:
        _require_cuda_tensor(torch, "out", out)
        if tuple(out.shape) != (groups, rows, cols):
            raise ValueError(f"out must have shape ({groups}, {rows}, {cols}); got {tuple(out.shape)}")
        if out.dtype != torch.float32:
            raise ValueError(f"out dtype must be torch.float32; got {out.dtype}")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")
    if config.split_k > 1:
        out.zero_()
    if groups == 0 or rows == 0 or cols == 0:
        return out
    a_shape = (groups, rows) if subchannel is None else (groups, rows, scale_cols)
    b_shape = (groups, cols) if subchannel is None else (groups, scale_cols, cols)
    a_scale, b_scale = _scales_or_ones(torch, a_scale, b_scale, a_shape, b_shape, lhs.device)
    from .native import launch_ragged_bwd

    gs = group_sizes.to(device=lhs.device, dtype=torch.int32).contiguous()
    fp6 = (kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_BWD, subchannel=subchannel, m=rows, n=cols, k_packed=k_packed)
           and _fp6_buffers_ok(out, b_scale))
    return launch_ragged_bwd(
        lhs, rhs, gs, a_scale=a_scale, b_scale=b_scale, out=out, layout=layout, subchannel=subchannel,
        split_k=config.split_k, rows=rows, cols=cols, k_packed=k_packed, fp6=fp6,
        library_path=native_library_path if native_library_path is not None else (
            None if native_root is None else f"{native_root}/libamd_strix_halo_kernels_gfx950.so"),
    )
