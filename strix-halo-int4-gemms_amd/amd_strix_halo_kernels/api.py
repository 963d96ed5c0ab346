"""Dense quantized GEMM API: mm, fused_swiglu_up_gate, explicit_mm.

Signatures, validation order and error messages follow the reference
(api.py:30-254) so callers and their tests keep working.  Dispatch is strict:
a shape no table kernel accepts raises ``LookupError`` from the registry and a
launch failure raises; nothing falls back to a slower path.
``use_reference=True`` evaluates ``reference_mm``, the torch numerical
definition of the same call (api.py:257-325), on whatever device the inputs
are on; it is an explicit opt-in for numerical checks, never a fallback.
"""

from __future__ import annotations

from typing import Any

from .exceptions import KernelNotAvailableError
from .metadata import (
    SUPPORTED_GEMM_LAYOUTS,
    Epilogue,
    GemmLayout,
    KernelMetadata,
    KernelSchedule,
    KernelStatus,
    OperandDType,
    ScaleMode,
    ScaleSpec,
)
from .native import launch_generated_kernel
from .quant import unpack_int4_k_major
from .registry import KernelRegistry, default_registry


def _torch() -> Any:
    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("torch is required for GEMM APIs") from exc
    return torch


def _require_supported_layout(layout: GemmLayout) -> None:
    if layout not in SUPPORTED_GEMM_LAYOUTS:
        supported = ", ".join(item.value for item in SUPPORTED_GEMM_LAYOUTS)
        raise ValueError(f"unsupported GEMM layout {layout.value}; generated layouts are {supported}")


def _packed(dtype: OperandDType, tensor: Any) -> bool:
    return dtype is OperandDType.INT4 and str(getattr(tensor, "dtype", "")) in {"torch.uint8", "uint8"}


def _logical_problem_shape(a: Any, b: Any, *, dtype: OperandDType, layout: GemmLayout, swiglu: bool):
    """Logical (M, N, K) of a call; packed uint8 int4 operands count two K
    values per byte (api.py:44-78)."""
    _require_supported_layout(layout)
    ka_mult = 2 if _packed(dtype, a) else 1
    kb_mult = 2 if _packed(dtype, b) else 1
    if layout is GemmLayout.NN:
        m, k_a = int(a.shape[-2]), int(a.shape[-1]) * ka_mult
        b_cols, k_b = int(b.shape[-1]), int(b.shape[-2]) * kb_mult
    elif layout is GemmLayout.NT:
        m, k_a = int(a.shape[-2]), int(a.shape[-1]) * ka_mult
        b_cols, k_b = int(b.shape[-2]), int(b.shape[-1]) * kb_mult
    else:  # TN
        m, k_a = int(a.shape[-1]), int(a.shape[-2]) * ka_mult
        b_cols, k_b = int(b.shape[-1]), int(b.shape[-2]) * kb_mult
    if k_a != k_b:
        raise ValueError(f"logical K mismatch for layout={layout.value}: A has {k_a}, B has {k_b}")
    if swiglu:
        if b_cols % 2:
            raise ValueError("fused_swiglu_up_gate requires the logical B output dimension to be even")
        b_cols //= 2
    return m, b_cols, k_a


def _scale_cols(k: int, scale: ScaleSpec) -> int:
    if scale.subchannel_size is None:
        raise ValueError("subchannel scale mode requires subchannel_size")
    return -(-k // scale.subchannel_size)


def _validate_scale_shapes(*, kernel: KernelMetadata, m: int, n: int, k: int, a_scale: Any, b_scale: Any) -> None:
    """Scale shape contract (api.py:88-116); None scales are allowed here."""
    b_cols = 2 * n if kernel.epilogue is Epilogue.SWIGLU else n
    if kernel.scale.mode is ScaleMode.PER_CHANNEL:
        if a_scale is not None and tuple(a_scale.shape) != (m,):
            raise ValueError(f"a_scale must have shape ({m},); got {tuple(a_scale.shape)}")
        if b_scale is not None and tuple(b_scale.shape) != (b_cols,):
            raise ValueError(f"b_scale must have shape ({b_cols},); got {tuple(b_scale.shape)}")
        return
    cols = _scale_cols(k, kernel.scale)
    if a_scale is not None and tuple(a_scale.shape) != (m, cols):
        raise ValueError(f"a_scale must have shape ({m}, {cols}); got {tuple(a_scale.shape)}")
    if b_scale is not None and tuple(b_scale.shape) != (cols, b_cols):
        raise ValueError(
            "subchannel b_scale must use weight-matched layout "
            f"{(cols, b_cols)} == (scale_cols, output_cols); got {tuple(b_scale.shape)}. "
            f"If you have logical layout {(b_cols, cols)} == (output_cols, scale_cols), "
            "call pack_rhs_subchannel_scales(...) first."
        )


def mm(
    a: Any,
    b: Any,
    *,
    a_scale: Any | None = None,
    b_scale: Any | None = None,
    gate: Any | None = None,
    dtype: OperandDType = OperandDType.INT4,
    layout: GemmLayout = GemmLayout.NN,
    scale: ScaleSpec = ScaleSpec(ScaleMode.PER_CHANNEL),
    epilogue: Epilogue = Epilogue.NONE,
    schedule: KernelSchedule = KernelSchedule.STANDARD,
    registry: KernelRegistry = default_registry,
    use_reference: bool = False,
) -> Any:
    """Selects and launches the gfx950 dense kernel for this call (api.py:119-164).

    Incompatible shapes raise instead of falling back.  ``use_reference=True``
    evaluates the torch numerical definition instead (numerical checks only).
    """
    if epilogue is Epilogue.SWIGLU:
        raise ValueError("SwiGLU is exposed through fused_swiglu_up_gate(...), not mm(...)")
    _require_supported_layout(layout)
    m, n, k = _logical_problem_shape(a, b, dtype=dtype, layout=layout, swiglu=False)
    if use_reference:
        kernel = registry.select_reference(dtype=dtype, layout=layout, scale=scale, epilogue=epilogue,
                                           schedule=schedule)
    else:
        kernel = registry.select(dtype=dtype, layout=layout, scale=scale, epilogue=epilogue, m=m, n=n, k=k,
                                 schedule=schedule)
    return explicit_mm(a, b, kernel=kernel, a_scale=a_scale, b_scale=b_scale, gate=gate,
                       use_reference=use_reference)


def fused_swiglu_up_gate(
    a: Any,
    b_up_gate: Any,
    *,
    a_scale: Any | None = None,
    b_scale: Any | None = None,
    dtype: OperandDType = OperandDType.INT4,
    layout: GemmLayout = GemmLayout.NN,
    scale: ScaleSpec = ScaleSpec(ScaleMode.PER_CHANNEL),
    registry: KernelRegistry = default_registry,
    use_reference: bool = False,
) -> Any:
    """Fused up/gate SwiGLU GEMM (api.py:167-214).

    ``b_up_gate`` holds ``[up | gate]`` along the output dimension (2D
    columns); the result is ``up * silu(gate)`` with D columns.
    """
    _require_supported_layout(layout)
    m, n, k = _logical_problem_shape(a, b_up_gate, dtype=dtype, layout=layout, swiglu=True)
    if use_reference:
        kernel = registry.select_reference(dtype=dtype, layout=layout, scale=scale, epilogue=Epilogue.SWIGLU,
                                           split_k=1)
    else:
        kernel = registry.select(dtype=dtype, layout=layout, scale=scale, epilogue=Epilogue.SWIGLU, m=m, n=n,
                                 k=k, split_k=1)
    return explicit_mm(a, b_up_gate, kernel=kernel, a_scale=a_scale, b_scale=b_scale, use_reference=use_reference)


def explicit_mm(
    a: Any,
    b: Any,
    *,
    kernel: KernelMetadata,
    a_scale: Any | None = None,
    b_scale: Any | None = None,
    gate: Any | None = None,
    use_reference: bool = False,
) -> Any:
    """Launches a caller-selected kernel (api.py:217-254)."""
    _require_supported_layout(kernel.layout)
    if kernel.epilogue is Epilogue.SWIGLU and gate is not None:
        raise ValueError("SwiGLU kernels use fused up/gate columns; pass gate through b_up_gate")
    m, n, k = _logical_problem_shape(a, b, dtype=kernel.a_dtype, layout=kernel.layout,
                                     swiglu=kernel.epilogue is Epilogue.SWIGLU)
    _validate_scale_shapes(kernel=kernel, m=m, n=n, k=k, a_scale=a_scale, b_scale=b_scale)
    if use_reference:
        return reference_mm(a, b, kernel=kernel, a_scale=a_scale, b_scale=b_scale, gate=gate)
    if kernel.status not in {KernelStatus.COMPILED, KernelStatus.BENCHMARKED}:
        try:
            return launch_generated_kernel(a, b, kernel=kernel, a_scale=a_scale, b_scale=b_scale, gate=gate)
        except Exception as exc:
            raise KernelNotAvailableError(
                f"{kernel.kernel_id} is {kernel.status.value}; native generated dispatch is unavailable: {exc}"
            ) from exc
    return launch_generated_kernel(a, b, kernel=kernel, a_scale=a_scale, b_scale=b_scale, gate=gate)


def reference_mm(a: Any, b: Any, *, kernel: KernelMetadata, a_scale: Any | None, b_scale: Any | None,
                 gate: Any | None = None) -> Any:
    """Torch numerical definition of a dense call (api.py:257-296): unpack per
    layout, exact int32 matmul, fp32 scaling in the kernel's order, epilogue,
    cast."""
    torch = _torch()
    a_t = kernel.layout in {GemmLayout.TN, GemmLayout.TT}
    b_t = kernel.layout in {GemmLayout.NT, GemmLayout.TT}
    if kernel.a_dtype is OperandDType.INT4:
        if a.dtype is torch.uint8:
            a = unpack_int4_k_major(a.transpose(-2, -1)).transpose(-2, -1) if a_t else unpack_int4_k_major(a)
        if b.dtype is torch.uint8:
            b = unpack_int4_k_major(b) if b_t else unpack_int4_k_major(b.transpose(-2, -1)).transpose(-2, -1)
    if a_t:
        a = a.transpose(-2, -1)
    if b_t:
        b = b.transpose(-2, -1)
    out = _scaled_reference_mm(a, b, kernel=kernel, a_scale=a_scale, b_scale=b_scale)
    if kernel.epilogue is Epilogue.SWIGLU:
        if gate is not None:
            raise ValueError("SwiGLU reference uses fused up/gate columns; external gate is not supported")
        if out.shape[-1] % 2:
            raise ValueError("fused SwiGLU reference requires an even output dimension")
        up, g = out.split(out.shape[-1] // 2, dim=-1)
        out = up * (g / (1.0 + torch.exp(-g)))
    elif kernel.epilogue is Epilogue.RELU2:
        out = torch.relu(out).square()
    if kernel.output_dtype == "bfloat16":
        return out.to(torch.bfloat16)
    if kernel.output_dtype == "float32":
        return out
    raise ValueError(f"unsupported kernel output dtype: {kernel.output_dtype}")


def _scaled_reference_mm(a: Any, b: Any, *, kernel: KernelMetadata, a_scale: Any | None, b_scale: Any | None):
    torch = _torch()
    ai = a.to(torch.int32)
    bi = b.to(torch.int32)
    sa = None if a_scale is None else a_scale.to(torch.float32)
    sb = None if b_scale is None else b_scale.to(torch.float32)
    if kernel.scale.mode is ScaleMode.PER_CHANNEL:
        out = torch.matmul(ai, bi).to(torch.float32)
        if sa is not None:
            out = out * sa[..., :, None]
        if sb is not None:
            out = out * sb[..., None, :]
        return out
    sub = kernel.scale.subchannel_size
    if sub is None:
        raise ValueError("subchannel scale mode requires subchannel_size")
    k = int(ai.shape[-1])
    out = torch.zeros((*ai.shape[:-1], bi.shape[-1]), device=ai.device, dtype=torch.float32)
    for g, k0 in enumerate(range(0, k, sub)):
        k1 = min(k0 + sub, k)
        part = torch.matmul(ai[..., k0:k1], bi[..., k0:k1, :]).to(torch.float32)
        if sa is not None:
            part = part * sa[..., :, g, None]
        if sb is not None:
            part = part * sb[..., g, :][..., None, :]
        out += part
    return out
