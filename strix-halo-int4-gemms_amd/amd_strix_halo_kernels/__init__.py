"""MI355X (gfx950) quantized GEMM kernels with the amd_strix_halo_kernels API.

Drop-in replacement for the hot path of the reference package: ``mm``,
``fused_swiglu_up_gate``, ``explicit_mm``, ``ragged_dot_int4``,
``ragged_dot_int4_bwd`` and ``calculate_group_info`` with the same arguments,
packed int4 format, scale layouts and errors, running hand-written HIP
kernels for CDNA4 from libamd_strix_halo_kernels_gfx950.so.
"""

from .api import explicit_mm, fused_swiglu_up_gate, mm, reference_mm
from .benchmarking import gemm_ops, tops_for_runtime
from .exceptions import KernelError, KernelNotAvailableError
from .metadata import (
    ACC_DTYPE,
    ARCH,
    RHS_SUBCHANNEL_SCALE_LAYOUT,
    SCALE_DTYPE_BF16,
    SUPPORTED_GEMM_LAYOUTS,
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
)
from .native import (
    NativeRuntimeStatus,
    dispatch_runtime_status,
    launch_generated_kernel,
    native_library_path,
)
from .quant import (
    fake_quant_int,
    pack_int4_k_major,
    pack_ragged_rhs_subchannel_scales,
    pack_rhs_subchannel_scales,
    quantize_pack_int4,
    unpack_int4_k_major,
)
from .ragged import (
    RaggedBwdDotConfig,
    RaggedDotConfig,
    RaggedGroupInfo,
    calculate_group_info,
    ragged_dot_int4,
    ragged_dot_int4_bwd,
)
from .registry import KernelRegistry, default_registry
from .torch_ops import TORCH_GEMM_OP, TORCH_OP_NAMESPACE, register_torch_ops, torch_gemm

__all__ = [
    "ACC_DTYPE",
    "ARCH",
    "Epilogue",
    "GemmLayout",
    "KernelError",
    "KernelMetadata",
    "KernelNotAvailableError",
    "KernelRegistry",
    "KernelSchedule",
    "KernelStatus",
    "NativeRuntimeStatus",
    "OperandDType",
    "RHS_SUBCHANNEL_SCALE_LAYOUT",
    "RaggedBwdDotConfig",
    "RaggedDotConfig",
    "RaggedGroupInfo",
    "SCALE_DTYPE_BF16",
    "SUPPORTED_GEMM_LAYOUTS",
    "SUPPORTED_SUBCHANNELS",
    "ScaleMode",
    "ScaleSpec",
    "TORCH_GEMM_OP",
    "TORCH_OP_NAMESPACE",
    "TileConfig",
    "calculate_group_info",
    "default_registry",
    "dispatch_runtime_status",
    "explicit_mm",
    "fake_quant_int",
    "fused_swiglu_up_gate",
    "gemm_ops",
    "launch_generated_kernel",
    "mm",
    "native_library_path",
    "pack_int4_k_major",
    "pack_ragged_rhs_subchannel_scales",
    "pack_rhs_subchannel_scales",
    "quantize_pack_int4",
    "ragged_dot_int4",
    "ragged_dot_int4_bwd",
    "reference_mm",
    "register_torch_ops",
    "tops_for_runtime",
    "torch_gemm",
    "unpack_int4_k_major",
]
