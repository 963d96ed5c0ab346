"""PyTorch custom-op integration around an explicit dense kernel.

Mirrors the reference's torch_ops.py:1-87: ``register_torch_ops()`` defines
``amd_strix_halo_kernels::gemm`` with the same schema, and ``torch_gemm``
calls it for a chosen ``KernelMetadata``.  The CUDA implementation launches
the gfx950 table kernel (``launch_generated_kernel``); the fake
implementation returns an empty tensor of the output's shape and dtype, so
the op traces under FakeTensorMode and torch.compile without running.  As in
the reference, no autograd formula is registered.

The output shape comes from the kernel's logical problem shape, so the fake
tensor is right for every layout (NN, NT, TN) and for SwiGLU, whose output has
half of B's logical columns.
"""

from __future__ import annotations

from typing import Any

from .metadata import KernelMetadata
from .native import _logical_problem_shape, _output_torch_dtype, launch_generated_kernel
from .registry import default_registry

TORCH_OP_NAMESPACE = "amd_strix_halo_kernels"
TORCH_GEMM_OP = f"{TORCH_OP_NAMESPACE}::gemm"
_GEMM_SCHEMA = "(Tensor a, Tensor b, Tensor a_scale, Tensor b_scale, Tensor gate, str kernel_id, bool has_gate) -> Tensor"

_REGISTERED = False


def _torch() -> Any:
    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("torch is required to register amd_strix_halo_kernels custom ops") from exc
    return torch


def register_torch_ops() -> None:
    """Defines ``amd_strix_halo_kernels::gemm`` once per process (torch_ops.py:24-74)."""
    global _REGISTERED
    if _REGISTERED:
        return
    torch = _torch()

    @torch.library.custom_op(TORCH_GEMM_OP, mutates_args=(), device_types="cuda", schema=_GEMM_SCHEMA)
    def gemm(a, b, a_scale, b_scale, gate, kernel_id, has_gate):
        kernel = default_registry.get(kernel_id)
        return launch_generated_kernel(a, b, kernel=kernel, a_scale=a_scale, b_scale=b_scale,
                                       gate=gate if has_gate else None)

    @gemm.register_fake
    def _(a, b, a_scale, b_scale, gate, kernel_id, has_gate):
        del a_scale, b_scale, gate, has_gate
        kernel = default_registry.get(kernel_id)
        m, n, _ = _logical_problem_shape(kernel, a, b)
        return a.new_empty((m, n), dtype=_output_torch_dtype(torch, kernel))

    _REGISTERED = True


def torch_gemm(a: Any, b: Any, *, kernel: KernelMetadata, a_scale: Any, b_scale: Any, gate: Any | None = None) -> Any:
    """``explicit_mm`` through the registered custom op (torch_ops.py:77-87)."""
    torch = _torch()
    register_torch_ops()
    gate_arg = gate if gate is not None else torch.empty((0,), device=a.device, dtype=torch.float32)
    return torch.ops.amd_strix_halo_kernels.gemm(a, b, a_scale, b_scale, gate_arg, kernel.kernel_id, gate is not None)
