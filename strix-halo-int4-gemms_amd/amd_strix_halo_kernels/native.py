"""ctypes bridge to the gfx950 kernel library (libamd_strix_halo_kernels_gfx950.so).

Replaces the reference's HSACO bridge (native.py:54-767).  Differences that
matter to callers:

* kernels are compiled into the library and addressed by kernel-table index;
  the library derives grid, block and LDS size, so no JSON metadata or HSACO
  file is read at launch time;
* the library handle and the verified kernel table are cached for the process
  (the reference re-opened the library and re-read JSON on every call);
* launches go to ``torch.cuda.current_stream(device)`` as before; errors raise
  ``RuntimeError(last_error)`` as before (native.py:158-162).

There is no fallback: every launch needs the library and a gfx950 device, and
raises otherwise.
"""

from __future__ import annotations

import contextlib
import ctypes
import functools
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from . import kernel_table as kt
from .metadata import Epilogue, GemmLayout, KernelMetadata, OperandDType, ScaleMode
from .template_config import LaunchShape

NATIVE_LIBRARY_NAME = "libamd_strix_halo_kernels_gfx950.so"


@dataclass(frozen=True, slots=True)
class NativeRuntimeStatus:
    library_path: Path
    dispatch_version: int
    has_compiled_code_objects: bool
    has_hip_runtime: bool
    has_linked_kernels: bool


class _Desc(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in (
        "index", "family", "dtype_bits", "layout", "scale_mode", "min_subchannel", "max_subchannel",
        "epilogue_kind", "block_m", "block_n", "block_k", "num_waves", "num_stages", "lds_bytes",
        "group_size_m", "operand_format", "schedule", "split_k")]


@functools.lru_cache(maxsize=None)
def package_root() -> Path:
    return Path(__file__).resolve().parent


def native_library_path(*, root: str | Path | None = None) -> Path:
    return (Path(root) if root is not None else package_root()) / NATIVE_LIBRARY_NAME


_LOCK = threading.Lock()
_LIBRARIES: dict[str, ctypes.CDLL] = {}
_VERIFIED: set[str] = set()


def _declare(lib: ctypes.CDLL) -> None:
    P = ctypes.c_void_p
    I32 = ctypes.c_int32
    I = ctypes.c_int
    U = ctypes.c_size_t  # uintptr_t
    lib.amd_strix_halo_kernels_dispatch_version.restype = I
    lib.amd_strix_halo_kernels_has_compiled_code_objects.restype = I
    lib.amd_strix_halo_kernels_has_hip_runtime.restype = I
    lib.amd_strix_halo_kernels_has_linked_kernels.restype = I
    lib.amd_strix_halo_kernels_last_error.restype = ctypes.c_char_p
    lib.amd_strix_halo_kernels_arch.restype = ctypes.c_char_p
    lib.amd_strix_halo_kernels_kernel_table_size.restype = I
    lib.amd_strix_halo_kernels_kernel_table_entry.argtypes = [I, ctypes.POINTER(_Desc)]
    lib.amd_strix_halo_kernels_kernel_table_entry.restype = I
    lib.amd_strix_halo_kernels_select_dense.argtypes = [I32, I32, I32, I32, I32, I32, I32, I32, I32,
                                                        ctypes.POINTER(I32)]
    lib.amd_strix_halo_kernels_select_dense.restype = I
    lib.amd_strix_halo_kernels_launch_gemm.argtypes = [I, I, U, P, P, P, P, P, I32, I32, I32, I32, I32, I32]
    lib.amd_strix_halo_kernels_launch_gemm.restype = I
    lib.amd_strix_halo_kernels_gemm_workspace_bytes.argtypes = [I, I32, I32, I32, ctypes.POINTER(ctypes.c_uint64)]
    lib.amd_strix_halo_kernels_gemm_workspace_bytes.restype = I
    lib.amd_strix_halo_kernels_launch_gemm_ws.argtypes = [I, I, U, P, P, P, P, P, I32, I32, I32, I32, I32, I32, P,
                                                          ctypes.c_uint64]
    lib.amd_strix_halo_kernels_launch_gemm_ws.restype = I
    lib.amd_strix_halo_kernels_launch_gemm_noalloc.argtypes = [I, I, U, P, P, P, P, P, I32, I32, I32, I32, I32,
                                                               I32]
    lib.amd_strix_halo_kernels_launch_gemm_noalloc.restype = I
    lib.amd_strix_halo_kernels_gemm_convert.argtypes = [I, I, U, I32, P, I32, I32, I32, P, ctypes.c_uint64]
    lib.amd_strix_halo_kernels_gemm_convert.restype = I
    lib.amd_strix_halo_kernels_launch_gemm_converted.argtypes = [I, I, U, P, P, P, I32, I32, I32, I32, I32, P,
                                                                 ctypes.c_uint64]
    lib.amd_strix_halo_kernels_launch_gemm_converted.restype = I
    lib.amd_strix_halo_kernels_ragged_task_capacity.argtypes = [I32, I32, I32, I32]
    lib.amd_strix_halo_kernels_ragged_task_capacity.restype = I32
    lib.amd_strix_halo_kernels_ragged_group_info.argtypes = [I, U, P, I32, I32, I32, I32, P, P, P]
    lib.amd_strix_halo_kernels_ragged_group_info.restype = I
    lib.amd_strix_halo_kernels_launch_ragged_fwd.argtypes = [I, I, U, P, P, P, P, P, P, I32, P, I32, I32, I32, I32,
                                                             I32, I32]
    lib.amd_strix_halo_kernels_launch_ragged_fwd.restype = I
    lib.amd_strix_halo_kernels_launch_ragged_bwd.argtypes = [I, I, U, P, P, P, P, P, P, I32, I32, I32, I32, I32,
                                                             I32, I32]
    lib.amd_strix_halo_kernels_launch_ragged_bwd.restype = I
    lib.amd_strix_halo_kernels_ragged_workspace_bytes.argtypes = [I, I32, I32, I32, I32,
                                                                  ctypes.POINTER(ctypes.c_uint64)]
    lib.amd_strix_halo_kernels_ragged_workspace_bytes.restype = I
    lib.amd_strix_halo_kernels_launch_ragged_fwd_ws.argtypes = [I, I, U, P, P, P, P, P, P, I32, P, I32, I32, I32,
                                                                I32, I32, I32, P, ctypes.c_uint64]
    lib.amd_strix_halo_kernels_launch_ragged_fwd_ws.restype = I
    lib.amd_strix_halo_kernels_launch_ragged_fwd_grouped.argtypes = [I, I, U, P, P, P, P, P, I32, P, P, I32, P, I32,
                                                                     I32, I32, I32, I32, I32, P, ctypes.c_uint64]
    lib.amd_strix_halo_kernels_launch_ragged_fwd_grouped.restype = I
    lib.amd_strix_halo_kernels_launch_ragged_bwd_ws.argtypes = [I, I, U, P, P, P, P, P, P, I32, I32, I32, I32, I32,
                                                                I32, I32, P, ctypes.c_uint64]
    lib.amd_strix_halo_kernels_launch_ragged_bwd_ws.restype = I
    I64 = ctypes.c_int64
    lib.amd_strix_halo_kernels_quantize.argtypes = [I, U, P, I32, I64, I64, I64, ctypes.c_float, I32, I32, P, I64]
    lib.amd_strix_halo_kernels_quantize.restype = I


def load_dispatch_library(path: str | Path | None = None) -> ctypes.CDLL:
    """Loads (once per path) and returns the kernel library."""
    library_path = Path(path) if path is not None else native_library_path()
    key = str(library_path)
    with _LOCK:
        lib = _LIBRARIES.get(key)
        if lib is not None:
            return lib
        if not library_path.exists():
            raise RuntimeError(f"native dispatch library is not installed at {library_path}")
        lib = ctypes.CDLL(key)
        _declare(lib)
        _LIBRARIES[key] = lib
        return lib


def library_kernel_table(lib: ctypes.CDLL) -> tuple[kt.KernelDesc, ...]:
    out = []
    for i in range(int(lib.amd_strix_halo_kernels_kernel_table_size())):
        d = _Desc()
        if lib.amd_strix_halo_kernels_kernel_table_entry(i, ctypes.byref(d)) != 0:
            raise RuntimeError(_library_last_error(lib))
        out.append(kt.KernelDesc(**{name: int(getattr(d, name)) for name, _ in _Desc._fields_}))
    return tuple(out)


_DEFAULT_LIBRARY: list[ctypes.CDLL] = []  # the verified default library, once loaded


def _verified_library(path: str | Path | None = None) -> ctypes.CDLL:
    if path is None and _DEFAULT_LIBRARY:
        return _DEFAULT_LIBRARY[0]
    lib = load_dispatch_library(path)
    key = str(Path(path) if path is not None else native_library_path())
    if key not in _VERIFIED:
        if library_kernel_table(lib) != kt.TABLE:
            raise RuntimeError(
                f"the kernel table of {key} does not match amd_strix_halo_kernels.kernel_table; rebuild the library"
            )
        _VERIFIED.add(key)
    if path is None:
        _DEFAULT_LIBRARY[:] = [lib]
    return lib


def dispatch_runtime_status(path: str | Path | None = None) -> NativeRuntimeStatus:
    library_path = Path(path) if path is not None else native_library_path()
    lib = load_dispatch_library(library_path)
    return NativeRuntimeStatus(
        library_path=library_path,
        dispatch_version=int(lib.amd_strix_halo_kernels_dispatch_version()),
        has_compiled_code_objects=bool(lib.amd_strix_halo_kernels_has_compiled_code_objects()),
        has_hip_runtime=bool(lib.amd_strix_halo_kernels_has_hip_runtime()),
        has_linked_kernels=bool(lib.amd_strix_halo_kernels_has_linked_kernels()),
    )


def _library_last_error(lib: ctypes.CDLL) -> str:
    err = lib.amd_strix_halo_kernels_last_error()
    if not err:
        return "unknown native dispatcher error"
    return err.decode("utf-8", errors="replace")


def _check(lib: ctypes.CDLL, rc: int) -> None:
    if rc != 0:
        raise RuntimeError(_library_last_error(lib))


def _torch() -> Any:
    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("torch is required for native kernel dispatch") from exc
    return torch


def _stream_handle(torch: Any, tensor: Any, stream: Any | None) -> int:
    if stream is not None:
        return int(stream.cuda_stream)
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:  # the handle alone, without building a Stream object per call
        return int(raw(_device_index(tensor)))
    return int(torch.cuda.current_stream(tensor.device).cuda_stream)


def _device_index(tensor: Any) -> int:
    index = tensor.device.index
    return 0 if index is None else int(index)


def _require_contiguous(name: str, tensor: Any) -> Any:
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous for native dispatch")
    return tensor


def _require_bfloat16_scale(torch: Any, name: str, tensor: Any) -> Any:
    if tensor.dtype != torch.bfloat16:
        raise ValueError(f"{name} must have dtype torch.bfloat16 for native dispatch; got {tensor.dtype}")
    return tensor


def _require_device(torch: Any, tensors: dict[str, Any]) -> None:
    first = None
    for name, t in tensors.items():
        if t is None:
            continue
        if not getattr(t, "is_cuda", False):
            if not torch.cuda.is_available():
                raise RuntimeError("native generated kernels require a CUDA/HIP torch device")
            raise RuntimeError(f"native generated kernels require CUDA/HIP tensors; {name} is on {t.device}")
        if first is None:
            first = t.device
        elif t.device != first:
            raise ValueError(f"{name} is on {t.device}, expected {first}")


def _k_dim(size: int, *, packed_int4: bool) -> int:
    return size * 2 if packed_int4 else size


def _logical_problem_shape(kernel: KernelMetadata, a: Any, b: Any) -> tuple[int, int, int]:
    packed = kernel.a_dtype is OperandDType.INT4
    if kernel.layout is GemmLayout.NN:
        m, k_a = int(a.shape[-2]), _k_dim(int(a.shape[-1]), packed_int4=packed)
        n, k_b = int(b.shape[-1]), _k_dim(int(b.shape[-2]), packed_int4=packed)
    elif kernel.layout is GemmLayout.NT:
        m, k_a = int(a.shape[-2]), _k_dim(int(a.shape[-1]), packed_int4=packed)
        n, k_b = int(b.shape[-2]), _k_dim(int(b.shape[-1]), packed_int4=packed)
    elif kernel.layout is GemmLayout.TN:
        m, k_a = int(a.shape[-1]), _k_dim(int(a.shape[-2]), packed_int4=packed)
        n, k_b = int(b.shape[-1]), _k_dim(int(b.shape[-2]), packed_int4=packed)
    else:
        raise ValueError(f"native dispatch does not support layout={kernel.layout.value}")
    if kernel.epilogue is Epilogue.SWIGLU:
        if n % 2 != 0:
            raise ValueError("fused SwiGLU native dispatch requires the logical B output dimension to be even")
        n //= 2
    if k_a != k_b:
        raise ValueError(f"logical K mismatch for layout={kernel.layout.value}: A has {k_a}, B has {k_b}")
    return m, n, k_a


def _validate_scale_shapes(kernel: KernelMetadata, *, m: int, n: int, k: int, a_scale: Any, b_scale: Any) -> None:
    b_cols = n * 2 if kernel.epilogue is Epilogue.SWIGLU else n
    if kernel.scale.mode is ScaleMode.PER_CHANNEL:
        if tuple(a_scale.shape) != (m,):
            raise ValueError(f"a_scale must have shape ({m},) for native dispatch; got {tuple(a_scale.shape)}")
        if tuple(b_scale.shape) != (b_cols,):
            raise ValueError(f"b_scale must have shape ({b_cols},) for native dispatch; got {tuple(b_scale.shape)}")
        return
    sub = kernel.scale.subchannel_size
    scale_cols = (k + sub - 1) // sub
    if tuple(a_scale.shape) != (m, scale_cols):
        raise ValueError(
            f"a_scale must have shape ({m}, {scale_cols}) for native dispatch; got {tuple(a_scale.shape)}"
        )
    expected_b = (scale_cols, b_cols)
    if tuple(b_scale.shape) != expected_b:
        raise ValueError(
            "subchannel b_scale must use weight-matched layout "
            f"{expected_b} == (scale_cols, output_cols) for native dispatch; got {tuple(b_scale.shape)}. "
            f"If you have logical layout {(b_cols, scale_cols)} == (output_cols, scale_cols), "
            "call pack_rhs_subchannel_scales(...) first."
        )


def _output_torch_dtype(torch: Any, kernel: KernelMetadata) -> Any:
    if kernel.output_dtype == "bfloat16":
        return torch.bfloat16
    if kernel.output_dtype == "float32":
        return torch.float32
    raise ValueError(f"unsupported kernel output dtype: {kernel.output_dtype}")


def _table_index(kernel: KernelMetadata) -> int:
    if kernel.table_index is None:
        raise RuntimeError(f"{kernel.kernel_id} has no gfx950 kernel-table entry")
    return int(kernel.table_index)


_EPILOGUE_CODE = {Epilogue.NONE: kt.EPILOGUE_NONE, Epilogue.RELU2: kt.EPILOGUE_RELU2,
                  Epilogue.SWIGLU: kt.EPILOGUE_SWIGLU}


def gemm_workspace_bytes(kernel: KernelMetadata, m: int, n: int, k: int, *, library_path=None) -> int:
    """Workspace bytes the kernel's table entry needs for (m, n, k)."""
    lib = _verified_library(library_path)
    out = ctypes.c_uint64(0)
    _check(lib, lib.amd_strix_halo_kernels_gemm_workspace_bytes(_table_index(kernel), m, n, k, ctypes.byref(out)))
    return int(out.value)


_SPLIT_LOCK = threading.Lock()
_SPLIT_WORKSPACES: dict[tuple[int, int], Any] = {}


def _split_workspace(torch, device, stream_handle: int, stream, nbytes: int):
    """The workspace of the skinny (STREAM) launches on one stream of one
    device: zero-filled when allocated, on that stream, and left zero by
    every launch (counters and partials), so launches of any shape in stream
    order share it.  It grows (to a new zero-filled buffer) when a shape
    needs more."""
    key = (0 if device.index is None else int(device.index), stream_handle)
    with _SPLIT_LOCK:
        buf = _SPLIT_WORKSPACES.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 2 * buf.numel() if buf is not None else 0)
            ctx = torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()
            with ctx:
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
            _SPLIT_WORKSPACES[key] = buf
        return buf


def _gemm_call(torch, a, b, a_scale, b_scale, out, kernel, m, n, k, out_mode, library_path, stream) -> None:
    lib = _verified_library(library_path)
    sub = kernel.scale.subchannel_size if kernel.scale.mode is ScaleMode.SUBCHANNEL else 0
    # fp6 entries convert both operands into a workspace first; it comes from
    # torch's caching allocator on the launch stream, so a later launch on
    # the same stream may reuse it.  Skinny entries that split K share one
    # zero-filled workspace per stream (it must be zero where a launch uses it).
    # (the table mirror's size, which gemm_workspace_bytes matches)
    desc = kt.TABLE[_table_index(kernel)]
    ws_bytes = desc.workspace_bytes(m, n, k)
    handle = _stream_handle(torch, a, stream)
    if desc.is_stream:
        work = _split_workspace(torch, a.device, handle, stream, ws_bytes) if ws_bytes else None
        ws_bytes = work.numel() if work is not None else 0
    else:
        work = torch.empty(ws_bytes, dtype=torch.uint8, device=a.device) if ws_bytes else None
        if work is not None and stream is not None:
            work.record_stream(stream)
    rc = lib.amd_strix_halo_kernels_launch_gemm_ws(
        _table_index(kernel),
        _device_index(a),
        handle,
        a.data_ptr(),
        b.data_ptr(),
        a_scale.data_ptr(),
        b_scale.data_ptr(),
        out.data_ptr(),
        m,
        n,
        k,
        sub or 0,
        _EPILOGUE_CODE[kernel.epilogue],
        out_mode,
        work.data_ptr() if work is not None else None,
        ws_bytes,
    )
    _check(lib, rc)


def gemm_workspace(kernel: KernelMetadata, m: int, n: int, k: int, *, device: Any, library_path=None) -> Any:
    """A uint8 workspace tensor for a fp6 kernel's converted operands."""
    torch = _torch()
    return torch.empty(gemm_workspace_bytes(kernel, m, n, k, library_path=library_path), dtype=torch.uint8,
                       device=device)


def convert_operand(kernel: KernelMetadata, operand: int, src: Any, *, m: int, n: int, k: int, workspace: Any,
                    library_path=None, stream: Any | None = None) -> None:
    """Converts A (operand 0) or B (operand 1) of a fp6 kernel into its part
    of `workspace` (amd_strix_halo_kernels_gemm_convert)."""
    torch = _torch()
    lib = _verified_library(library_path)
    src = _require_contiguous("src", src)
    _require_device(torch, {"src": src, "workspace": workspace})
    rc = lib.amd_strix_halo_kernels_gemm_convert(_table_index(kernel), _device_index(src),
                                                 _stream_handle(torch, src, stream), operand, src.data_ptr(), m, n,
                                                 k, workspace.data_ptr(), workspace.numel())
    _check(lib, rc)


def launch_converted(kernel: KernelMetadata, *, m: int, n: int, k: int, workspace: Any, a_scale: Any, b_scale: Any,
                     out: Any, out_mode: int = kt.OUT_BF16, library_path=None, stream: Any | None = None) -> Any:
    """GEMM of a fp6 kernel on operands already converted into `workspace`
    (amd_strix_halo_kernels_launch_gemm_converted)."""
    torch = _torch()
    lib = _verified_library(library_path)
    _require_device(torch, {"workspace": workspace, "a_scale": a_scale, "b_scale": b_scale, "out": out})
    rc = lib.amd_strix_halo_kernels_launch_gemm_converted(
        _table_index(kernel), _device_index(out), _stream_handle(torch, out, stream), a_scale.data_ptr(),
        b_scale.data_ptr(), out.data_ptr(), m, n, k, _EPILOGUE_CODE[kernel.epilogue], out_mode,
        workspace.data_ptr(), workspace.numel())
    _check(lib, rc)
    return out


def _prepare_dense(torch, a, b, kernel, a_scale, b_scale, gate):
    _require_device(torch, {"a": a, "b": b, "a_scale": a_scale, "b_scale": b_scale})
    if a_scale is None or b_scale is None:
        raise ValueError("native generated kernels require a_scale and b_scale tensors")
    if kernel.epilogue is Epilogue.SWIGLU and gate is not None:
        raise ValueError("SwiGLU native dispatch uses fused up/gate columns; external gate is not supported")
    if kernel.epilogue in {Epilogue.RELU2, Epilogue.SWIGLU} and kernel.tile.split_k != 1:
        raise ValueError(f"{kernel.epilogue.value} native dispatch currently supports SPLIT_K=1 only")
    expected = torch.uint8 if kernel.a_dtype is OperandDType.INT4 else torch.int8
    for name, t in (("a", a), ("b", b)):
        if t.dtype != expected:
            raise ValueError(f"{name} must have dtype {expected} for {kernel.a_dtype.value} kernels; got {t.dtype}")
    a = _require_contiguous("a", a)
    b = _require_contiguous("b", b)
    a_scale = _require_bfloat16_scale(torch, "a_scale", _require_contiguous("a_scale", a_scale))
    b_scale = _require_bfloat16_scale(torch, "b_scale", _require_contiguous("b_scale", b_scale))
    m, n, k = _logical_problem_shape(kernel, a, b)
    LaunchShape(m, n, k).validate_for(kernel)
    _validate_scale_shapes(kernel, m=m, n=n, k=k, a_scale=a_scale, b_scale=b_scale)
    return a, b, a_scale, b_scale, m, n, k


def launch_generated_kernel(
    a: Any,
    b: Any,
    *,
    kernel: KernelMetadata,
    a_scale: Any,
    b_scale: Any,
    c: Any | None = None,
    gate: Any | None = None,
    root: str | Path | None = None,
    library_path: str | Path | None = None,
    stream: Any | None = None,
) -> Any:
    """Launches a dense table kernel (reference native.py:690-767)."""
    torch = _torch()
    a, b, a_scale, b_scale, m, n, k = _prepare_dense(torch, a, b, kernel, a_scale, b_scale, gate)
    out_dtype = _output_torch_dtype(torch, kernel)
    if c is None:
        c = torch.empty((m, n), device=a.device, dtype=out_dtype)
    c = _require_contiguous("c", c)
    if c.dtype != out_dtype:
        raise ValueError(f"output dtype must be {out_dtype}; got {c.dtype}")
    if tuple(c.shape[-2:]) != (m, n):
        raise ValueError(f"output shape must be {(m, n)}; got {tuple(c.shape[-2:])}")
    out_mode = kt.OUT_BF16 if out_dtype == torch.bfloat16 else kt.OUT_F32
    lib_path = library_path if library_path is not None else (native_library_path(root=root) if root else None)
    if kernel.tile.split_k > 1:
        # K slices add into the output (native.py:739-740 zeroes it too), on the launch stream
        if stream is None:
            c.zero_()
        else:
            with torch.cuda.stream(stream):
                c.zero_()
    _gemm_call(torch, a, b, a_scale, b_scale, c, kernel, m, n, k, out_mode, lib_path, stream)
    return c


def launch_generated_kernel_i32(
    a: Any,
    b: Any,
    *,
    kernel: KernelMetadata,
    a_scale: Any,
    b_scale: Any,
    library_path: str | Path | None = None,
    stream: Any | None = None,
) -> Any:
    """Runs a dense table kernel in verification mode: returns the exact int32
    accumulators (int32 [M, N]; [M, 2D] = [up | gate] for SwiGLU kernels;
    the full-K integer sum for subchannel kernels)."""
    torch = _torch()
    a, b, a_scale, b_scale, m, n, k = _prepare_dense(torch, a, b, kernel, a_scale, b_scale, None)
    cols = 2 * n if kernel.epilogue is Epilogue.SWIGLU else n
    c = torch.empty((m, cols), device=a.device, dtype=torch.int32)
    _gemm_call(torch, a, b, a_scale, b_scale, c, kernel, m, n, k, kt.OUT_I32, library_path, stream)
    return c


# ---------------------------------------------------------------------------
# Device quantization and int4 packing


def _quant_source(torch: Any, x: Any) -> int:
    codes = {torch.float32: kt.SRC_F32, torch.float16: kt.SRC_F16, torch.bfloat16: kt.SRC_BF16,
             torch.int8: kt.SRC_I8}
    if x.dtype not in codes:
        raise ValueError(f"device quantization reads float32, float16, bfloat16 or int8 tensors; got {x.dtype}")
    return codes[x.dtype]


def quantize_device(x: Any, *, mode: int, bits: int = 4, inv_scale: float = 1.0, library_path=None,
                    stream: Any | None = None) -> Any:
    """Runs amd_strix_halo_kernels_quantize over the rows of a 2-D CUDA tensor
    whose rows are contiguous (x.stride(1) == 1): int8 codes (QUANT_CODES),
    int4 pairs along each row (QUANT_PACK_COLS, [rows, ceil(cols/2)] uint8) or
    int4 pairs of consecutive rows (QUANT_PACK_ROWS, [ceil(rows/2), cols]
    uint8).  inv_scale is the fp32 reciprocal of the scale (unused for int8
    sources, which are packed as given)."""
    torch = _torch()
    if x.dim() != 2:
        raise ValueError(f"device quantization takes a 2-D tensor; got {x.dim()} dimensions")
    if x.device.type != "cuda":
        raise ValueError("device quantization requires a CUDA tensor")
    if x.numel() > 0 and (x.stride(1) != 1 or (x.shape[0] > 1 and x.stride(0) < x.shape[1])):
        x = x.contiguous()
    src = _quant_source(torch, x)
    rows, cols = int(x.shape[0]), int(x.shape[1])
    if mode == kt.QUANT_CODES:
        out = torch.empty((rows, cols), device=x.device, dtype=torch.int8)
    elif mode == kt.QUANT_PACK_COLS:
        out = torch.empty((rows, (cols + 1) // 2), device=x.device, dtype=torch.uint8)
    elif mode == kt.QUANT_PACK_ROWS:
        out = torch.empty(((rows + 1) // 2, cols), device=x.device, dtype=torch.uint8)
    else:
        raise ValueError(f"unknown quantize mode {mode}")
    if out.numel() == 0:
        return out
    lib = _verified_library(library_path)
    ld_x = int(x.stride(0)) if rows > 1 else cols
    rc = lib.amd_strix_halo_kernels_quantize(_device_index(x), _stream_handle(torch, x, stream), x.data_ptr(), src,
                                             rows, cols, ld_x, float(inv_scale), bits, mode, out.data_ptr(),
                                             int(out.shape[1]))
    _check(lib, rc)
    return out


def select_dense_index(*, dtype_bits: int, layout: int, subchannel: int, epilogue: int, schedule: int,
                       split_k: int, m: int, n: int, k: int, library_path=None) -> int:
    """The table index amd_strix_halo_kernels_select_dense picks (the
    registry's selection rule, evaluated by the library)."""
    lib = _verified_library(library_path)
    out = ctypes.c_int32(-1)
    _check(lib, lib.amd_strix_halo_kernels_select_dense(dtype_bits, layout, subchannel, epilogue, schedule, split_k,
                                                        m, n, k, ctypes.byref(out)))
    return int(out.value)


_LAYOUT_CODES = {"nn": kt.LAYOUT_NN, "nt": kt.LAYOUT_NT, "tn": kt.LAYOUT_TN, "tt": kt.LAYOUT_TT}
_EPILOGUE_CODES = {"none": kt.EPILOGUE_NONE, "relu2": kt.EPILOGUE_RELU2, "swiglu": kt.EPILOGUE_SWIGLU}


def index_for_foreign_kernel(kernel: Any, *, m: int, n: int, k: int, library_path=None) -> int:
    """The gfx950 table index for a KernelMetadata of another registry (the
    reference's gfx1151 tiles, registry.py:112-176, which have no entry
    here), read by its public fields only (a_dtype, layout, scale,
    epilogue, schedule, tile.split_k) and the call's logical shape: what a
    bridge that keeps the reference's registry passes to
    amd_strix_halo_kernels_select_dense."""
    sub = kernel.scale.subchannel_size if kernel.scale.mode.value == "subchannel" else 0
    return select_dense_index(dtype_bits=4 if kernel.a_dtype.value == "int4" else 8,
                              layout=_LAYOUT_CODES[kernel.layout.value], subchannel=int(sub or 0),
                              epilogue=_EPILOGUE_CODES[kernel.epilogue.value],
                              schedule=kt.SCHEDULE_PERSISTENT if kernel.schedule.value == "persistent"
                              else kt.SCHEDULE_STANDARD,
                              split_k=int(kernel.tile.split_k), m=m, n=n, k=k, library_path=library_path)


# ---------------------------------------------------------------------------
# Ragged


def ragged_task_capacity(rows: int, groups: int, tile: int, align_tile: int, *, library_path=None) -> int:
    lib = _verified_library(library_path)
    return int(lib.amd_strix_halo_kernels_ragged_task_capacity(rows, groups, tile, align_tile))


def ragged_group_info_device(
    group_sizes_i32: Any,
    *,
    tile: int,
    align_tile: int,
    capacity: int,
    with_info: bool,
    library_path: str | Path | None = None,
    stream: Any | None = None,
) -> tuple[Any, Any, Any | None]:
    """Builds the task list on the device (replaces calculate_group_info's
    Triton kernel, ragged.py:127-185, 284-305).  Returns (tasks int32
    [capacity, 4], num_tasks int32 [1], info int64 [6, capacity] or None)."""
    torch = _torch()
    lib = _verified_library(library_path)
    dev = group_sizes_i32.device
    tasks = torch.empty((max(capacity, 1), 4), device=dev, dtype=torch.int32)
    num = torch.empty((1,), device=dev, dtype=torch.int32)
    info = torch.empty((6, max(capacity, 1)), device=dev, dtype=torch.int64) if with_info else None
    rc = lib.amd_strix_halo_kernels_ragged_group_info(
        _device_index(group_sizes_i32),
        _stream_handle(torch, group_sizes_i32, stream),
        group_sizes_i32.data_ptr(),
        int(group_sizes_i32.shape[0]),
        tile,
        align_tile,
        capacity,
        tasks.data_ptr(),
        num.data_ptr(),
        info.data_ptr() if info is not None else None,
    )
    _check(lib, rc)
    return tasks, num, info


def ragged_workspace_bytes(desc: kt.KernelDesc, m: int, n: int, k_packed: int, groups: int, *,
                           library_path=None) -> int:
    """Workspace bytes a ragged table entry needs (0 unless FP6)."""
    lib = _verified_library(library_path)
    out = ctypes.c_uint64(0)
    _check(lib, lib.amd_strix_halo_kernels_ragged_workspace_bytes(desc.index, m, n, k_packed, groups,
                                                                   ctypes.byref(out)))
    return int(out.value)


def _ragged_workspace(torch, desc, like, m, n, k_packed, groups, stream, head: int = 0):
    """One uint8 buffer of `head` bytes followed by the entry's operand
    workspace (sized by the table mirror, which the library's
    amd_strix_halo_kernels_ragged_workspace_bytes matches), from torch's
    caching allocator on the launch stream (see _gemm_call)."""
    nbytes = desc.ragged_workspace_bytes(m, n, k_packed, groups)
    total = head + nbytes
    buf = torch.empty(total, dtype=torch.uint8, device=like.device) if total else None
    if buf is not None and stream is not None:
        buf.record_stream(stream)
    return buf, nbytes


def launch_ragged_fwd(
    lhs: Any,
    rhs: Any,
    group_sizes_i32: Any,
    *,
    a_scale: Any,
    b_scale: Any,
    out: Any,
    layout: GemmLayout,
    subchannel: int | None,
    block_m: int,
    align_tile: int,
    rows: int,
    cols: int,
    k_packed: int,
    out_mode: int,
    fp6: bool = False,
    library_path: str | Path | None = None,
    stream: Any | None = None,
) -> Any:
    """Device task list + grouped forward in one library call (replaces
    calculate_group_info + launch_ragged_fwd_kernel, ragged.py:201-323 and
    native.py:533-600).  No host synchronisation.  fp6: run the fp6 entry
    (per-channel or subchannel; block_m must be its task tile, kt.RAGGED_FP6_BLOCK_M),
    whose operands are converted into a workspace and whose tasks need
    align_tile a multiple of 32.  The task list, its count and the
    workspace share one allocation."""
    torch = _torch()
    lib = _verified_library(library_path)
    if fp6 and block_m != kt.RAGGED_FP6_BLOCK_M:
        raise ValueError(f"the fp6 ragged forward takes tasks of {kt.RAGGED_FP6_BLOCK_M} rows; got block_m={block_m}")
    desc = kt.find_ragged(kt.FAMILY_RAGGED_FWD, layout=kt.LAYOUT_CODES[layout.value], subchannel=subchannel,
                          block_m=block_m, fp6=fp6)
    if fp6 and align_tile % 32:
        raise ValueError(f"the fp6 ragged forward needs align_tile a multiple of 32; got {align_tile}")
    groups = int(group_sizes_i32.shape[0])
    capacity = kt.ragged_task_capacity(rows, groups, block_m)
    # tasks [capacity, 4] int32, then num_tasks (16 bytes), then the workspace
    head = 16 * max(capacity, 1) + 16
    buf, nbytes = _ragged_workspace(torch, desc, lhs, rows, cols, k_packed, groups, stream, head)
    base = buf.data_ptr()
    # the task list and the forward in one library call (one launch fewer for
    # the fp6 entries, whose conversion launch builds the list)
    rc = lib.amd_strix_halo_kernels_launch_ragged_fwd_grouped(
        desc.index,
        _device_index(lhs),
        _stream_handle(torch, lhs, stream),
        lhs.data_ptr(),
        rhs.data_ptr(),
        a_scale.data_ptr(),
        b_scale.data_ptr(),
        group_sizes_i32.data_ptr(),
        align_tile,
        base,
        base + head - 16,
        capacity,
        out.data_ptr(),
        rows,
        cols,
        k_packed,
        groups,
        subchannel or 0,
        out_mode,
        base + head if nbytes else None,
        nbytes,
    )
    _check(lib, rc)
    return out


def launch_ragged_bwd(
    lhs: Any,
    rhs: Any,
    group_sizes_i32: Any,
    *,
    a_scale: Any,
    b_scale: Any,
    out: Any,
    layout: GemmLayout,
    subchannel: int | None,
    split_k: int,
    rows: int,
    cols: int,
    k_packed: int,
    out_mode: int = kt.OUT_F32,
    fp6: bool = False,
    library_path: str | Path | None = None,
    stream: Any | None = None,
) -> Any:
    """Grouped K-ragged backward (replaces launch_ragged_bwd_kernel,
    native.py:603-667).  fp6: run the fp6 entry of the scale mode, whose operands
    are converted into a workspace."""
    torch = _torch()
    lib = _verified_library(library_path)
    desc = kt.find_ragged(kt.FAMILY_RAGGED_BWD, layout=kt.LAYOUT_CODES[layout.value], subchannel=subchannel,
                          fp6=fp6)
    groups = int(group_sizes_i32.shape[0])
    work, nbytes = _ragged_workspace(torch, desc, lhs, rows, cols, k_packed, groups, stream)
    rc = lib.amd_strix_halo_kernels_launch_ragged_bwd_ws(
        desc.index,
        _device_index(lhs),
        _stream_handle(torch, lhs, stream),
        lhs.data_ptr(),
        rhs.data_ptr(),
        a_scale.data_ptr(),
        b_scale.data_ptr(),
        group_sizes_i32.data_ptr(),
        out.data_ptr(),
        rows,
        cols,
        k_packed,
        groups,
        subchannel or 0,
        split_k,
        out_mode,
        work.data_ptr() if work is not None else None,
        nbytes,
    )
    _check(lib, rc)
    return out
