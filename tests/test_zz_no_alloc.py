"""amd_strix_halo_kernels_launch_gemm_noalloc against launch_gemm_ws.

The no-allocation entry point runs the fp6 entries with the library's static
scratch array in place of a caller workspace.  Each case calls it through the
C ABI and compares the output with launch_gemm_ws on a torch-allocated
workspace, bit for bit (the bar for per-channel and subchannel bf16 output),
and with the CPU oracle.  Calls come in a row on one device, each smaller
than the one before, so a later call runs on the scratch contents an earlier
one left behind.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import ref
from tests._util import bf16_bits, dense_case, stable_seed, to_dev

torch = pytest.importorskip("torch")

from amd_strix_halo_kernels import kernel_table as kt  # noqa: E402
from amd_strix_halo_kernels import native  # noqa: E402

pytestmark = pytest.mark.gpu

_LAYOUT = {"nn": kt.LAYOUT_NN, "nt": kt.LAYOUT_NT, "tn": kt.LAYOUT_TN}


def _fp6_index(layout: str, scale_mode: int) -> int:
    for d in kt.entries(kt.FAMILY_DENSE):
        if (d.operand_format == kt.OPERANDS_FP6 and d.layout == _LAYOUT[layout] and d.scale_mode == scale_mode
                and d.epilogue_kind == kt.EPI_KIND_PLAIN and d.schedule == 0 and d.split_k == 1):
            return d.index
    raise LookupError((layout, scale_mode))


def _call(lib, fn, index, device, a, b, sa, sb, out, m, n, k, sub, epi, *extra):
    stream = torch.cuda.current_stream(device).cuda_stream
    rc = fn(index, device.index or 0, stream, a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
            out.data_ptr(), m, n, k, sub, epi, kt.OUT_BF16, *extra)
    assert rc == 0, lib.amd_strix_halo_kernels_last_error().decode()


# (layout, subchannel, epilogue, m, n, k): each case smaller than the one before
_CASES = [
    ("nn", None, kt.EPILOGUE_NONE, 512, 768, 2048),
    ("tn", 128, kt.EPILOGUE_RELU2, 256, 512, 1024),
    ("nt", None, kt.EPILOGUE_RELU2, 256, 256, 256),
]


def test_noalloc_matches_workspace_entry_point_in_a_row(device):
    lib = native.load_dispatch_library()
    results = []
    for layout, sub, epi, m, n, k in _CASES:
        index = _fp6_index(layout, kt.SCALE_SUBCHANNEL if sub else kt.SCALE_PER_CHANNEL)
        seed = stable_seed("noalloc", layout, sub, m, n, k)
        _, _, a_arg, b_arg, sa, sb = dense_case(seed, bits=4, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                               swiglu=False)
        print(f"case noalloc kernel={index} layout={layout} sub={sub} shape=({m},{n},{k})", flush=True)
        a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
        ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
        want_out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        got_out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
        need = ctypes.c_uint64(0)
        assert lib.amd_strix_halo_kernels_gemm_workspace_bytes(index, m, n, k, ctypes.byref(need)) == 0
        assert 0 < need.value <= kt.NOALLOC_SCRATCH_BYTES
        work = torch.empty(need.value, dtype=torch.uint8, device=device)
        _call(lib, lib.amd_strix_halo_kernels_launch_gemm_ws, index, device, a, b, ta, tb, want_out, m, n, k,
              sub or 0, epi, work.data_ptr(), need.value)
        _call(lib, lib.amd_strix_halo_kernels_launch_gemm_noalloc, index, device, a, b, ta, tb, got_out, m, n, k,
              sub or 0, epi)
        torch.cuda.synchronize()
        got, want = bf16_bits(torch, got_out), bf16_bits(torch, want_out)
        assert np.array_equal(got, want), f"no-alloc output differs from launch_gemm_ws ({layout}, {m}x{n}x{k})"
        oracle = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, layout=layout, a_scale=sa, b_scale=sb,
                                         subchannel=sub, epilogue="relu2" if epi == kt.EPILOGUE_RELU2 else "none")
        assert np.array_equal(got, oracle), f"no-alloc output differs from the oracle ({layout}, {m}x{n}x{k})"
        results.append(got)
    assert len(results) == len(_CASES)


def test_noalloc_rejects_shapes_beyond_the_scratch(device):
    lib = native.load_dispatch_library()
    index = _fp6_index("nn", kt.SCALE_PER_CHANNEL)
    m = n = k = 16384  # 0.75 * 2 * 16384^2 bytes of fp6 operands: 384 MiB
    fake = 0x10000
    rc = lib.amd_strix_halo_kernels_launch_gemm_noalloc(index, device.index or 0, 0, fake, fake, fake, fake, fake,
                                                         m, n, k, 0, kt.EPILOGUE_NONE, kt.OUT_BF16)
    assert rc == 1
    assert "scratch holds at most" in lib.amd_strix_halo_kernels_last_error().decode()
