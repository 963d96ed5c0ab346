"""amd_strix_halo_kernels_launch_gemm_noalloc against launch_gemm_ws.

The no-allocation entry point runs the fp6 entries with the library's static
scratch array in place of a caller workspace, and the skinny (STREAM) entries
that split K keep their counters and partials there.  Each case calls it
through the C ABI and compares the output with launch_gemm_ws on a
torch-allocated workspace, bit for bit, and with the CPU oracle (within
2 ulp for SwiGLU).  Calls come in a row on one device, each of a kind smaller
than the one before, so a later call runs on the scratch contents an earlier
one left behind (a skinny split call after fp6 conversions filled it).  The
entry point allocates nothing: free device memory and torch's allocated
bytes stay the same across calls, and a call captured in a HIP graph
replays to the eager result.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import ref
from tests._util import bf16_bits, dense_case, max_ulp, stable_seed, to_dev

torch = pytest.importorskip("torch")

from amd_strix_halo_kernels import kernel_table as kt  # noqa: E402
from amd_strix_halo_kernels import native  # noqa: E402

pytestmark = pytest.mark.gpu

_LAYOUT = {"nn": kt.LAYOUT_NN, "nt": kt.LAYOUT_NT, "tn": kt.LAYOUT_TN}
_EPI_NAME = {kt.EPILOGUE_NONE: "none", kt.EPILOGUE_RELU2: "relu2", kt.EPILOGUE_SWIGLU: "swiglu"}


def _index(kind: str, layout: str, scale_mode: int, epilogue: int, block_m: int = 0) -> int:
    fmt = kt.OPERANDS_FP6 if kind == "fp6" else kt.OPERANDS_STREAM
    epi_kind = kt.EPI_KIND_SWIGLU if epilogue == kt.EPILOGUE_SWIGLU else kt.EPI_KIND_PLAIN
    for d in kt.entries(kt.FAMILY_DENSE):
        if (d.operand_format == fmt and d.layout == _LAYOUT[layout] and d.scale_mode == scale_mode
                and d.epilogue_kind == epi_kind and d.schedule == 0 and d.split_k == 1 and d.dtype_bits == 4
                and (block_m == 0 or d.block_m == block_m)):
            return d.index
    raise LookupError((kind, layout, scale_mode, epilogue, block_m))


def _call(lib, fn, index, device, a, b, sa, sb, out, m, n, k, sub, epi, *extra, stream=None):
    handle = (stream if stream is not None else torch.cuda.current_stream(device)).cuda_stream
    rc = fn(index, device.index or 0, handle, a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
            out.data_ptr(), m, n, k, sub, epi, kt.OUT_BF16, *extra)
    assert rc == 0, lib.amd_strix_halo_kernels_last_error().decode()


def _operands(kind, layout, sub, epi, m, n, k, device):
    seed = stable_seed("noalloc", kind, layout, sub, epi, m, n, k)
    _, _, a_arg, b_arg, sa, sb = dense_case(seed, bits=4, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                           swiglu=epi == kt.EPILOGUE_SWIGLU)
    dev = [to_dev(torch, x, device) for x in (a_arg, b_arg, sa, sb)]
    return (a_arg, b_arg, sa, sb), dev


def _workspace(lib, index, m, n, k, device):
    need = ctypes.c_uint64(0)
    assert lib.amd_strix_halo_kernels_gemm_workspace_bytes(index, m, n, k, ctypes.byref(need)) == 0
    assert 0 < need.value <= kt.NOALLOC_SCRATCH_BYTES
    # zero-filled: the skinny split entries need zero counters in a caller workspace
    return torch.zeros(need.value, dtype=torch.uint8, device=device), need.value


# (kind, layout, subchannel, epilogue, m, n, k): fp6 and skinny-split calls in
# a row, each smaller than the one of its kind before it
_CASES = [
    ("fp6", "nn", None, kt.EPILOGUE_NONE, 512, 768, 2048),
    ("fp6", "nn", None, kt.EPILOGUE_SWIGLU, 256, 512, 1024),
    ("stream", "nn", None, kt.EPILOGUE_NONE, 16, 8192, 8192),
    ("fp6", "tn", 128, kt.EPILOGUE_RELU2, 256, 512, 1024),
    ("stream", "nn", None, kt.EPILOGUE_NONE, 16, 128, 8192 + 32),
    ("fp6", "nt", None, kt.EPILOGUE_RELU2, 256, 256, 256),
]


def test_noalloc_matches_workspace_entry_point_in_a_row(device):
    lib = native.load_dispatch_library()
    results = []
    for kind, layout, sub, epi, m, n, k in _CASES:
        index = _index(kind, layout, kt.SCALE_SUBCHANNEL if sub else kt.SCALE_PER_CHANNEL, epi,
                       block_m=16 if kind == "stream" else 0)
        if kind == "stream":
            assert kt.sk_split_count(kt.TABLE[index], m, n, k) > 1
        (a_arg, b_arg, sa, sb), (a, b, ta, tb) = _operands(kind, layout, sub, epi, m, n, k, device)
        print(f"case noalloc {kind} kernel={index} layout={layout} sub={sub} epi={epi} shape=({m},{n},{k})",
              flush=True)
        want_out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        got_out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
        work, nbytes = _workspace(lib, index, m, n, k, device)
        _call(lib, lib.amd_strix_halo_kernels_launch_gemm_ws, index, device, a, b, ta, tb, want_out, m, n, k,
              sub or 0, epi, work.data_ptr(), nbytes)
        _call(lib, lib.amd_strix_halo_kernels_launch_gemm_noalloc, index, device, a, b, ta, tb, got_out, m, n, k,
              sub or 0, epi)
        torch.cuda.synchronize()
        got, want = bf16_bits(torch, got_out), bf16_bits(torch, want_out)
        assert np.array_equal(got, want), f"no-alloc differs from launch_gemm_ws ({kind} {layout} {m}x{n}x{k})"
        oracle = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, layout=layout, a_scale=sa, b_scale=sb,
                                         subchannel=sub, epilogue=_EPI_NAME[epi])
        if epi == kt.EPILOGUE_SWIGLU:
            assert max_ulp(got, oracle) <= 2, f"no-alloc SwiGLU output beyond 2 ulp of the oracle ({m}x{n}x{k})"
        else:
            assert np.array_equal(got, oracle), f"no-alloc output differs from the oracle ({kind} {m}x{n}x{k})"
        results.append(got)
    assert len(results) == len(_CASES)


def test_noalloc_allocates_nothing(device):
    """After one warm-up call per entry, further calls leave the device's
    free memory and torch's allocated bytes unchanged."""
    lib = native.load_dispatch_library()
    calls = []
    for kind, layout, sub, epi, m, n, k in (_CASES[0], _CASES[2]):
        index = _index(kind, layout, kt.SCALE_PER_CHANNEL, epi, block_m=16 if kind == "stream" else 0)
        _, (a, b, ta, tb) = _operands(kind, layout, sub, epi, m, n, k, device)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        calls.append((index, a, b, ta, tb, out, m, n, k, epi))
    for index, a, b, ta, tb, out, m, n, k, epi in calls:  # warm-up
        _call(lib, lib.amd_strix_halo_kernels_launch_gemm_noalloc, index, device, a, b, ta, tb, out, m, n, k, 0, epi)
    torch.cuda.synchronize()
    free0, allocated0 = torch.cuda.mem_get_info(device)[0], torch.cuda.memory_allocated(device)
    for _ in range(3):
        for index, a, b, ta, tb, out, m, n, k, epi in calls:
            _call(lib, lib.amd_strix_halo_kernels_launch_gemm_noalloc, index, device, a, b, ta, tb, out, m, n, k, 0,
                  epi)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(device)[0] == free0
    assert torch.cuda.memory_allocated(device) == allocated0


@pytest.mark.parametrize("case", [0, 2], ids=["fp6", "stream_split"])
def test_noalloc_call_replays_in_a_graph(case, device):
    """A no-allocation call captured in a HIP graph (fp6: two conversions and
    the GEMM; skinny split: the counter clear and the GEMM) replays to the
    eager result, with eager work and synchronizations between replays."""
    lib = native.load_dispatch_library()
    kind, layout, sub, epi, m, n, k = _CASES[case]
    index = _index(kind, layout, kt.SCALE_PER_CHANNEL, epi, block_m=16 if kind == "stream" else 0)
    _, (a, b, ta, tb) = _operands(kind, layout, sub, epi, m, n, k, device)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    print(f"case noalloc graph {kind} kernel={index} shape=({m},{n},{k})", flush=True)
    _call(lib, lib.amd_strix_halo_kernels_launch_gemm_noalloc, index, device, a, b, ta, tb, out, m, n, k, 0, epi,
          stream=stream)
    torch.cuda.current_stream(device).wait_stream(stream)
    torch.cuda.synchronize()
    eager = bf16_bits(torch, out)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _call(lib, lib.amd_strix_halo_kernels_launch_gemm_noalloc, index, device, a, b, ta, tb, out, m, n, k, 0,
              epi, stream=stream)
    other = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    for i in range(3):
        out.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(torch, out), eager), f"replay {i}"
        # an eager call on the same scratch between replays
        _call(lib, lib.amd_strix_halo_kernels_launch_gemm_noalloc, index, device, a, b, ta, tb, other, m, n, k, 0,
              epi)
        torch.cuda.synchronize()


def test_noalloc_rejects_shapes_beyond_the_scratch(device):
    lib = native.load_dispatch_library()
    index = _index("fp6", "nn", kt.SCALE_PER_CHANNEL, kt.EPILOGUE_NONE)
    m = n = k = 16384  # 0.75 * 2 * 16384^2 bytes of fp6 operands: 384 MiB
    fake = 0x10000
    rc = lib.amd_strix_halo_kernels_launch_gemm_noalloc(index, device.index or 0, 0, fake, fake, fake, fake, fake,
                                                         m, n, k, 0, kt.EPILOGUE_NONE, kt.OUT_BF16)
    assert rc == 1
    assert "scratch holds at most" in lib.amd_strix_halo_kernels_last_error().decode()
