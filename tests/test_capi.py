"""C ABI of libamd_strix_halo_kernels_gfx950.so, checked without a GPU.

The library must load on a machine without a GPU, export every symbol that
include/strix_halo_gfx950.h declares, report its status, describe its kernel
table, and reject bad launches with rc=1 and a readable last_error before it
touches the HIP runtime (the reference's dispatcher contract,
native/src/dispatch.cpp:18-23, 206-283).
"""

from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

import pytest

from amd_strix_halo_kernels import kernel_table as kt
from amd_strix_halo_kernels import native

HEADER = Path(__file__).resolve().parents[1] / "include" / "strix_halo_gfx950.h"
FAKE = 0x10000  # never dereferenced: every call below fails validation first


@pytest.fixture(scope="module")
def lib():
    return native.load_dispatch_library()


def _declared_functions() -> list[str]:
    # declarations start a line with a return type: "int name(", "const char* name("
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:const\s+)?\w+\s*\*?\s*(amd_strix_halo_kernels_\w+)\(", text, re.M)))


def test_every_declared_symbol_is_exported(lib):
    names = _declared_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name


def test_status_functions(lib):
    assert lib.amd_strix_halo_kernels_dispatch_version() == 2
    assert lib.amd_strix_halo_kernels_has_compiled_code_objects() == 1
    assert lib.amd_strix_halo_kernels_arch() == b"gfx950"
    assert lib.amd_strix_halo_kernels_has_hip_runtime() in (0, 1)
    assert lib.amd_strix_halo_kernels_has_linked_kernels() in (0, 1)
    status = native.dispatch_runtime_status()
    assert status.dispatch_version == 2 and status.has_compiled_code_objects


def test_kernel_table_matches_python_mirror(lib):
    table = native.library_kernel_table(lib)
    assert table == kt.TABLE
    assert [d.index for d in table] == list(range(len(table)))
    desc = native._Desc()
    assert lib.amd_strix_halo_kernels_kernel_table_entry(len(table), ctypes.byref(desc)) == 1
    assert b"out of range" in lib.amd_strix_halo_kernels_last_error()


def _dense_index(**want) -> int:
    for d in kt.entries(kt.FAMILY_DENSE):
        if all(getattr(d, k) == v for k, v in want.items()):
            return d.index
    raise LookupError(want)


def _gemm(lib, index, m, n, k, *, sub=0, epi=0, mode=0, out=FAKE, ptr=FAKE):
    return lib.amd_strix_halo_kernels_launch_gemm(index, 0, 0, ptr, ptr, ptr, ptr, out, m, n, k, sub, epi, mode)


def _err(lib) -> str:
    return lib.amd_strix_halo_kernels_last_error().decode()


def test_gemm_rejects_bad_index_and_family(lib):
    assert _gemm(lib, len(kt.TABLE) + 5, 64, 64, 64) == 1
    assert "out of range" in _err(lib)
    fwd = kt.entries(kt.FAMILY_RAGGED_FWD)[0].index
    assert _gemm(lib, fwd, 64, 64, 64) == 1
    assert "another kernel family" in _err(lib)


def test_gemm_rejects_null_pointers(lib):
    idx = _dense_index(dtype_bits=4, layout=0, block_m=64, block_n=64, scale_mode=0, epilogue_kind=0)
    assert _gemm(lib, idx, 64, 64, 64, ptr=0) == 1
    assert "non-null" in _err(lib)


def test_gemm_tile_multiple_messages_follow_the_reference(lib):
    idx = _dense_index(dtype_bits=4, layout=0, block_m=256, block_n=256, scale_mode=0, epilogue_kind=0)
    assert _gemm(lib, idx, 100, 256, 128) == 1
    assert "M=100 is not divisible by BLOCK_M=256" in _err(lib)
    assert _gemm(lib, idx, 256, 100, 96) == 1
    msg = _err(lib)
    assert "N=100 is not divisible by BLOCK_N=256" in msg
    assert "K=96 is not divisible by BLOCK_K*SPLIT_K=128" in msg
    assert _gemm(lib, idx, 0, 256, 128) == 1
    assert "must be positive" in _err(lib)


def test_noalloc_validates_before_touching_the_device(lib):
    f6 = _dense_index(dtype_bits=4, layout=0, block_m=256, block_n=256, scale_mode=0, epilogue_kind=0,
                      operand_format=kt.OPERANDS_FP6, schedule=0, split_k=1)
    noalloc = lib.amd_strix_halo_kernels_launch_gemm_noalloc
    # 0.75 * (16384 * 16384 * 2) bytes of fp6 operands do not fit the scratch
    assert noalloc(f6, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, 16384, 16384, 16384, 0, 0, 0) == 1
    assert f"scratch holds at most {kt.NOALLOC_SCRATCH_BYTES} bytes" in _err(lib)
    need = ctypes.c_uint64(0)
    assert lib.amd_strix_halo_kernels_gemm_workspace_bytes(f6, 8192, 8192, 8192, ctypes.byref(need)) == 0
    assert need.value <= kt.NOALLOC_SCRATCH_BYTES  # C2 fits
    assert noalloc(f6, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, 100, 256, 128, 0, 0, 0) == 1
    assert "M=100 is not divisible by BLOCK_M=256" in _err(lib)
    assert noalloc(f6, 0, 0, 0, FAKE, FAKE, FAKE, FAKE, 256, 256, 128, 0, 0, 0) == 1
    assert "non-null" in _err(lib)


def test_gemm_rejects_mismatched_modes(lib):
    pc = _dense_index(dtype_bits=4, layout=0, block_m=64, block_n=64, scale_mode=0, epilogue_kind=0)
    sc = _dense_index(dtype_bits=4, layout=0, block_m=64, block_n=64, scale_mode=1, epilogue_kind=0,
                      min_subchannel=64)
    assert _gemm(lib, pc, 64, 64, 64, sub=64) == 1
    assert "subchannel = 0" in _err(lib)
    assert _gemm(lib, sc, 64, 64, 128, sub=32) == 1
    assert "not served" in _err(lib)
    assert _gemm(lib, pc, 64, 64, 64, epi=2) == 1
    assert "epilogue" in _err(lib)
    assert _gemm(lib, pc, 64, 64, 64, mode=7) == 1
    assert "output mode" in _err(lib)
    assert _gemm(lib, pc, 64, 64, 262144) == 1
    assert "K <= 131071" in _err(lib)
    assert _gemm(lib, pc, 64, 64, 131072) == 1  # a -8 row times a -8 column would sum to 2^31
    assert "K <= 131071" in _err(lib)
    assert _gemm(lib, pc, 64, 64, 64, out=FAKE + 4) == 1
    assert "aligned" in _err(lib)


def test_ragged_entry_points_validate_before_launch(lib):
    I = lib.amd_strix_halo_kernels_ragged_group_info
    assert I(0, 0, FAKE, 3, 32, 12, 8, FAKE, FAKE, None) == 1
    assert "multiple of align_tile" in _err(lib)
    assert I(0, 0, FAKE, 1 << 20, 32, 8, 8, FAKE, FAKE, None) == 1
    assert "groups are supported" in _err(lib)
    bwd = kt.entries(kt.FAMILY_RAGGED_BWD)[0].index
    B = lib.amd_strix_halo_kernels_launch_ragged_bwd
    assert B(bwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 16, 16, 2, 0, 0, 0) == 1
    assert "split_k" in _err(lib)
    assert B(bwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 16, 16, 2, 0, 1, 0) == 1
    assert "fp32" in _err(lib)
    fwd = kt.entries(kt.FAMILY_RAGGED_FWD)[0].index
    F = lib.amd_strix_halo_kernels_launch_ragged_fwd
    assert F(fwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 16, 16, 16, 2, 32, 0) == 1
    assert "subchannel = 0" in _err(lib)
    # the one-call forward checks the task-list arguments against the entry's tile
    G = lib.amd_strix_halo_kernels_launch_ragged_fwd_grouped
    fp6 = kt.find_ragged(kt.FAMILY_RAGGED_FWD, layout=kt.LAYOUT_NN, subchannel=None, fp6=True)
    args = (FAKE, FAKE, FAKE, FAKE, FAKE)
    assert G(fp6.index, 0, 0, *args, 96, FAKE, FAKE, 8, FAKE, 16, 16, 64, 2, 0, 0, FAKE, 1 << 20) == 1
    assert "multiple of align_tile" in _err(lib)
    assert G(fp6.index, 0, 0, *args, 16, FAKE, FAKE, 8, FAKE, 16, 16, 64, 2, 0, 0, FAKE, 1 << 20) == 1
    assert "multiple of 32" in _err(lib)
    assert G(fp6.index, 0, 0, *args, 32, FAKE, FAKE, 8, FAKE, 16, 16, 64, 1 << 20, 0, 0, FAKE, 1 << 20) == 1
    assert "groups are supported" in _err(lib)
    assert G(fp6.index, 0, 0, *args, 32, None, FAKE, 8, FAKE, 16, 16, 64, 2, 0, 0, FAKE, 1 << 20) == 1
    assert "task list pointers" in _err(lib)
    assert G(fp6.index, 0, 0, *args, 32, FAKE, FAKE, 8, FAKE, 16, 16, 64, 2, 0, 0, FAKE, 16) == 1
    assert "workspace" in _err(lib)
    # a task buffer below amd_strix_halo_kernels_ragged_task_capacity is refused
    need = lib.amd_strix_halo_kernels_ragged_task_capacity(4096, 2, fp6.block_m, 32)
    assert G(fp6.index, 0, 0, *args, 32, FAKE, FAKE, need - 1, FAKE, 4096, 16, 64, 2, 0, 0, FAKE, 1 << 30) == 1
    assert f"below the {need} tasks" in _err(lib)
    assert G(bwd, 0, 0, *args, 32, FAKE, FAKE, 8, FAKE, 16, 16, 64, 2, 0, 0, FAKE, 1 << 20) == 1


@pytest.mark.parametrize("rows,groups,tile,align", [(8192, 8, 64, 8), (0, 3, 16, 8), (17, 40, 16, 16), (1, 1, 128, 8)])
def test_task_capacity_bounds_the_task_list(lib, rows, groups, tile, align):
    from oracle import ref

    cap = lib.amd_strix_halo_kernels_ragged_task_capacity(rows, groups, tile, align)
    assert cap == rows // tile + 2 * groups + 1 == kt.ragged_task_capacity(rows, groups, tile)
    # worst case: every group starts one row past an aligned boundary
    r = ref.rng(rows + groups)
    for _ in range(20):
        sizes = r.multinomial(rows, r.dirichlet(ref.np.ones(groups))) if rows else ref.np.zeros(groups, int)
        assert ref.calculate_group_info(sizes, tile, align_tile=align).num_tasks <= cap


def test_last_error_is_thread_local(lib):
    assert _gemm(lib, -1, 64, 64, 64) == 1
    mine = _err(lib)
    seen = {}

    def other():
        idx = _dense_index(dtype_bits=4, layout=0, block_m=64, block_n=64, scale_mode=0, epilogue_kind=0)
        _gemm(lib, idx, 64, 64, 64, ptr=0)
        seen["msg"] = _err(lib)

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "non-null" in seen["msg"]
    assert _err(lib) == mine


def _ws(lib, index, m, n, k):
    out = ctypes.c_uint64(0)
    rc = lib.amd_strix_halo_kernels_gemm_workspace_bytes(index, m, n, k, ctypes.byref(out))
    return rc, int(out.value)


def _gemm_ws(lib, index, m, n, k, *, work, work_bytes, epi=0, mode=0):
    return lib.amd_strix_halo_kernels_launch_gemm_ws(index, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, m, n, k, 0, epi,
                                                     mode, work, work_bytes)


def test_fp6_entries_report_their_workspace(lib):
    fp6 = [d for d in kt.entries(kt.FAMILY_DENSE) if d.operand_format == kt.OPERANDS_FP6]
    layouts = (kt.LAYOUT_NN, kt.LAYOUT_NT, kt.LAYOUT_TN)
    assert {(d.layout, d.epilogue_kind, d.scale_mode) for d in fp6} == {
        (layout, epi, kt.SCALE_PER_CHANNEL) for layout in layouts for epi in (kt.EPI_KIND_PLAIN, kt.EPI_KIND_SWIGLU)
    } | {(layout, kt.EPI_KIND_PLAIN, kt.SCALE_SUBCHANNEL) for layout in layouts}
    for d in fp6:
        if d.scale_mode == kt.SCALE_SUBCHANNEL:
            # 128 x 128 tiles, three 24 KiB stages and the 8 KiB scale ring; groups of 32 to 256
            assert (d.block_m, d.block_n, d.num_stages, d.lds_bytes) == (128, 128, 3, 81920)
            assert (d.min_subchannel, d.max_subchannel) == (32, 256)
        else:
            assert d.block_m == 256 and d.num_stages == 3 and d.lds_bytes == 148480
        assert d.dtype_bits == 4
        for m, n, k in ((256, 256, 128), (512, 1024, 4096), (8192, 8192, 8192)):
            rc, got = _ws(lib, d.index, m, n, k)
            b_cols = 2 * n if d.epilogue_kind == kt.EPI_KIND_SWIGLU else n
            # 6 bits per value: 3/4 byte per logical element of A and B
            assert rc == 0 and got == (m * k + b_cols * k) * 3 // 4 == d.workspace_bytes(m, n, k)
    packed = _dense_index(dtype_bits=4, layout=0, block_m=64, block_n=64, scale_mode=0, epilogue_kind=0)
    assert _ws(lib, packed, 256, 256, 128) == (0, 0)
    assert lib.amd_strix_halo_kernels_gemm_workspace_bytes(packed, 1, 1, 1, None) == 1
    assert "non-null" in _err(lib)


def test_fp6_launch_needs_a_workspace(lib):
    idx = _dense_index(dtype_bits=4, layout=0, block_m=256, block_n=256, operand_format=kt.OPERANDS_FP6)
    assert _gemm(lib, idx, 256, 256, 128) == 1
    assert "workspace of 49152 bytes" in _err(lib)
    assert _gemm_ws(lib, idx, 256, 256, 128, work=FAKE, work_bytes=49151) == 1
    assert "workspace of 49152 bytes" in _err(lib)
    assert _gemm_ws(lib, idx, 256, 256, 128, work=FAKE + 8, work_bytes=49152 + 8) == 1
    assert "16-byte aligned" in _err(lib)


def test_fp6_k_bounds(lib):
    # one fp32 pass is exact while |sum| <= 64 * K <= 2^24; a longer K runs in
    # slices of FP6_MAX_K whose int32 sums add into the workspace, up to
    # FP6_MAX_K_SLICED; the persistent tile multiplies K in one pass
    idx = _dense_index(dtype_bits=4, layout=0, block_m=256, block_n=256, operand_format=kt.OPERANDS_FP6,
                       schedule=kt.SCHEDULE_STANDARD, scale_mode=0, epilogue_kind=0)
    per = _dense_index(dtype_bits=4, layout=0, block_m=256, block_n=256, operand_format=kt.OPERANDS_FP6,
                       schedule=kt.SCHEDULE_PERSISTENT, scale_mode=0)
    assert kt.FP6_MAX_K * 64 == 1 << 24
    m = n = 256
    k = kt.FP6_MAX_K + 128
    need = (m + n) * k * 3 // 4 + 4 * m * n
    assert _ws(lib, idx, m, n, k) == (0, need) and kt.TABLE[idx].workspace_bytes(m, n, k) == need
    assert _gemm_ws(lib, idx, m, n, k, work=FAKE, work_bytes=need - 1) == 1
    assert f"workspace of {need} bytes" in _err(lib)
    assert _gemm_ws(lib, per, m, n, k, work=FAKE, work_bytes=1 << 40) == 1
    assert f"supports K <= {kt.FP6_MAX_K}" in _err(lib)
    assert _gemm_ws(lib, idx, m, n, kt.FP6_MAX_K_SLICED + 128, work=FAKE, work_bytes=1 << 62) == 1
    assert f"supports K <= {kt.FP6_MAX_K_SLICED}" in _err(lib)
    assert kt.TABLE[idx].max_k == kt.FP6_MAX_K_SLICED and kt.TABLE[per].max_k == kt.FP6_MAX_K


def test_split_k_bound_is_per_slice(lib):
    # each slice's int32 accumulator holds K / SPLIT_K x16-widened products
    sk2 = _dense_index(dtype_bits=4, layout=0, block_m=128, block_n=128, scale_mode=0, epilogue_kind=0, split_k=2)
    assert kt.TABLE[sk2].max_k == 2 * kt.INT4_ACC_MAX_K and kt.TABLE[sk2].supports_k(2 * kt.INT4_ACC_MAX_K)
    k = 2 * 131072  # slices of 131072: one too many for an exact accumulator
    assert lib.amd_strix_halo_kernels_launch_gemm(sk2, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, 128, 128, k, 0, 0,
                                                  kt.OUT_F32) == 1
    assert f"K <= {kt.INT4_ACC_MAX_K} per K slice (K/SPLIT_K); got K/SPLIT_K={k // 2}" in _err(lib)


def test_split_fp6_phases_validate_their_arguments(lib):
    fp6 = _dense_index(dtype_bits=4, layout=0, block_m=256, block_n=256, operand_format=kt.OPERANDS_FP6)
    packed = _dense_index(dtype_bits=4, layout=0, block_m=64, block_n=64, scale_mode=0, epilogue_kind=0)
    conv = lib.amd_strix_halo_kernels_gemm_convert
    gemm = lib.amd_strix_halo_kernels_launch_gemm_converted
    assert conv(packed, 0, 0, 0, FAKE, 256, 256, 128, FAKE, 1 << 20) == 1
    assert "only fp6 entries" in _err(lib)
    assert conv(fp6, 0, 0, 2, FAKE, 256, 256, 128, FAKE, 1 << 20) == 1
    assert "operand must be 0 (A) or 1 (B)" in _err(lib)
    assert conv(fp6, 0, 0, 1, None, 256, 256, 128, FAKE, 1 << 20) == 1
    assert "non-null" in _err(lib)
    assert conv(fp6, 0, 0, 0, FAKE, 256, 256, 128, FAKE, 100) == 1
    assert "workspace of 49152 bytes" in _err(lib)
    assert conv(fp6, 0, 0, 0, FAKE, 250, 256, 128, FAKE, 1 << 20) == 1
    assert "M=250 is not divisible by BLOCK_M=256" in _err(lib)
    assert gemm(packed, 0, 0, FAKE, FAKE, FAKE, 64, 64, 64, 0, 0, FAKE, 1 << 20) == 1
    assert "only fp6 entries" in _err(lib)
    assert gemm(fp6, 0, 0, FAKE, FAKE, FAKE, 256, 256, 128, kt.EPILOGUE_SWIGLU, 0, FAKE, 1 << 20) == 1
    assert "does not match the kernel's epilogue kind" in _err(lib)
    assert gemm(fp6, 0, 0, FAKE, FAKE, None, 256, 256, 128, 0, 0, FAKE, 1 << 20) == 1
    assert "a_scale, b_scale, and out pointers must be non-null" in _err(lib)


def _ragged_f6(family, layout=kt.LAYOUT_NN, scale_mode=kt.SCALE_PER_CHANNEL):
    return next(d for d in kt.entries(family)
                if d.layout == layout and d.operand_format == kt.OPERANDS_FP6 and d.scale_mode == scale_mode)


def _ragged_ws(lib, index, m, n, k_packed, groups):
    out = ctypes.c_uint64(0)
    rc = lib.amd_strix_halo_kernels_ragged_workspace_bytes(index, m, n, k_packed, groups, ctypes.byref(out))
    return rc, int(out.value)


def test_fp6_ragged_entries_report_their_workspace(lib):
    for family in (kt.FAMILY_RAGGED_FWD, kt.FAMILY_RAGGED_BWD):
        fp6 = [d for d in kt.entries(family) if d.operand_format == kt.OPERANDS_FP6]
        layouts = [kt.LAYOUT_NN, kt.LAYOUT_NT, kt.LAYOUT_TN, kt.LAYOUT_TT]
        per_channel = [d for d in fp6 if d.scale_mode == kt.SCALE_PER_CHANNEL]
        sub = [d for d in fp6 if d.scale_mode == kt.SCALE_SUBCHANNEL]
        assert sorted(d.layout for d in per_channel) == layouts
        # and one fp6 subchannel entry per layout
        assert sorted(d.layout for d in sub) == layouts
        for d in fp6:
            if d.scale_mode == kt.SCALE_PER_CHANNEL:
                # 128 x 128 tiles, two 24 KiB stages of 128 K and the B-scale slots: three per CU
                assert (d.block_m, d.block_k, d.num_stages) == (128, 128, 2)
                assert d.lds_bytes == 50176
            else:
                # the subchannel engine: a ring of 64-K stages, groups of 32 to 256
                assert (d.block_m, d.block_n, d.min_subchannel, d.max_subchannel) == (128, 128, 32, 256)
                assert d.lds_bytes == 81920
            # the subchannel entries pad K to 256, the per-channel ones to 128
            step = 256 if d.scale_mode == kt.SCALE_SUBCHANNEL else 128
            for m, n, kp, g in ((8192, 1408, 1024, 8), (17, 24, 32, 3), (2048, 1408, 1001, 8), (1, 8, 1, 1)):
                kw = -(-2 * kp // step) * step
                m32, n32 = -(-m // 32) * 32, -(-n // 32) * 32
                if family == kt.FAMILY_RAGGED_FWD:
                    want = (m32 * kw + g * n32 * kw) * 3 // 4
                else:
                    want = g * (m32 * kw + n32 * kw) * 3 // 4
                assert _ragged_ws(lib, d.index, m, n, kp, g) == (0, want)
                assert d.ragged_workspace_bytes(m, n, kp, g) == want
    packed = next(d for d in kt.entries(kt.FAMILY_RAGGED_FWD) if not d.needs_workspace)
    assert _ragged_ws(lib, packed.index, 8192, 1408, 1024, 8) == (0, 0)
    dense = kt.entries(kt.FAMILY_DENSE)[0].index
    assert _ragged_ws(lib, dense, 16, 16, 16, 1)[0] == 1
    assert "not a ragged kernel" in _err(lib)


def test_fp6_ragged_launch_validation(lib):
    fwd = _ragged_f6(kt.FAMILY_RAGGED_FWD).index
    F = lib.amd_strix_halo_kernels_launch_ragged_fwd
    FW = lib.amd_strix_halo_kernels_launch_ragged_fwd_ws
    # 64 x 16 x 64 (k_packed 32), 2 groups: A 64 x 128 + 2 x (32 x 128) in fp6
    need = (64 * 128 + 2 * 32 * 128) * 3 // 4
    assert F(fwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 64, 16, 32, 2, 0, 0) == 1
    assert f"workspace of {need} bytes" in _err(lib)
    args = (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 64, 16, 32, 2, 0, 0)
    assert FW(fwd, 0, 0, *args, FAKE, need - 1) == 1
    assert f"workspace of {need} bytes" in _err(lib)
    assert FW(fwd, 0, 0, *args, FAKE + 4, need + 4) == 1
    assert "16-byte aligned" in _err(lib)
    assert FW(fwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 64, 12, 32, 2, 0, 0, FAKE, 1 << 30) == 1
    assert "N to be a multiple of 8" in _err(lib)
    assert FW(fwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE + 8, 64, 16, 32, 2, 0, 0, FAKE, 1 << 30) == 1
    assert "out must be 16-byte aligned" in _err(lib)
    assert FW(fwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 64, 16, kt.FP6_MAX_K // 2 + 64, 2, 0, 0,
              FAKE, 1 << 40) == 1
    assert "K <= 262144" in _err(lib)
    sub = _ragged_f6(kt.FAMILY_RAGGED_FWD, scale_mode=kt.SCALE_SUBCHANNEL).index
    # K 96: three groups of 32 per row, whose a_scale values do not pair up in dwords
    assert FW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 64, 16, 48, 2, 32, 0, FAKE, 1 << 30) == 1
    assert "ceil(K/32) to be even with subchannel 32; got 3" in _err(lib)
    # the subchannel forward pads K to 256: 64 x 16 x 64, 2 groups
    need_sub = (64 * 256 + 2 * 32 * 256) * 3 // 4
    assert FW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 64, 16, 32, 2, 64, 0, FAKE, need) == 1
    assert f"workspace of {need_sub} bytes" in _err(lib)
    assert FW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 64, 16, 128, 2, 16, 0, FAKE, 1 << 30) == 1
    assert "subchannel size 16 is not served" in _err(lib)
    assert FW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 63, 16, 384, 2, 256, 0, FAKE, 1 << 30) == 1
    assert "M * ceil(K/subchannel) to be even; got M=63, ceil(K/subchannel)=3" in _err(lib)
    bwd = _ragged_f6(kt.FAMILY_RAGGED_BWD, kt.LAYOUT_TN).index
    B = lib.amd_strix_halo_kernels_launch_ragged_bwd
    BW = lib.amd_strix_halo_kernels_launch_ragged_bwd_ws
    # 3 groups of 48 x 16 with K capacity 39 (k_packed 20 -> 128)
    need = 3 * (64 * 128 + 32 * 128) * 3 // 4
    assert B(bwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 20, 3, 0, 2, kt.OUT_F32) == 1
    assert f"workspace of {need} bytes" in _err(lib)
    assert BW(bwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 20, 3, 0, 1, kt.OUT_BF16, FAKE, need) == 1
    assert "fp32" in _err(lib)
    assert BW(bwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 20, 3, 64, 1, kt.OUT_F32, FAKE, need) == 1
    assert "subchannel = 0" in _err(lib)
    sub = _ragged_f6(kt.FAMILY_RAGGED_BWD, kt.LAYOUT_TN, scale_mode=kt.SCALE_SUBCHANNEL).index
    # the same call with K padded to 256
    need_sub = 3 * (64 * 256 + 32 * 256) * 3 // 4
    assert BW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 20, 3, 64, 1, kt.OUT_F32, FAKE, need) == 1
    assert f"workspace of {need_sub} bytes" in _err(lib)
    assert BW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 20, 3, 16, 1, kt.OUT_F32, FAKE, need_sub) == 1
    assert "subchannel size 16 is not served" in _err(lib)
    # K 72: three groups of 32 per row, whose a_scale values do not pair up in dwords
    assert BW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 36, 3, 32, 1, kt.OUT_F32, FAKE, need_sub) == 1
    assert "ceil(K/32) to be even with subchannel 32; got 3" in _err(lib)
    assert BW(sub, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 47, 16, 20, 3, 64, 1, kt.OUT_F32, FAKE, need_sub) == 1
    assert "M * ceil(K/subchannel) to be even; got M=47, ceil(K/subchannel)=1" in _err(lib)
    # nothing to run: no workspace needed
    assert BW(bwd, 0, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 48, 16, 20, 0, 0, 1, kt.OUT_F32, None, 0) == 0


def test_fp6_ragged_eligibility():
    fwd, bwd = kt.FAMILY_RAGGED_FWD, kt.FAMILY_RAGGED_BWD
    assert kt.ragged_fp6_eligible(fwd, subchannel=None, m=8192, n=1408, k_packed=1024)
    assert kt.ragged_fp6_eligible(bwd, subchannel=None, m=2048, n=1408, k_packed=1001)
    assert kt.ragged_fp6_eligible(fwd, subchannel=None, m=17, n=24, k_packed=32)
    # subchannel: any K (padded to 256), M * ceil(K/S) even, ceil(K/32) even for groups of 32
    assert kt.ragged_fp6_eligible(fwd, subchannel=32, m=8192, n=1408, k_packed=1024)
    assert kt.ragged_fp6_eligible(fwd, subchannel=128, m=18, n=24, k_packed=64)
    assert kt.ragged_fp6_eligible(fwd, subchannel=256, m=18, n=24, k_packed=128)
    assert kt.ragged_fp6_eligible(fwd, subchannel=256, m=17, n=24, k_packed=256)
    assert kt.ragged_fp6_eligible(fwd, subchannel=256, m=17, n=24, k_packed=192)  # 2 groups, the last half full
    assert kt.ragged_fp6_eligible(fwd, subchannel=64, m=8192, n=1408, k_packed=1056)
    assert kt.ragged_fp6_eligible(fwd, subchannel=32, m=8192, n=2880, k_packed=1440)  # K 2880: 90 groups
    assert not kt.ragged_fp6_eligible(fwd, subchannel=256, m=17, n=24, k_packed=128)  # M * K/S odd
    assert not kt.ragged_fp6_eligible(fwd, subchannel=32, m=18, n=24, k_packed=48)  # 3 groups of 32
    # the backward pads K: any capacity; groups of 32 need an even ceil(K/32)
    assert kt.ragged_fp6_eligible(bwd, subchannel=128, m=2048, n=1408, k_packed=1001)
    assert kt.ragged_fp6_eligible(bwd, subchannel=256, m=2048, n=1408, k_packed=50)
    assert kt.ragged_fp6_eligible(bwd, subchannel=32, m=2048, n=1408, k_packed=990)  # 62 groups
    assert not kt.ragged_fp6_eligible(bwd, subchannel=32, m=2048, n=1408, k_packed=1001)
    assert not kt.ragged_fp6_eligible(bwd, subchannel=64, m=17, n=24, k_packed=96)  # 17 * 3 scale columns
    assert not kt.ragged_fp6_eligible(bwd, subchannel=None, m=16, n=20, k_packed=16)
    assert not kt.ragged_fp6_eligible(fwd, subchannel=None, m=16, n=16, k_packed=kt.FP6_MAX_K // 2 + 1)
    with pytest.raises(LookupError):
        kt.find_ragged(bwd, layout=kt.LAYOUT_NN, subchannel=512, fp6=True)
    assert kt.find_ragged(bwd, layout=kt.LAYOUT_NN, subchannel=32, fp6=True).scale_mode == kt.SCALE_SUBCHANNEL
    assert kt.find_ragged(fwd, layout=kt.LAYOUT_NN, subchannel=32, fp6=True).scale_mode == kt.SCALE_SUBCHANNEL
    assert kt.find_ragged(fwd, layout=kt.LAYOUT_NN, subchannel=None, fp6=True).block_m == kt.RAGGED_FP6_BLOCK_M
    assert kt.find_ragged(bwd, layout=kt.LAYOUT_NN, subchannel=None).operand_format == kt.OPERANDS_PACKED
    assert kt.RAGGED_FP6_CONFIG_BLOCK_M not in kt.RAGGED_FWD_BLOCK_M


def test_quantize_validates_before_launch(lib):
    q = lib.amd_strix_halo_kernels_quantize

    def call(src=kt.SRC_BF16, rows=4, cols=8, ld_x=8, inv=10.0, bits=4, mode=kt.QUANT_PACK_COLS, out=FAKE, ld_out=4,
             x=FAKE):
        return q(0, 0, x, src, rows, cols, ld_x, inv, bits, mode, out, ld_out)

    for kwargs, msg in (
        (dict(src=9), b"unknown source"),
        (dict(mode=7), b"unknown quantize mode"),
        (dict(bits=6), b"bits must be 4 or 8"),
        (dict(bits=8), b"only int4 codes are packed"),
        (dict(src=kt.SRC_I8, mode=kt.QUANT_CODES, ld_out=8), b"codes already"),
        (dict(inv=0.0), b"inv_scale must be positive"),
        (dict(inv=float("nan")), b"inv_scale must be positive"),
        (dict(rows=-1), b"non-negative"),
        (dict(ld_x=7), b"ld_x must be at least cols"),
        (dict(ld_out=3), b"ld_out must be at least"),
        (dict(mode=kt.QUANT_PACK_ROWS, ld_out=7), b"ld_out must be at least"),
        (dict(x=None), b"non-null"),
        (dict(out=None), b"non-null"),
    ):
        assert call(**kwargs) == 1, kwargs
        assert msg in lib.amd_strix_halo_kernels_last_error(), (kwargs, lib.amd_strix_halo_kernels_last_error())
    # nothing to do: no pointer is touched
    assert call(rows=0, x=None, out=None) == 0
    assert call(cols=0, ld_x=0, ld_out=0, x=None, out=None) == 0
    # int8 codes are packed without a scale
    assert call(src=kt.SRC_I8, inv=0.0, x=None) == 1
    assert b"non-null" in lib.amd_strix_halo_kernels_last_error()


def test_split_k_entries_validate_before_launch(lib):
    """Split-K entries take float32 output, the NONE epilogue, K a multiple of
    BLOCK_K*SPLIT_K, and (subchannel) whole scale groups per K slice."""
    pc = _dense_index(dtype_bits=4, layout=kt.LAYOUT_NN, scale_mode=kt.SCALE_PER_CHANNEL, split_k=8, block_m=128)
    assert _gemm(lib, pc, 128, 128, 256, mode=kt.OUT_F32) == 1
    assert "BLOCK_K*SPLIT_K=512" in _err(lib)
    assert _gemm(lib, pc, 128, 128, 512, mode=kt.OUT_BF16) == 1
    assert "float32" in _err(lib)
    assert _gemm(lib, pc, 128, 128, 512, epi=kt.EPILOGUE_RELU2, mode=kt.OUT_F32) == 1
    assert "NONE epilogue" in _err(lib)
    sc = _dense_index(dtype_bits=4, layout=kt.LAYOUT_NN, scale_mode=kt.SCALE_SUBCHANNEL, split_k=2, block_m=64,
                      max_subchannel=256)
    assert _gemm(lib, sc, 64, 64, 384, sub=128, mode=kt.OUT_F32) == 1
    assert "K/SPLIT_K=192 is not divisible by SUBCHANNEL=128" in _err(lib)
