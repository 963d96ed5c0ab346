"""Host-side checks of the skinny tiles: every dense shape the reference's
registry accepts is accepted here, the reference's small-M selection cases
hold, and the library's workspace sizes equal the Python mirror.

The reference's tile rule is restated below from registry.py:29-251 (seed
tiles, the 16/32-row and 128-column variants, split-K and persistent
variants) and template_config.py:22-38 (M % BLOCK_M, N % BLOCK_N,
K % (BLOCK_K * SPLIT_K), K % SUBCHANNEL).  This is test data: the product's
registry is built from the gfx950 kernel table instead.
"""

from __future__ import annotations

import ctypes
import itertools

import pytest

import amd_strix_halo_kernels as shk
from amd_strix_halo_kernels import kernel_table as kt
from amd_strix_halo_kernels import native

SMALL_M = (32, 16)  # ref registry.py:29
SMALL_N = (128,)  # ref registry.py:30
SPLITS = (1, 2, 4, 8)  # ref metadata.py:12


def _bm_variants(bm):
    return tuple(dict.fromkeys((bm, *SMALL_M)))


def _shape_variants(bm, bn):
    """(bm, bn) pairs of _tile_shape_variants (ref registry.py:48-59)."""
    return tuple((m, n) for m in _bm_variants(bm) for n in dict.fromkeys((bn, *SMALL_N)))


def reference_tiles(dtype, scale_mode, epilogue):
    """(block_m, block_n, block_k, split_k) of the reference's even-K tiles
    of one family (ref registry.py:112-176 and the variant helpers)."""
    tiles = []
    if dtype == "int4":
        if scale_mode == "sc":
            # _int4_subchannel_tile_variants: 64x128x128 (GM1 and GM4), 16/32/64 rows
            splits = SPLITS if epilogue == "none" else (1,)
            for s in splits:
                for m in _bm_variants(64):
                    tiles.append((m, 128, 128, s))
            return tiles
        base = {"swiglu": (128, 256, 32), "relu2": (64, 512, 32), "none": (64, 512, 32)}[epilogue]
        splits = SPLITS if epilogue == "none" else (1,)
        for s in splits:
            bm, bn, bk = base
            if s > 1:  # _int4_split_tile (registry.py:33-39)
                bn = min(bn, 256)
            for m, n in _shape_variants(bm, bn):
                tiles.append((m, n, bk, s))
        return tiles
    # int8: the same tiles for every scale spec
    if epilogue == "swiglu":  # _paired_n_tile_variants (registry.py:62-77)
        for bm, bn, bk in ((64, 128, 64), (64, 256, 32)):
            for m in _bm_variants(bm):
                tiles.append((m, bn, bk, 1))
        return tiles
    splits = SPLITS if epilogue == "none" else (1,)
    for s in splits:
        for m, n in _shape_variants(64, 256):
            tiles.append((m, n, 64, s))
    return tiles


def reference_accepts(tiles, m, n, k, sub, split):
    for bm, bn, bk, s in tiles:
        if s != split:
            continue
        if m % bm or n % bn or k % (bk * s):
            continue
        if sub and k % sub:
            continue
        return True
    return False


SCALES = (None, 32, 64, 128, 256)
M_GRID = (16, 32, 48, 64, 96, 128, 256)
N_GRID = (128, 256, 384, 512, 1024)
K_GRID = (32, 64, 96, 128, 256, 384, 512, 1024)


def _families():
    for dtype in ("int4", "int8"):
        for sub in SCALES:
            for epilogue in ("none", "relu2", "swiglu"):
                for split in (SPLITS if epilogue == "none" else (1,)):
                    yield dtype, sub, epilogue, shk.KernelSchedule.STANDARD, split
                    if dtype == "int4" and epilogue == "none":
                        # the persistent int4 tiles are the NONE tiles with one stage (registry.py:230-251)
                        yield dtype, sub, epilogue, shk.KernelSchedule.PERSISTENT, split


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_select_accepts_every_shape_the_reference_accepts(layout):
    """For every family (dtype, scale, epilogue, schedule, split_k) and every
    shape of the grid that one of the reference's tiles accepts, select()
    returns a kernel of that family whose table entry runs the shape."""
    checked = 0
    for dtype, sub, epilogue, schedule, split in _families():
        tiles = reference_tiles(dtype, "sc" if sub else "pc", epilogue)
        spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL) if sub is None else shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL,
                                                                                          sub)
        for m, n, k in itertools.product(M_GRID, N_GRID, K_GRID):
            if not reference_accepts(tiles, m, n, k, sub, split):
                continue
            kern = shk.default_registry.select(
                dtype=shk.OperandDType.INT4 if dtype == "int4" else shk.OperandDType.INT8, scale=spec,
                epilogue=shk.Epilogue(epilogue), m=m, n=n, k=k, layout=shk.GemmLayout(layout), split_k=split,
                schedule=schedule)
            assert kern.tile.split_k == split and kern.schedule is schedule and kern.scale == spec
            assert m % kern.tile.block_m == 0 and n % kern.tile.block_n == 0
            assert k % (kern.tile.block_k * kern.tile.split_k) == 0
            assert kt.TABLE[kern.table_index].supports_k(k)
            checked += 1
    assert checked > 10000


def test_reference_small_m_selection_cases():
    """ref tests/test_registry.py:206-227: M = 16, 32, 64 at N = 512, K = 32
    select a tile of exactly that height; SwiGLU at M = 32 as well."""
    pc = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL)
    for m in (16, 32, 64):
        kern = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=m,
                                           n=512, k=32)
        assert kern.tile.block_m == m
    kern = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.SWIGLU, m=32,
                                       n=256, k=32)
    assert kern.tile.block_m == 32
    # ref tests/test_registry.py:262-271: 17 x 129 fits no tile
    with pytest.raises(LookupError):
        shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=17, n=129,
                                    k=32)


def test_skinny_split_count_rule():
    """About 256 workgroups (one per CU), at least two stages per wave, at most 16 splits;
    int4 waves stay within 1023 stages of 128 K; subchannel tiles never
    split; without a workspace only the unsplit launch (or none)."""
    d = next(x for x in kt.TABLE if x.is_stream and x.block_m == 16 and x.dtype_bits == 4 and x.scale_mode == 0
             and x.epilogue_kind == kt.EPI_KIND_PLAIN and x.split_k == 1 and x.schedule == 0)
    assert kt.sk_split_count(d, 16, 8192, 8192) == 2  # 128 tiles, 64 stages
    assert kt.sk_split_count(d, 16, 64, 8192) == 8  # 64 stages: 2 per wave
    assert kt.sk_split_count(d, 256, 8192, 8192) == 1  # 2048 tiles
    assert kt.sk_split_count(d, 16, 64, 32) == 1
    long_k = 4 * 1023 * 128 + 128
    assert kt.sk_split_count(d, 16, 64, long_k, with_workspace=False) == 0
    assert kt.sk_split_count(d, 16, 64, 4 * 1023 * 128, with_workspace=False) == 1
    assert kt.sk_split_count(d, 4096, 8192, 1 << 24) == 64
    sc = next(x for x in kt.TABLE if x.is_stream and x.scale_mode == kt.SCALE_SUBCHANNEL)
    assert kt.sk_split_count(sc, 16, 64, 1 << 20) == 1 and sc.workspace_bytes(16, 64, 1 << 20) == 0
    # counters of 128 tiles, then 128 tiles x 2 splits x 4 output tiles x 1 KiB
    assert d.workspace_bytes(16, 8192, 8192) == 512 + 128 * 2 * 4 * 1024


def test_workspace_bytes_match_the_library():
    """amd_strix_halo_kernels_gemm_workspace_bytes equals the mirror for
    every skinny entry over split and unsplit shapes."""
    lib = native.load_dispatch_library()
    out = ctypes.c_uint64()
    for d in kt.TABLE:
        if not d.is_stream:
            continue
        for m, n, k in ((16, 8192, 8192), (64, 64, 32), (32, 128, 1 << 20), (64, 1024, 4096)):
            if m % d.block_m:
                continue
            assert lib.amd_strix_halo_kernels_gemm_workspace_bytes(d.index, m, n, k, ctypes.byref(out)) == 0
            assert out.value == d.workspace_bytes(m, n, k), (d, m, n, k)
