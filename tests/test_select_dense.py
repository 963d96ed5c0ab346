"""amd_strix_halo_kernels_select_dense: the registry's selection evaluated
by the library, for a bridge that keeps the reference's own registry.

The reference's registry hands its native bridge a gfx1151 KernelMetadata
(ref native.py:690-767) whose tile (e.g. 64x512x32, 128x256x32; ref
registry.py:112-176) has no gfx950 entry.  The C call maps the metadata's
family fields and the call's shape to the entry this package's
registry.select() picks; these CPU tests pin the two together over a grid of
families and shapes, errors included, and map metadata built with the
reference's tile seeds.
"""

from __future__ import annotations

import itertools

import pytest

import amd_strix_halo_kernels as shk
from amd_strix_halo_kernels import kernel_table as kt
from amd_strix_halo_kernels import native
from amd_strix_halo_kernels.metadata import KernelMetadata, TileConfig

_LAYOUT = {"nn": kt.LAYOUT_NN, "nt": kt.LAYOUT_NT, "tn": kt.LAYOUT_TN, "tt": kt.LAYOUT_TT}
_EPI = {"none": kt.EPILOGUE_NONE, "relu2": kt.EPILOGUE_RELU2, "swiglu": kt.EPILOGUE_SWIGLU}
SHAPES = [(16, 128, 32), (16, 8192, 8192), (32, 256, 96), (48, 512, 1024), (64, 128, 4096), (128, 1024, 512),
          (256, 256, 256), (512, 768, 2048), (1024, 4096, 4096), (8192, 8192, 8192), (17, 129, 65),
          (64, 64, 1 << 20), (4096, 16384, 4096)]


def _registry_pick(bits, layout, sub, epi, schedule, split, m, n, k):
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL) if sub == 0 else shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, sub)
    try:
        return shk.default_registry.select(
            dtype=shk.OperandDType.INT4 if bits == 4 else shk.OperandDType.INT8, scale=spec, epilogue=shk.Epilogue(epi),
            m=m, n=n, k=k, layout=shk.GemmLayout(layout), split_k=split or None,
            schedule=shk.KernelSchedule.PERSISTENT if schedule else shk.KernelSchedule.STANDARD).table_index
    except LookupError:
        return None


def _library_pick(bits, layout, sub, epi, schedule, split, m, n, k):
    try:
        return native.select_dense_index(dtype_bits=bits, layout=_LAYOUT[layout], subchannel=sub, epilogue=_EPI[epi],
                                         schedule=schedule, split_k=split, m=m, n=n, k=k)
    except RuntimeError as exc:
        assert "no kernel for" in str(exc)
        return None


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn", "tt"])
def test_library_selection_equals_the_registry(bits, layout):
    found = 0
    for sub, epi, schedule, split in itertools.product((0, 32, 128, 256), ("none", "relu2", "swiglu"), (0, 1),
                                                       (0, 1, 2, 4, 8)):
        for m, n, k in SHAPES:
            want = _registry_pick(bits, layout, sub, epi, schedule, split, m, n, k)
            got = _library_pick(bits, layout, sub, epi, schedule, split, m, n, k)
            assert got == want, (bits, layout, sub, epi, schedule, split, m, n, k)
            found += want is not None
    # TT has no dense entries (the reference rejects it, api.py:30-34): every request raises alike
    assert found == 0 if layout == "tt" else found > 50


def _foreign(bits, layout, sub, epi, tile, schedule="standard"):
    """A KernelMetadata as the reference's registry builds it for gfx1151."""
    dtype = shk.OperandDType.INT4 if bits == 4 else shk.OperandDType.INT8
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL) if sub is None else shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, sub)
    bm, bn, bk, split = tile
    return KernelMetadata(kernel_id=f"gfx1151_{dtype.value}_{layout}_bm{bm}_bn{bn}_bk{bk}_sk{split}", arch="gfx1151",
                          a_dtype=dtype, b_dtype=dtype, acc_dtype="int32",
                          output_dtype="float32" if split > 1 else "bfloat16", scale_dtype="bfloat16", scale=spec,
                          epilogue=shk.Epilogue(epi),
                          tile=TileConfig(bm, bn, bk, 8, 4, 2, 1, True, split), triton_kernel_name="triton_kernel",
                          layout=shk.GemmLayout(layout), schedule=shk.KernelSchedule(schedule))


@pytest.mark.parametrize("bits,sub,epi,tile,shape", [
    (4, None, "none", (64, 512, 32, 1), (8192, 8192, 8192)),      # ref registry.py:126-127
    (4, None, "none", (16, 512, 32, 1), (16, 8192, 8192)),        # its 16-row variant (registry.py:29)
    (4, None, "relu2", (64, 512, 32, 1), (128, 1024, 96)),
    (4, None, "swiglu", (128, 256, 32, 1), (256, 256, 4096)),     # ref registry.py:138-139
    (4, 256, "relu2", (64, 128, 128, 1), (4096, 16384, 4096)),    # the subchannel seed
    (4, None, "none", (64, 256, 32, 4), (256, 1024, 8192)),       # split-K (registry.py:33-39)
    (8, None, "swiglu", (64, 256, 32, 1), (4096, 11008, 4096)),   # ref registry.py:151-153
    (8, 64, "none", (32, 256, 64, 1), (32, 512, 256)),
])
def test_reference_tiles_map_to_the_registry_pick(bits, sub, epi, tile, shape):
    m, n, k = shape
    kernel = _foreign(bits, "nn", sub, epi, tile)
    index = native.index_for_foreign_kernel(kernel, m=m, n=n, k=k)
    assert index == _registry_pick(bits, "nn", sub or 0, epi, 0, tile[3], m, n, k)
    d = kt.TABLE[index]
    assert d.family == kt.FAMILY_DENSE and d.dtype_bits == bits and (d.split_k or 1) == tile[3]
    assert m % d.block_m == 0 and n % d.block_n == 0 and k % (d.block_k * max(1, d.split_k)) == 0


def test_persistent_reference_tile_maps_to_a_persistent_entry():
    kernel = _foreign(4, "nn", None, "none", (64, 512, 32, 1), schedule="persistent")
    d = kt.TABLE[native.index_for_foreign_kernel(kernel, m=8192, n=8192, k=8192)]
    assert d.schedule == kt.SCHEDULE_PERSISTENT


def test_selection_errors():
    with pytest.raises(RuntimeError, match="no kernel for"):
        native.select_dense_index(dtype_bits=4, layout=kt.LAYOUT_NN, subchannel=0, epilogue=kt.EPILOGUE_NONE,
                                  schedule=0, split_k=0, m=17, n=129, k=32)
    with pytest.raises(RuntimeError, match="subchannel must be"):
        native.select_dense_index(dtype_bits=4, layout=kt.LAYOUT_NN, subchannel=96, epilogue=kt.EPILOGUE_NONE,
                                  schedule=0, split_k=0, m=64, n=64, k=96)
    with pytest.raises(RuntimeError, match="dtype_bits"):
        native.select_dense_index(dtype_bits=6, layout=kt.LAYOUT_NN, subchannel=0, epilogue=kt.EPILOGUE_NONE,
                                  schedule=0, split_k=0, m=64, n=64, k=64)
