"""The hand-scheduled K loops never let the compiler touch a register of an
LDS read that is still in flight, or an asm MFMA's result before it has
arrived (tests/_asm_check.py).

A late LDS return into a register the compiler had already handed to
another value corrupted the ragged fp6 forward's B-scale address for 16
lanes of a wave, in a few tiles per call; the engines now name every
fragment register in their waits.  This test compiles each translation unit
that holds such a loop to gfx950 assembly (hipcc -S, as build.py compiles
it) and scans it.  CPU only; about a minute."""

from __future__ import annotations

import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from tests._asm_check import inflight_lds_hazards, sgpr_vmem_hazards

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "strix-halo-int4-gemms_amd"))

UNITS = ("dense_f6", "ragged_f6", "dense_dma_4_0", "dense_dma_4_1", "dense_dma_4_2", "dense_dma_8_0", "dense_dma_8_1",
         "dense_dma_8_2", "skinny_4_0", "skinny_4_1", "skinny_4_2", "skinny_8_0", "skinny_8_1", "skinny_8_2")
# every kernel unit (the SGPR-operand scan covers all of them)
ALL_UNITS = UNITS + ("dense_4_0", "dense_4_1", "dense_4_2", "dense_8_0", "dense_8_1", "dense_8_2", "f6pack", "quant",
                     "ragged_0", "ragged_1", "ragged_2", "ragged_3")


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    import build

    if shutil.which(build.hipcc()) is None and not Path(build.hipcc()).exists():
        pytest.skip("hipcc is not available")
    out = tmp_path_factory.mktemp("asm")
    units = {name: (src, extra) for name, src, extra in build.translation_units() if name in ALL_UNITS}
    assert set(units) == set(ALL_UNITS)

    def one(name):
        src, extra = units[name]
        dst = out / f"{name}.s"
        cmd = [build.hipcc(), *build.HIP_FLAGS, *extra, "--offload-device-only", "-S", str(src), "-o", str(dst)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return name, dst.read_text()

    with ThreadPoolExecutor(8) as ex:
        return dict(ex.map(one, ALL_UNITS))


@pytest.mark.parametrize("unit", UNITS)
def test_no_register_of_an_inflight_lds_read_is_touched(assembly, unit):
    found = inflight_lds_hazards(assembly[unit])
    assert not found, "\n".join(found[:10])


@pytest.mark.parametrize("unit", ALL_UNITS)
def test_asm_loads_wait_for_valu_written_sgprs(assembly, unit):
    """No asm vector-memory load (LDS-DMA) reads an SGPR or M0 fewer than 5
    wait states after a VALU instruction wrote it: a v_readlane_b32 reload
    of a spilled offset one wait state before an LDS-DMA load let the load
    use a stale offset, and a wave's B scales came out wrong."""
    found = sgpr_vmem_hazards(assembly[unit])
    assert not found, "\n".join(found[:10])


def _functions(asm: str):
    import re

    for m in re.finditer(r"^(_Z\S+):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        yield m.group(1), asm[m.end():end].splitlines()


def test_fp6_gemm_accumulators_are_written_only_by_mfmas(assembly):
    """In every fp6 GEMM kernel, nothing but MFMAs writes the accumulators
    between the first MFMA and the last: no VALU write or register copy of
    an AGPR (a VALU-written C operand after an earlier MFMA of the wave was
    read stale) and no scratch access (a spilled accumulator).  The
    persistent kernels, which run the K loop once per tile, keep their
    scratch under 64 bytes per lane."""
    import re

    checked = 0
    for name, lines in _functions(assembly["dense_f6"]):
        if "f6_gemm_kernel" not in name and "f6_gemm_persistent" not in name:
            continue
        mf = [i for i, line in enumerate(lines) if "v_mfma" in line]
        assert mf, name
        bad = [lines[i].strip() for i in range(mf[0], mf[-1])
               if re.search(r"v_accvgpr_(write|mov)|scratch_|^\s*v_\w+(_e\d+)?\s+a\[?\d", lines[i])
               and "v_mfma" not in lines[i]]
        assert not bad, (name, bad[:4])
        if "f6_gemm_persistent" in name:
            size = re.search(re.escape(name) + r"\.private_seg_size, (\d+)", assembly["dense_f6"])
            assert size and int(size.group(1)) < 64, (name, size and size.group(1))
        checked += 1
    assert checked >= 10


def test_the_sgpr_scan_finds_a_reload_before_an_asm_load():
    asm = "\n".join([
        "_Zk:", "v_readlane_b32 s8, v112, 14", ";;#ASMSTART", "s_nop 0",
        "buffer_load_dword v67, s[28:31], s8 offen lds", ";;#ASMEND",   # 1 wait state: stale s8
        "v_readlane_b32 s9, v112, 15", ";;#ASMSTART", "s_nop 4",
        "buffer_load_dword v67, s[28:31], s9 offen lds", ";;#ASMEND",   # 5 wait states: fine
        "v_readfirstlane_b32 s30, v1", "buffer_load_dword v2, s[28:31], 0 offen",  # compiler's own load: its job
    ])
    found = sgpr_vmem_hazards(asm)
    assert len(found) == 1 and "reads s8 1 wait states" in found[0]


def test_the_scan_finds_a_reuse_and_a_copy():
    asm = "\n".join([
        "_Zkern:",
        ";;#ASMSTART", "ds_read_b128 v[10:13], v1 offset:0", ";;#ASMEND",
        "v_mov_b32_e32 v20, v11",       # copy before the wait: stale
        "v_lshrrev_b32_e32 v12, 2, v0",  # reuse before the wait: clobbered
        "s_waitcnt lgkmcnt(0)",
        "v_mov_b32_e32 v21, v10",       # after the wait: fine
    ])
    found = inflight_lds_hazards(asm)
    assert len(found) == 2 and "v[11]" in found[0] and "v[12]" in found[1]
    # a counted wait that leaves the read outstanding does not retire it
    asm2 = "\n".join(["_Zk:", ";;#ASMSTART", "ds_read_b64 v[4:5], v1", ";;#ASMEND", "ds_read_b64 v[6:7], v1",
                      "s_waitcnt lgkmcnt(2)", "v_mov_b32_e32 v9, v4", "s_waitcnt lgkmcnt(1)", "v_mov_b32_e32 v9, v4"])
    assert len(inflight_lds_hazards(asm2)) == 1
    # an asm MFMA's result read 5 wait states later (s_nop 4), then after 22
    asm3 = "\n".join(["_Zm:", ";;#ASMSTART",
                       "v_mfma_f32_32x32x64_f8f6f4 v[2:17], v[20:25], v[30:35], v[2:17] cbsz:2 blgp:2",
                       ";;#ASMEND", "s_nop 4", "v_mov_b32_e32 v40, v5", "s_nop 7", "s_nop 7",
                       "v_mov_b32_e32 v41, v6"])
    found = inflight_lds_hazards(asm3)
    assert len(found) == 1 and "after 5 wait states" in found[0]
    # control flow: a loop laid out with its latch block before its header
    # (as the compiler rotates loops) waits on every real path
    asm4 = "\n".join(["_Zl:", ";;#ASMSTART", "ds_read_b128 v[10:13], v1", ";;#ASMEND", "s_branch .LBB0_2",
                       ".LBB0_1:", "v_mov_b32_e32 v20, v10", "s_cbranch_scc0 .LBB0_3",
                       ".LBB0_2:", "s_waitcnt lgkmcnt(0)", "s_branch .LBB0_1",
                       ".LBB0_3:", "s_endpgm"])
    assert inflight_lds_hazards(asm4) == []
    # ... while a path that skips the wait is found, whatever the layout
    asm5 = asm4.replace("s_branch .LBB0_2", "s_cbranch_vccz .LBB0_1\ns_branch .LBB0_2")
    found = inflight_lds_hazards(asm5)
    assert len(found) == 1 and "v[10]" in found[0]
    # a read retired by 15 younger LDS operations
    asm6 = "\n".join(["_Zq:", ";;#ASMSTART", "ds_read_b32 v10, v1", ";;#ASMEND"] + ["ds_read_b32 v11, v1"] * 15 +
                      ["v_mov_b32_e32 v20, v10"])
    assert inflight_lds_hazards(asm6) == []
    # ... but not while a scalar load (which may return out of order) is
    # pending: then neither a counted wait nor 15 younger operations retire it
    asm7 = "\n".join(["_Zs:", ";;#ASMSTART", "ds_read_b32 v10, v1", ";;#ASMEND", "s_load_dword s4, s[0:1], 0x0",
                       "ds_read_b32 v11, v1", "s_waitcnt lgkmcnt(1)", "v_mov_b32_e32 v20, v10"])
    found = inflight_lds_hazards(asm7)
    assert len(found) == 1 and "v[10]" in found[0]
    asm8 = "\n".join(["_Zt:", ";;#ASMSTART", "ds_read_b32 v10, v1", ";;#ASMEND", "s_load_dword s4, s[0:1], 0x0"] +
                      ["ds_read_b32 v11, v1"] * 15 + ["v_mov_b32_e32 v20, v10"])
    assert len(inflight_lds_hazards(asm8)) == 1
    assert inflight_lds_hazards(asm7.replace("lgkmcnt(1)", "lgkmcnt(0)")) == []
    # an in-flight fragment register used as an LDS address or as ds_write data
    asm9 = "\n".join(["_Zd:", ";;#ASMSTART", "ds_read_b64 v[10:11], v1", ";;#ASMEND", "ds_read_b32 v12, v10",
                       "ds_write_b32 v2, v11", "s_waitcnt lgkmcnt(0)", "ds_write_b32 v10, v11"])
    found = inflight_lds_hazards(asm9)
    assert len(found) == 2 and "v[10]" in found[0] and "v[11]" in found[1]
