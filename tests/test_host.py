"""Host-side logic of the Python layer, on the CPU.

Covers what runs before any kernel: registry selection over the gfx950 table,
shape / scale / layout validation with the reference's messages, the loud
failure when no GPU path exists, the explicit use_reference numerical path
(checked against the oracle), the quantization helpers, the CPU task list and
the ragged configuration / eligibility predicates (mirroring
tests/test_quant.py, tests/test_api_shapes.py, tests/test_registry.py,
tests/test_template_config.py and tests/test_ragged_dot.py of the reference).
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import amd_strix_halo_kernels as shk  # noqa: E402
from amd_strix_halo_kernels import kernel_table as kt  # noqa: E402
from amd_strix_halo_kernels.ragged import _can_use_bwd_even_k_fast_path, _can_use_even_k_fast_path  # noqa: E402
from amd_strix_halo_kernels.template_config import (  # noqa: E402
    LaunchShape,
    representative_generation_shape,
    tile_multiple_rejection_reasons,
)
from oracle import ref  # noqa: E402
from tests._util import stable_seed  # noqa: E402

PC = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL)


def _bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------------------
# registry


def test_registry_is_built_from_the_table():
    kernels = shk.default_registry.all()
    assert len({k.kernel_id for k in kernels}) == len(kernels)
    dense = kt.entries(kt.FAMILY_DENSE)
    for k in kernels:
        d = kt.TABLE[k.table_index]
        assert d.family == kt.FAMILY_DENSE
        assert d.dtype_bits == (4 if k.a_dtype is shk.OperandDType.INT4 else 8)
        assert (d.block_m, d.block_n, d.block_k) == (k.tile.block_m, k.tile.block_n, k.tile.block_k)
        assert kt.LAYOUT_CODES[k.layout.value] == d.layout
        assert k.arch == "gfx950" and k.kernel_id.startswith("gfx950_")
        assert k.status is shk.KernelStatus.COMPILED
    assert {k.table_index for k in kernels} == {d.index for d in dense}


@pytest.mark.parametrize(
    "dtype,scale,epilogue,shape,tile",
    [
        (shk.OperandDType.INT4, PC, shk.Epilogue.NONE, (128, 1024, 64), (64, 64)),             # C1 (skinny)
        (shk.OperandDType.INT4, PC, shk.Epilogue.NONE, (8192, 8192, 8192), (256, 256)),        # C2
        (shk.OperandDType.INT4, shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 256), shk.Epilogue.RELU2,
         (4096, 16384, 4096), (128, 128)),                                                     # C3
        (shk.OperandDType.INT8, PC, shk.Epilogue.SWIGLU, (4096, 11008, 4096), (256, 128)),     # C4
        (shk.OperandDType.INT4, shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 64), shk.Epilogue.NONE,
         (4096, 4096, 4096), (128, 128)),
        (shk.OperandDType.INT4, shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 64), shk.Epilogue.NONE,
         (4096, 4096, 4160), (64, 64)),
        (shk.OperandDType.INT4, shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 32), shk.Epilogue.RELU2,
         (4096, 16384, 4096), (128, 128)),
        (shk.OperandDType.INT4, shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 128), shk.Epilogue.NONE,
         (64, 4096, 4096), (32, 16)),
        (shk.OperandDType.INT4, shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 128), shk.Epilogue.NONE,
         (576, 4096, 4096), (64, 64)),
    ],
)
def test_select_picks_the_fastest_then_the_largest_fitting_tile(dtype, scale, epilogue, shape, tile):
    """Measured MI355X throughput ranks first (C2-C4 pick the measured fp6
    and int8 32x32 entries, C1 the measured skinny tiles, the tallest of
    them, subchannel 32 and 64 the fp6 subchannel entry, subchannel M = 64
    the 32-row skinny subchannel tile, whose figure holds up to 256 rows), tile
    area next (subchannel 64 with K not a multiple of the 128-K tiles,
    subchannel M = 576)."""
    m, n, k = shape
    kernel = shk.default_registry.select(dtype=dtype, scale=scale, epilogue=epilogue, m=m, n=n, k=k)
    assert (kernel.tile.block_m, kernel.tile.block_n) == tile
    assert not tile_multiple_rejection_reasons(kernel, LaunchShape(m, n, k))
    fitting = [c for c in shk.default_registry.all() if c.scale == scale and c.epilogue is epilogue
               and c.a_dtype is dtype and c.layout is kernel.layout
               and not tile_multiple_rejection_reasons(c, LaunchShape(m, n, k))]
    assert (kt.selection_tops(kt.TABLE[kernel.table_index], m) or 0) == max(
        kt.selection_tops(kt.TABLE[c.table_index], m) or 0 for c in fitting)


def test_select_raises_for_shapes_no_kernel_accepts():
    with pytest.raises(LookupError, match="no kernel for dtype=int4"):
        shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=PC, epilogue=shk.Epilogue.NONE,
                                    m=100, n=64, k=64)
    with pytest.raises(LookupError):
        shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=PC, epilogue=shk.Epilogue.NONE,
                                    m=24, n=64, k=64, schedule=shk.KernelSchedule.PERSISTENT)
    with pytest.raises(LookupError):  # K a multiple of 32 only
        shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=PC, epilogue=shk.Epilogue.NONE,
                                    m=16, n=64, k=48)


def test_select_knows_each_entry_k_bound():
    """K past an entry's gfx950 bound is never selected: int4 per-channel K
    of 131072 and above skips the int8 engines' unsplit tiles (x16-widened int32
    accumulators) for a split-K, skinny (K split over workgroups) or fp6
    entry, K above 262144 runs on the fp6
    tile in K slices, and past 2^24 no kernel fits (LookupError, the
    registry's contract for an unserved shape)."""
    pc = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL)
    for m, n, k in ((128, 128, 196608), (256, 256, 524288), (256, 256, kt.FP6_MAX_K_SLICED)):
        kern = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=m, n=n,
                                           k=k)
        assert kt.TABLE[kern.table_index].supports_k(k), kern.kernel_id
    kern = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=128,
                                       n=128, k=196608)
    assert kern.tile.split_k > 1 or kt.TABLE[kern.table_index].is_stream
    kern = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=256,
                                       n=256, k=524288)
    assert kt.TABLE[kern.table_index].operand_format == kt.OPERANDS_FP6
    with pytest.raises(LookupError):
        shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=256, n=256,
                                    k=kt.FP6_MAX_K_SLICED + 128)
    # the persistent fp6 tile multiplies K <= 262144 in one pass; the skinny
    # persistent tiles take longer K (split over workgroups), up to 2^24
    kern = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=256,
                                       n=256, k=524288, schedule=shk.KernelSchedule.PERSISTENT)
    assert kt.TABLE[kern.table_index].operand_format == kt.OPERANDS_STREAM
    with pytest.raises(LookupError):
        shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=pc, epilogue=shk.Epilogue.NONE, m=256, n=256,
                                    k=kt.FP6_MAX_K_SLICED + 128, schedule=shk.KernelSchedule.PERSISTENT)
    assert not shk.kernel_supports_shape(
        next(k for k in shk.default_registry.all() if k.table_index is not None
             and kt.TABLE[k.table_index].max_k == kt.INT4_ACC_MAX_K), m=256, n=256, k=262144)


def test_select_reference_ignores_shape():
    k = shk.default_registry.select_reference(dtype=shk.OperandDType.INT8, scale=PC, epilogue=shk.Epilogue.RELU2)
    assert k.epilogue is shk.Epilogue.RELU2 and k.tile.split_k == 1


def test_measured_tops_overrides_tile_size():
    reg = shk.default_registry
    small = reg.select(dtype=shk.OperandDType.INT4, scale=PC, epilogue=shk.Epilogue.NONE, m=64, n=64, k=64)
    top = max(k.measured_tops or 0.0 for k in reg.all())
    bumped = reg.with_status(small.kernel_id, shk.KernelStatus.BENCHMARKED, measured_tops=top + 1.0)
    pick = bumped.select(dtype=shk.OperandDType.INT4, scale=PC, epilogue=shk.Epilogue.NONE, m=256, n=256, k=128)
    assert pick.kernel_id == small.kernel_id


def test_tile_multiple_messages():
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=PC, epilogue=shk.Epilogue.NONE,
                                         m=8192, n=8192, k=8192)
    reasons = tile_multiple_rejection_reasons(kernel, LaunchShape(100, 200, 300))
    assert reasons == (
        "M=100 is not divisible by BLOCK_M=256",
        "N=200 is not divisible by BLOCK_N=256",
        "K=300 is not divisible by BLOCK_K*SPLIT_K=128",
    )
    with pytest.raises(ValueError, match="requires tile-multiple shape"):
        LaunchShape(100, 256, 128).validate_for(kernel)
    shape = representative_generation_shape(kernel)
    assert (shape.m, shape.n, shape.k) == (256, 256, 128)


# ---------------------------------------------------------------------------
# API validation (raises before any launch)


def _i8(*shape):
    return torch.zeros(shape, dtype=torch.int8)


def test_mm_rejects_swiglu_and_tt():
    with pytest.raises(ValueError, match="fused_swiglu_up_gate"):
        shk.mm(_i8(64, 32), _i8(32, 512), dtype=shk.OperandDType.INT8, epilogue=shk.Epilogue.SWIGLU,
               use_reference=True)
    with pytest.raises(ValueError, match="unsupported GEMM layout tt"):
        shk.fused_swiglu_up_gate(_i8(64, 32), _i8(32, 512), dtype=shk.OperandDType.INT8,
                                 layout=shk.GemmLayout.TT, use_reference=True)


def test_k_mismatch_and_odd_swiglu():
    with pytest.raises(ValueError, match="logical K mismatch"):
        shk.mm(torch.zeros((64, 16), dtype=torch.uint8), torch.zeros((8, 64), dtype=torch.uint8), use_reference=True)
    with pytest.raises(ValueError, match="even"):
        shk.fused_swiglu_up_gate(_i8(64, 32), _i8(32, 511), dtype=shk.OperandDType.INT8, use_reference=True)


def test_subchannel_rhs_scale_layout_is_checked():
    # tests/test_api_shapes.py:87-104
    with pytest.raises(ValueError, match="weight-matched layout"):
        shk.mm(shk.pack_int4_k_major(_i8(32, 64)),
               shk.pack_int4_k_major(_i8(128, 64)).t().contiguous(),
               a_scale=torch.ones((32, 2), dtype=torch.bfloat16),
               b_scale=torch.ones((128, 2), dtype=torch.bfloat16),
               scale=shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 32), use_reference=True)


def test_swiglu_rejects_external_gate():
    kernel = shk.default_registry.select_reference(dtype=shk.OperandDType.INT8, scale=PC,
                                                   epilogue=shk.Epilogue.SWIGLU)
    with pytest.raises(ValueError, match="fused up/gate"):
        shk.explicit_mm(_i8(64, 32), _i8(32, 128), kernel=kernel, gate=torch.zeros((64, 64)), use_reference=True)


def test_native_path_fails_loudly_without_a_gpu():
    if torch.cuda.is_available():
        pytest.skip("this host has a GPU")
    a = shk.pack_int4_k_major(_i8(64, 64))
    b = shk.pack_int4_k_major(_i8(64, 64)).t().contiguous()
    with pytest.raises(RuntimeError, match="CUDA/HIP"):
        shk.mm(a, b, a_scale=torch.ones(64, dtype=torch.bfloat16), b_scale=torch.ones(64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CUDA/HIP tensor"):
        shk.ragged_dot_int4(torch.zeros((8, 16), dtype=torch.uint8), torch.zeros((2, 16, 8), dtype=torch.uint8),
                            torch.tensor([4, 4]))


# ---------------------------------------------------------------------------
# use_reference vs the oracle (tests/test_api_shapes.py:47-165)


@pytest.mark.parametrize(
    "bits,scale,epilogue,shape",
    [
        (4, None, "none", (128, 512, 64)),
        (4, None, "relu2", (128, 512, 64)),
        (4, 128, "none", (128, 1024, 128)),
        (8, None, "relu2", (64, 512, 48)),
        (8, 64, "none", (128, 1024, 64)),
        (4, 32, "none", (17, 129, 65)),
        (4, 32, "swiglu", (64, 512, 66)),
        (8, None, "swiglu", (64, 512, 48)),
        (8, 256, "swiglu", (64, 512, 272)),
    ],
)
def test_use_reference_matches_oracle(bits, scale, epilogue, shape):
    m, n, k = shape
    r = ref.rng(stable_seed(bits, scale, epilogue, shape))
    b_cols = 2 * n if epilogue == "swiglu" else n
    a_q = ref.randn_bf16_fake_quant(r, (m, k), bits=bits)
    b_q = ref.randn_bf16_fake_quant(r, (k, b_cols), bits=bits)
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=bits, layout="nn")
    if scale:
        cols = -(-k // scale)
        sa = ref.uniform_bf16(r, (m, cols), 0.8, 1.2)
        sb = ref.uniform_bf16(r, (cols, b_cols), 0.85, 1.15)
        spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, scale)
    else:
        sa = ref.uniform_bf16(r, (m,), 0.75, 1.25)
        sb = ref.uniform_bf16(r, (b_cols,), 0.9, 1.1)
        spec = PC
    dtype = shk.OperandDType.INT4 if bits == 4 else shk.OperandDType.INT8
    args = dict(a_scale=_bf16(sa), b_scale=_bf16(sb), dtype=dtype, scale=spec, use_reference=True)
    if epilogue == "swiglu":
        out = shk.fused_swiglu_up_gate(torch.from_numpy(a_arg), torch.from_numpy(b_arg), **args)
    else:
        out = shk.mm(torch.from_numpy(a_arg), torch.from_numpy(b_arg), epilogue=shk.Epilogue(epilogue), **args)
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, a_scale=sa, b_scale=sb, subchannel=scale,
                                   epilogue=epilogue)
    d = ref.bf16_ulp_diff(_bits(out), want)
    assert d.max() <= (1 if epilogue == "swiglu" else 0)


def test_use_reference_layouts_agree():
    # tests/test_quant.py:193-208
    r = ref.rng(9)
    a = ref.randn_bf16_fake_quant(r, (64, 32), bits=8)
    b = ref.randn_bf16_fake_quant(r, (32, 512), bits=8)
    a, b = torch.from_numpy(a), torch.from_numpy(b)
    kw = dict(dtype=shk.OperandDType.INT8, use_reference=True)
    nn = shk.mm(a, b, **kw)
    assert torch.equal(shk.mm(a, b.t().contiguous(), layout=shk.GemmLayout.NT, **kw), nn)
    assert torch.equal(shk.mm(a.t().contiguous(), b, layout=shk.GemmLayout.TN, **kw), nn)


# ---------------------------------------------------------------------------
# quantization helpers vs the oracle (quant.py)


def test_quant_helpers_match_oracle():
    r = ref.rng(12)
    x = (r.standard_normal((16, 37)) * 0.3).astype(np.float32)
    for bits in (4, 8):
        got = shk.fake_quant_int(torch.from_numpy(x), bits=bits, scale=0.1).numpy()
        assert np.array_equal(got, ref.fake_quant_int(x, bits=bits, scale=0.1))
    q = ref.randint4(r, (5, 37))
    p = shk.pack_int4_k_major(torch.from_numpy(q)).numpy()
    assert np.array_equal(p, ref.pack_int4_k_major(q))
    assert np.array_equal(shk.unpack_int4_k_major(torch.from_numpy(p)).numpy(), ref.unpack_int4_k_major(p))
    with pytest.raises(ValueError, match="scale must be positive"):
        shk.fake_quant_int(torch.ones(2), bits=4, scale=0.0)
    with pytest.raises(TypeError, match="scalar"):
        shk.fake_quant_int(torch.ones(2), bits=4, scale=torch.ones(2))
    s = torch.arange(24, dtype=torch.bfloat16).reshape(2, 3, 4)
    assert torch.equal(shk.pack_rhs_subchannel_scales(s), s.transpose(-2, -1).contiguous())
    with pytest.raises(ValueError, match="\\(G, N, scale_cols\\)"):
        shk.pack_ragged_rhs_subchannel_scales(torch.ones(3, 4))


def test_tops_known_answer():
    assert shk.tops_for_runtime(shk.BenchmarkShape(1024, 1024, 1024), 1.0) == pytest.approx(2.147483648)


# ---------------------------------------------------------------------------
# ragged host logic


def test_group_info_cpu_matches_oracle():
    cases = [([17, 31, 24], 32, None, 8), ([2, 0, 7], 16, 4, 8), ([300, 0, 1000, 17, 2779], 64, None, 8),
             ([], 16, 3, 8), ([0, 0], 16, None, 8)]
    r = ref.rng(4)
    cases += [(r.integers(0, 150, size=int(r.integers(1, 9))).tolist(), int(r.choice([16, 32, 64])), None,
               int(r.choice([4, 8]))) for _ in range(20)]
    for sizes, tile, tid, align in cases:
        info = shk.calculate_group_info(torch.tensor(sizes, dtype=torch.int32), tile, tid_size=tid, align_tile=align)
        want = ref.calculate_group_info(np.array(sizes, dtype=np.int64), tile, tid_size=tid, align_tile=align)
        assert info.num_tasks == want.num_tasks
        for f in ("group_id", "block_start", "actual_start", "actual_end", "start_within_block", "actual_size"):
            assert np.array_equal(getattr(info, f).numpy(), getattr(want, f)), (sizes, f)


def test_group_info_validation():
    with pytest.raises(ValueError, match="tid_size must be at least 3"):
        shk.calculate_group_info(torch.tensor([17, 31, 24]), 32, tid_size=2)
    with pytest.raises(ValueError, match="1D"):
        shk.calculate_group_info(torch.zeros((2, 2), dtype=torch.int32), 16)
    with pytest.raises(ValueError, match="integer dtype"):
        shk.calculate_group_info(torch.zeros(3), 16)
    with pytest.raises(ValueError, match="multiple of align_tile"):
        shk.calculate_group_info(torch.tensor([1, 2]), 12, align_tile=8)
    with pytest.raises(TypeError):
        shk.calculate_group_info([1, 2], 16)


def test_ragged_configs_validate():
    with pytest.raises(ValueError, match="group_size_tasks must be positive"):
        shk.RaggedDotConfig(group_size_tasks=0)
    with pytest.raises(ValueError, match="block_k must be even"):
        shk.RaggedDotConfig(block_k=33)
    with pytest.raises(ValueError, match="multiple of align_tile"):
        shk.RaggedDotConfig(block_m=12)
    with pytest.raises(ValueError, match="split_k must be positive"):
        shk.RaggedBwdDotConfig(split_k=0)


def test_even_k_eligibility_predicates():
    # tests/test_ragged_dot.py:175-237
    cfg = shk.RaggedDotConfig(block_m=16, block_n=32, block_k=32)
    assert _can_use_even_k_fast_path(logical_k=64, scale=PC, config=cfg)
    assert not _can_use_even_k_fast_path(logical_k=48, scale=PC, config=cfg)
    assert _can_use_even_k_fast_path(logical_k=64, scale=shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 32), config=cfg)
    assert not _can_use_even_k_fast_path(logical_k=96, scale=shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 64), config=cfg)
    bcfg = shk.RaggedBwdDotConfig(block_k=16)
    sc32 = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 32)
    assert _can_use_bwd_even_k_fast_path(torch, group_sizes=torch.tensor([32, 0, 64]), scale=PC, config=bcfg)
    assert not _can_use_bwd_even_k_fast_path(torch, group_sizes=torch.tensor([32, 7, 64]), scale=PC, config=bcfg)
    assert _can_use_bwd_even_k_fast_path(torch, group_sizes=torch.tensor([32, 0, 64]), scale=sc32, config=bcfg)
    assert not _can_use_bwd_even_k_fast_path(torch, group_sizes=torch.tensor([16, 0, 32]), scale=sc32, config=bcfg)
    assert not _can_use_bwd_even_k_fast_path(
        torch, group_sizes=torch.tensor([32, 0, 64]), scale=PC,
        config=shk.RaggedBwdDotConfig(block_k=16, enable_even_k_fast_path=False))


def test_public_api_surface():
    for name in ("mm", "fused_swiglu_up_gate", "explicit_mm", "ragged_dot_int4", "ragged_dot_int4_bwd",
                 "calculate_group_info", "RaggedDotConfig", "RaggedBwdDotConfig", "RaggedGroupInfo",
                 "KernelRegistry", "default_registry", "KernelMetadata", "TileConfig", "ScaleSpec",
                 "dispatch_runtime_status", "launch_generated_kernel"):
        assert hasattr(shk, name), name
    assert shk.ARCH == "gfx950" and shk.ACC_DTYPE == "int32"
    assert shk.SUPPORTED_SUBCHANNELS == (32, 64, 128, 256)
    assert [layout.value for layout in shk.SUPPORTED_GEMM_LAYOUTS] == ["nn", "nt", "tn"]


# ---------------------------------------------------------------------------
# torch custom op (torch_ops.py of the reference)


def _logical_operand_shapes(kernel, m, n, k):
    packed = kernel.a_dtype is shk.OperandDType.INT4
    kk = k // 2 if packed else k
    b_cols = 2 * n if kernel.epilogue is shk.Epilogue.SWIGLU else n
    a_shape = (kk, m) if kernel.layout is shk.GemmLayout.TN else (m, kk)
    b_shape = (b_cols, kk) if kernel.layout is shk.GemmLayout.NT else (kk, b_cols)
    return a_shape, b_shape, torch.uint8 if packed else torch.int8


def test_torch_op_registers_once_and_fakes_every_layout():
    from torch._subclasses.fake_tensor import FakeTensorMode

    shk.register_torch_ops()
    shk.register_torch_ops()
    assert shk.TORCH_GEMM_OP == "amd_strix_halo_kernels::gemm"
    assert hasattr(torch.ops.amd_strix_halo_kernels, "gemm")
    seen = set()
    for kernel in shk.default_registry.all():
        key = (kernel.a_dtype, kernel.layout, kernel.epilogue, kernel.scale.mode)
        if key in seen:
            continue
        seen.add(key)
        shape = representative_generation_shape(kernel)
        m, n, k = shape.m, shape.n, shape.k
        a_shape, b_shape, dtype = _logical_operand_shapes(kernel, m, n, k)
        with FakeTensorMode():
            a = torch.empty(a_shape, device="cuda", dtype=dtype)
            b = torch.empty(b_shape, device="cuda", dtype=dtype)
            sa = torch.empty((m,), device="cuda", dtype=torch.bfloat16)
            sb = torch.empty((n,), device="cuda", dtype=torch.bfloat16)
            out = shk.torch_gemm(a, b, kernel=kernel, a_scale=sa, b_scale=sb)
            assert tuple(out.shape) == (m, n), kernel.kernel_id
            want = torch.bfloat16 if kernel.output_dtype == "bfloat16" else torch.float32
            assert out.dtype == want and out.device.type == "cuda", kernel.kernel_id
    assert len(seen) >= 8


def test_persistent_schedule_selection():
    """The persistent schedule serves int4 with the NONE epilogue for every
    scale mode and layout, and nothing else (reference registry.py:230-251)."""
    for layout in (shk.GemmLayout.NN, shk.GemmLayout.NT, shk.GemmLayout.TN):
        for spec in (PC, *(shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, s) for s in (32, 64, 128, 256))):
            k = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=spec, epilogue=shk.Epilogue.NONE,
                                            layout=layout, m=1024, n=1024, k=1024,
                                            schedule=shk.KernelSchedule.PERSISTENT)
            assert k.schedule is shk.KernelSchedule.PERSISTENT and "_none_persistent_" in k.kernel_id
            assert k.kernel_id.startswith(f"gfx950_int4xint4_{layout.value}_{spec.label}_none_persistent_")
    for dtype, epilogue in ((shk.OperandDType.INT4, shk.Epilogue.RELU2), (shk.OperandDType.INT8, shk.Epilogue.NONE)):
        with pytest.raises(LookupError):
            shk.default_registry.select(dtype=dtype, scale=PC, epilogue=epilogue, m=1024, n=1024, k=1024,
                                        schedule=shk.KernelSchedule.PERSISTENT)
    # the standard schedule never picks a persistent kernel
    assert all(k.schedule is shk.KernelSchedule.STANDARD for k in (
        shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=PC, epilogue=shk.Epilogue.NONE,
                                    m=8192, n=8192, k=8192),))
