"""GPU parity of the dense path (mm / fused_swiglu_up_gate / explicit_mm)
against the CPU oracle.

Bar: the int32 accumulators are bit-exact against the
integer matmul; bf16 outputs are within 2 bf16 ulp of the oracle (per-channel
and subchannel NONE / RELU2 come out bit-identical; SwiGLU may differ by an
ulp through exp).  Mirrors the reference's every-registry-kernel check
(tests/test_native_generated.py:74-108) and adds the benchmark configs C2-C4 at full
size, every output checked.
"""

from __future__ import annotations

import math
import numpy as np
import pytest

from oracle import ref
from tests._util import bf16_bits, dense_case, max_ulp, stable_seed, to_dev

torch = pytest.importorskip("torch")

import amd_strix_halo_kernels as shk  # noqa: E402
from amd_strix_halo_kernels import kernel_table as kt  # noqa: E402
from amd_strix_halo_kernels import native  # noqa: E402
from amd_strix_halo_kernels.template_config import representative_generation_shape  # noqa: E402

pytestmark = pytest.mark.gpu

# split-K kernels write fp32 sums of K slices; tests/test_gpu_splitk.py covers them
_UNSPLIT = tuple(k for k in shk.default_registry.all() if k.tile.split_k == 1)

ULP_TOL = 2


def _run_kernel(kernel, a_arg, b_arg, sa, sb, device):
    a = to_dev(torch, a_arg, device)
    b = to_dev(torch, b_arg, device)
    ta = to_dev(torch, sa, device)
    tb = to_dev(torch, sb, device)
    out = shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    return bf16_bits(torch, out), raw.cpu().numpy()


def _kernel_params(kernel):
    bits = 4 if kernel.a_dtype is shk.OperandDType.INT4 else 8
    sub = kernel.scale.subchannel_size if kernel.scale.mode is shk.ScaleMode.SUBCHANNEL else None
    return bits, kernel.layout.value, sub, kernel.epilogue.value


@pytest.mark.parametrize("kernel", _UNSPLIT, ids=lambda k: k.kernel_id)
def test_every_registry_kernel_matches_oracle(kernel, device):
    bits, layout, sub, epi = _kernel_params(kernel)
    shape = representative_generation_shape(kernel)
    k = max(shape.k, 2 * kernel.tile.block_k)  # at least two K stages
    if sub:
        k = -(-k // sub) * sub
    m, n = 2 * shape.m, 2 * shape.n  # several tiles
    seed = stable_seed(kernel.kernel_id)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=epi == "swiglu")
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, ref.int_matmul(a_q, b_q)), "int32 accumulators differ"
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, layout=layout, a_scale=sa, b_scale=sb,
                                   subchannel=sub, epilogue=epi)
    if epi == "swiglu":
        assert max_ulp(got, want) <= ULP_TOL
    else:
        assert np.array_equal(got, want)


def _odd_stage_k(kernel):
    """Three K periods of the kernel (block_k, or the least common multiple
    with the sub-channel group), when that is an odd number of K blocks."""
    bk = kernel.tile.block_k * kernel.tile.split_k
    sub = kernel.scale.subchannel_size if kernel.scale.mode is shk.ScaleMode.SUBCHANNEL else None
    unit = math.lcm(bk, sub) if sub else bk
    return 3 * unit if (3 * unit // bk) % 2 == 1 else None


@pytest.mark.parametrize("kernel", [k for k in _UNSPLIT if _odd_stage_k(k)],
                         ids=lambda k: k.kernel_id)
def test_every_registry_kernel_odd_stage_count(kernel, device):
    """Pipelined kernels run K blocks in pairs; an odd count ends on a single
    block, which must not multiply a stale ring slot."""
    bits, layout, sub, epi = _kernel_params(kernel)
    shape = representative_generation_shape(kernel)
    k = _odd_stage_k(kernel)
    m, n = 2 * shape.m, 2 * shape.n
    seed = stable_seed(kernel.kernel_id, "odd")
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=epi == "swiglu")
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, ref.int_matmul(a_q, b_q)), "int32 accumulators differ"
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, layout=layout, a_scale=sa, b_scale=sb,
                                   subchannel=sub, epilogue=epi)
    if epi == "swiglu":
        assert max_ulp(got, want) <= ULP_TOL
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("scale", ["pc", "sc32", "sc64", "sc128", "sc256"])
@pytest.mark.parametrize("epilogue", ["none", "relu2", "swiglu"])
def test_surface_api_matches_oracle(bits, layout, scale, epilogue, device):
    m, n, k = 256, 256, 512
    sub = None if scale == "pc" else int(scale[2:])
    seed = stable_seed(bits, layout, scale, epilogue)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=epilogue == "swiglu")
    dtype = shk.OperandDType.INT4 if bits == 4 else shk.OperandDType.INT8
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL) if sub is None else shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, sub)
    lay = shk.GemmLayout(layout)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    print(f"case bits={bits} {layout} {scale} {epilogue}", flush=True)
    if epilogue == "swiglu":
        out = shk.fused_swiglu_up_gate(a, b, a_scale=ta, b_scale=tb, dtype=dtype, layout=lay, scale=spec)
    else:
        out = shk.mm(a, b, a_scale=ta, b_scale=tb, dtype=dtype, layout=lay, scale=spec,
                     epilogue=shk.Epilogue(epilogue))
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (m, n)
    got = bf16_bits(torch, out)
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, layout=layout, a_scale=sa, b_scale=sb, subchannel=sub,
                                   epilogue=epilogue)
    if epilogue == "swiglu":
        assert max_ulp(got, want) <= ULP_TOL
    else:
        assert np.array_equal(got, want)


def test_config_c1_plumbing_exact(device):
    """C1: 128x1024x64 int4 per-channel, randn*0.1 fake-quantized, unit scales."""
    r = ref.rng(1)
    a_q = ref.randn_bf16_fake_quant(r, (128, 64), bits=4)
    b_q = ref.randn_bf16_fake_quant(r, (64, 1024), bits=4)
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=4, layout="nn")
    sa = ref.bf16_from_f32(np.ones(128))
    sb = ref.bf16_from_f32(np.ones(1024))
    out = shk.mm(to_dev(torch, a_arg, device), to_dev(torch, b_arg, device), a_scale=to_dev(torch, sa, device),
                 b_scale=to_dev(torch, sb, device))
    got = bf16_bits(torch, out)
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, a_scale=sa, b_scale=sb)
    assert np.array_equal(got, want)
    # unit scales: the output is the integer matmul, rounded to bf16
    assert np.array_equal(got, ref.bf16_round(ref.int_matmul(a_q, b_q).astype(np.float32)))


def _big_dense(device, *, bits, m, n, k, sub, epilogue, seed, scale_lo=0.005, scale_hi=0.02):
    """A benchmark config at full size through mm / fused_swiglu_up_gate, with
    every output checked: the raw int32 accumulators against the C oracle's
    exact integer matmul, and the bf16 result against the oracle's whole
    dense path (the C restatement for int4 NONE / RELU2, numpy for SwiGLU)."""
    from oracle import native as oracle_native

    if not oracle_native.available():
        from oracle import build as obuild

        obuild.build(verbose=False)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout="nn", m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=epilogue == "swiglu", scale_lo=scale_lo,
                                                 scale_hi=scale_hi)
    dtype = shk.OperandDType.INT4 if bits == 4 else shk.OperandDType.INT8
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL) if sub is None else shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, sub)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    if epilogue == "swiglu":
        kernel = shk.default_registry.select(dtype=dtype, scale=spec, epilogue=shk.Epilogue.SWIGLU, m=m, n=n, k=k)
        out = shk.fused_swiglu_up_gate(a, b, a_scale=ta, b_scale=tb, dtype=dtype, scale=spec)
    else:
        kernel = shk.default_registry.select(dtype=dtype, scale=spec, epilogue=shk.Epilogue(epilogue), m=m, n=n,
                                             k=k)
        out = shk.mm(a, b, a_scale=ta, b_scale=tb, dtype=dtype, scale=spec, epilogue=shk.Epilogue(epilogue))
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    got = bf16_bits(torch, out)
    del out, a, b
    raw_np = raw.cpu().numpy()
    del raw
    assert np.array_equal(raw_np, oracle_native.matmul_i8(a_q, b_q)), "int32 accumulators differ"
    del raw_np
    if epilogue == "swiglu":
        want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, a_scale=sa, b_scale=sb, subchannel=sub,
                                       epilogue=epilogue)
    else:
        assert bits == 4
        want = oracle_native.dense_int4_nn(a_arg, b_arg, sa, sb, m=m, n=n, k=k, subchannel=sub or 0,
                                           epilogue=1 if epilogue == "relu2" else 0)
    return got, want, kernel


def test_config_c2_8192_cubed(device):
    got, want, kernel = _big_dense(device, bits=4, m=8192, n=8192, k=8192, sub=None, epilogue="none", seed=2)
    assert kernel.tile.block_m == 256 and kernel.tile.block_n == 256
    assert got.shape == (8192, 8192)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("sub", [256, 128, 64, 32])
def test_config_c3_subchannel_relu2(sub, device):
    """C3 at full size, every output checked, for every group size the fp6
    subchannel tile serves (256 is the C3 config): 16 to 128 groups
    folded in order, groups of 32 two to a 64-K stage."""
    print(f"case C3 shape subchannel {sub}", flush=True)
    got, want, _ = _big_dense(device, bits=4, m=4096, n=16384, k=4096, sub=sub, epilogue="relu2", seed=3)
    assert got.shape == (4096, 16384)
    assert np.array_equal(got, want)


def test_config_c4_int8_swiglu(device):
    got, want, _ = _big_dense(device, bits=8, m=4096, n=11008, k=4096, sub=None, epilogue="swiglu", seed=4,
                              scale_lo=1e-4, scale_hi=1e-3)
    assert got.shape == (4096, 11008)
    assert max_ulp(got, want) <= ULP_TOL


# the int8 32x32 engine's 256-row tiles (four-stage ring) with a K-major A
_I8_BIG = [k for k in _UNSPLIT
           if kt.TABLE[k.table_index].dtype_bits == 8 and kt.TABLE[k.table_index].num_stages == 4
           and k.tile.block_m == 256 and k.layout.value in ("nn", "nt")]


@pytest.mark.parametrize("kernel", _I8_BIG, ids=lambda k: k.kernel_id)
def test_int8_partial_last_round_runs_half_height_tiles(kernel, device):
    """17 column tiles x 16 row tiles = 272 of the 256-row int8 tiles: one
    full round on the chip's CUs and 16 tiles over.  The launcher then runs
    the last column tile as 32 tiles of 128 rows (i8_gemm_kernel's split),
    so both tile heights and the split's column mapping are exercised; every
    output is checked: int32 exact against the C oracle, bf16 exact (plain)
    or within 2 ulp (SwiGLU) against the oracle."""
    from oracle import native as oracle_native

    if not oracle_native.available():
        from oracle import build as obuild

        obuild.build(verbose=False)
    bits, layout, sub, epi = _kernel_params(kernel)
    swiglu = epi == "swiglu"
    m, n, k = 4096, 17 * kernel.tile.block_n, 256
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = (m // 256) * 17
    # a partial last round that one column tile holds, and whose 2 x 16
    # half-height tiles fit one round
    assert tiles > cus and 0 < tiles % cus <= m // 256 and 2 * (m // 256) <= cus
    seed = stable_seed("i8-split", kernel.kernel_id)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=8, layout=layout, m=m, n=n, k=k, subchannel=None,
                                                 swiglu=swiglu, scale_lo=1e-4, scale_hi=1e-3)
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, oracle_native.matmul_i8(a_q, b_q)), "int32 accumulators differ"
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=8, layout=layout, a_scale=sa, b_scale=sb, epilogue=epi)
    if swiglu:
        assert max_ulp(got, want) <= ULP_TOL
    else:
        assert np.array_equal(got, want)


def test_shape_and_layout_errors(device):
    a = torch.zeros((100, 32), dtype=torch.uint8, device=device)
    b = torch.zeros((32, 64), dtype=torch.uint8, device=device)
    with pytest.raises(LookupError):
        shk.mm(a, b, a_scale=torch.ones(100, dtype=torch.bfloat16, device=device),
               b_scale=torch.ones(64, dtype=torch.bfloat16, device=device))
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL),
                                         epilogue=shk.Epilogue.NONE, m=64, n=64, k=64)
    a = torch.zeros((64, 32), dtype=torch.uint8, device=device)
    b = torch.zeros((32, 96), dtype=torch.uint8, device=device)
    with pytest.raises(ValueError, match="tile-multiple"):
        shk.explicit_mm(a, b, kernel=kernel, a_scale=torch.ones(64, dtype=torch.bfloat16, device=device),
                        b_scale=torch.ones(96, dtype=torch.bfloat16, device=device))
    with pytest.raises(ValueError, match="require a_scale and b_scale"):
        shk.explicit_mm(a[:, :32], b[:, :64].contiguous(), kernel=kernel)


# bf16 scale bit patterns that exercise the store path: subnormal, smallest
# normal, largest finite, +-inf, NaN with payload and negative NaN, signed
# zero, one, and values whose products land in the fp32 subnormal range.
SPECIAL_SCALES = np.array([0x0001, 0x0080, 0x007F, 0x7F7F, 0x7F80, 0xFF80, 0x7FC1, 0xFFC0, 0x0000, 0x8000, 0x3F80,
                           0x0200, 0x1000, 0x2000, 0xBF80], dtype=np.uint16)


def _sprinkle(scales, seed, every):
    s = scales.copy()
    r = ref.rng(seed)
    pos = np.arange(0, s.size, every)
    s.reshape(-1)[pos] = SPECIAL_SCALES[r.integers(0, SPECIAL_SCALES.size, size=pos.size)]
    return s


@pytest.mark.parametrize("kernel", [k for k in _UNSPLIT if k.scale.mode is shk.ScaleMode.PER_CHANNEL
                                    and k.layout is shk.GemmLayout.NN], ids=lambda k: k.kernel_id)
def test_special_scale_values_store_like_torch(kernel, device):
    """Per-channel bf16 outputs stay bit-exact (NaN canonical 0x7FC0, subnormals
    kept, overflow to inf) when the scales hold special values."""
    bits, layout, sub, epi = _kernel_params(kernel)
    m, n = 2 * kernel.tile.block_m, 2 * kernel.tile.block_n
    k = 2 * kernel.tile.block_k
    seed = stable_seed("special", kernel.kernel_id)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=None,
                                                 swiglu=epi == "swiglu")
    sa = _sprinkle(sa, seed, 5)
    sb = _sprinkle(sb, seed + 1, 7)
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, ref.int_matmul(a_q, b_q))
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, layout=layout, a_scale=sa, b_scale=sb,
                                       subchannel=None, epilogue=epi)
    nan_want = (want & 0x7FFF) > 0x7F80
    assert np.array_equal(got[nan_want], want[nan_want]), "NaN results must be the canonical 0x7FC0"
    if epi == "swiglu":
        assert max_ulp(got[~nan_want], want[~nan_want]) <= ULP_TOL
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("kernel", [k for k in _UNSPLIT if k.epilogue is shk.Epilogue.SWIGLU
                                    and k.scale.mode is shk.ScaleMode.PER_CHANNEL and k.layout is shk.GemmLayout.NN],
                         ids=lambda k: k.kernel_id)
def test_swiglu_gates_on_both_sides_of_the_fast_range(kernel, device):
    """SwiGLU takes the hardware exp2 / reciprocal path for a wave's group of
    outputs only when every gate of the group has |gate| <= 80, and the exact
    path otherwise.  Rows 0..255 get small A scales, so their tiles hold only
    small gates (the fast path); below them the gates straddle 80 (mostly the
    exact path, including large negative gates, whose outputs underflow
    towards zero).  Every output stays within the bf16 tolerance."""
    bits, layout, _, _ = _kernel_params(kernel)
    m, n = 512, 256
    k, lo, hi = (1024, 0.1, 0.6) if bits == 4 else (256, 0.01, 0.05)
    seed = stable_seed("swiglu-range", kernel.kernel_id)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=None,
                                                 swiglu=True, scale_lo=lo, scale_hi=hi)
    sa[:256] = ref.uniform_bf16(ref.rng(seed + 1), (256,), lo / 20, lo / 10)
    gate = np.abs(ref.scaled_mm(a_q, b_q, sa, sb, subchannel=None)[:, n:])
    assert gate[:256].max() <= 80.0, "rows 0..255 must hold only small gates"
    assert 0.1 < np.mean(gate[256:] > 80.0) < 0.9, "rows 256.. must put gates on both sides of 80"
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, ref.int_matmul(a_q, b_q))
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, layout=layout, a_scale=sa, b_scale=sb,
                                   subchannel=None, epilogue="swiglu")
    assert max_ulp(got, want) <= ULP_TOL


_FP6 = [k for k in _UNSPLIT
        if kt.TABLE[k.table_index].operand_format == kt.OPERANDS_FP6 and k.epilogue is not shk.Epilogue.RELU2
        and k.scale.mode is shk.ScaleMode.PER_CHANNEL]
_FP6_SUB = [k for k in _UNSPLIT
            if kt.TABLE[k.table_index].operand_format == kt.OPERANDS_FP6 and k.scale.mode is shk.ScaleMode.SUBCHANNEL]


@pytest.mark.parametrize("kernel", _FP6, ids=lambda k: k.kernel_id)
@pytest.mark.parametrize("k", [128, 256, 384, 640])
def test_fp6_kernels_every_stage_count(kernel, k, device):
    """One to five K blocks: the ring prologue, the tail and the main loop."""
    _, layout, _, epi = _kernel_params(kernel)
    m, n = 512, 512 if epi != "swiglu" else 256
    seed = stable_seed(f"{kernel.kernel_id}/{k}")
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=4, layout=layout, m=m, n=n, k=k, subchannel=None,
                                                 swiglu=epi == "swiglu")
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, ref.int_matmul(a_q, b_q)), "int32 accumulators differ"
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, layout=layout, a_scale=sa, b_scale=sb, epilogue=epi)
    if epi == "swiglu":
        assert max_ulp(got, want) <= ULP_TOL
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("kernel", _FP6_SUB, ids=lambda k: k.kernel_id)
@pytest.mark.parametrize("groups", [1, 2, 3, 5])
def test_fp6_subchannel_every_group_count(kernel, groups, device):
    """One to five scale groups (groups of 64 in pairs: K is a multiple of the
    tile's 128): each is folded into the fp32 totals in group order, as the
    oracle sums them, so the results are bit-identical; the int32 output is
    the whole exact sum.  Scales spread over two decades so that a fold in the
    wrong order or with the wrong group's scales shows."""
    _, layout, sub, epi = _kernel_params(kernel)
    m, n, k = 256, 384, groups * max(sub, kernel.tile.block_k)
    seed = stable_seed(f"{kernel.kernel_id}/{groups}")
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=4, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=False, scale_lo=0.001, scale_hi=0.1)
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, ref.int_matmul(a_q, b_q)), "int32 accumulators differ"
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, layout=layout, a_scale=sa, b_scale=sb, subchannel=sub,
                                   epilogue=epi)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("kernel", [k for k in _FP6_SUB
                                    if k.layout is shk.GemmLayout.NN and k.epilogue is shk.Epilogue.NONE],
                         ids=lambda k: k.kernel_id)
def test_fp6_subchannel_a_scale_at_two_byte_offset(kernel, device):
    """a_scale needs only 2-byte alignment: the tile's dword loads of it then
    start 2 bytes into a dword, and still pick each row's group scales."""
    from amd_strix_halo_kernels import native
    _, layout, sub, epi = _kernel_params(kernel)
    m, n, k = 256, 256, 4 * max(sub, kernel.tile.block_k)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(stable_seed("sub-offset", kernel.kernel_id), bits=4, layout=layout,
                                                 m=m, n=n, k=k, subchannel=sub, swiglu=False, scale_lo=0.001,
                                                 scale_hi=0.1)
    buf = torch.empty(sa.size + 1, dtype=torch.bfloat16, device=device)
    ta = buf[1:].view(sa.shape)
    ta.copy_(to_dev(torch, sa, device))
    assert ta.data_ptr() % 4 == 2 and ta.is_contiguous()
    out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    print(f"case {kernel.kernel_id} a_scale at +2 bytes", flush=True)
    native.launch_generated_kernel(to_dev(torch, a_arg, device), to_dev(torch, b_arg, device), kernel=kernel,
                                   a_scale=ta, b_scale=to_dev(torch, sb, device), c=out)
    torch.cuda.synchronize()
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, layout=layout, a_scale=sa, b_scale=sb, subchannel=sub,
                                   epilogue=epi)
    assert np.array_equal(bf16_bits(torch, out), want)


@pytest.mark.parametrize("kernel", _FP6_SUB, ids=lambda k: k.kernel_id)
def test_fp6_subchannel_special_scales(kernel, device):
    """The subchannel fold takes its two-operation form (a * b from a rank-1
    MFMA) only for waves whose group scales are all zero or normal within
    [2^-60, 2^60], and the reference's three-operation order otherwise.
    Scales sprinkled with subnormals, huge finite values, infinities, NaN
    and zeros put waves on both paths in every group; every output is
    bit-identical to the oracle (NaN as the canonical 0x7FC0)."""
    _, layout, sub, epi = _kernel_params(kernel)
    m, n, k = 256, 256, 3 * max(sub, kernel.tile.block_k)
    seed = stable_seed("sub-special", kernel.kernel_id)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=4, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=False, scale_lo=0.001, scale_hi=0.1)
    sa = _sprinkle(sa, seed, 37)
    sb = _sprinkle(sb, seed + 1, 53)
    big = ref.bf16_from_f32(np.float32(2.0 ** 61))
    sa[200:, 1] = big  # the lower waves' second group: finite but outside the fast range
    print(f"case {kernel.kernel_id} special scales shape=({m},{n},{k})", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    assert np.array_equal(raw, ref.int_matmul(a_q, b_q))
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        want = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, layout=layout, a_scale=sa, b_scale=sb, subchannel=sub,
                                       epilogue=epi)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_fp6_exact_at_the_k_bound(layout, device):
    """K = 262144 with rows of A and columns of B constant: every output is
    K * c_i * d_j, up to 64 * K = 2^24 for c = d = -8, the largest integer
    magnitude the fp32 accumulation must still hold exactly."""
    m = n = 256
    k = kt.FP6_MAX_K
    c = np.resize(np.arange(-8, 8, dtype=np.int8), m)
    d = np.resize(np.arange(7, -9, -1, dtype=np.int8), n)
    c[:8] = -8
    d[:8] = -8
    a_q = np.repeat(c[:, None], k, axis=1)
    b_q = np.repeat(d[None, :], k, axis=0)
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=4, layout=layout)
    del a_q, b_q
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL),
                                         epilogue=shk.Epilogue.NONE, m=m, n=n, k=k, layout=shk.GemmLayout(layout))
    assert kt.TABLE[kernel.table_index].operand_format == kt.OPERANDS_FP6
    sa = ref.bf16_from_f32(np.ones(m))
    sb = ref.bf16_from_f32(np.ones(n))
    print(f"case fp6 k-bound {layout}", flush=True)
    got, raw = _run_kernel(kernel, a_arg, b_arg, sa, sb, device)
    want = k * c[:, None].astype(np.int64) * d[None, :].astype(np.int64)
    assert raw[0, 0] == 1 << 24
    assert np.array_equal(raw, want)
    assert np.array_equal(got, ref.bf16_round(want.astype(np.float32)))


def _large_k_case(seed, *, m, b_cols, k):
    """int4 operands for a large-K call: random values, with row 0 of A and
    column 0 of B held at -8, so out[0, 0] = 64 * K exceeds fp32's 2^24."""
    r = ref.rng(seed)
    a_q = ref.randint4(r, (m, k))
    b_q = ref.randint4(r, (k, b_cols))
    a_q[0, :] = -8
    b_q[:, 0] = -8
    return a_q, b_q


@pytest.mark.parametrize("layout,epilogue", [("nn", "none"), ("nt", "none"), ("tn", "none"), ("nn", "relu2")])
def test_fp6_large_k_runs_in_exact_slices(layout, epilogue, device):
    """int4 per-channel K above 262144 (the limit of one exact fp32 pass):
    K = 2 * 262144 + 384 runs as three K slices (two full, one of 384) whose
    exact int32 sums add into the workspace, then one pass applies the
    scales and the epilogue.  The raw sums equal the integer matmul (out[0,0]
    = 64 * K > 2^25), and the bf16 output is the oracle's bit for bit, as
    the reference's int32 accumulator gives for any tile-multiple K
    (scripts/generate_amdgcn.py:102-138)."""
    from oracle import native as oracle_native

    m = n = 256
    k = 2 * kt.FP6_MAX_K + 384
    a_q, b_q = _large_k_case(stable_seed("large-k", layout, epilogue), m=m, b_cols=n, k=k)
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=4, layout=layout)
    r = ref.rng(5)
    sa = ref.uniform_bf16(r, (m,), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (n,), 0.005, 0.02)
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL)
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=spec, epilogue=shk.Epilogue(epilogue),
                                         m=m, n=n, k=k, layout=shk.GemmLayout(layout))
    assert kt.TABLE[kernel.table_index].operand_format == kt.OPERANDS_FP6
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    print(f"case fp6 large K {layout} {epilogue} shape=({m},{n},{k})", flush=True)
    out = shk.mm(a, b, a_scale=ta, b_scale=tb, layout=shk.GemmLayout(layout), epilogue=shk.Epilogue(epilogue))
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    want_raw = oracle_native.matmul_i8(a_q, b_q)
    assert want_raw[0, 0] == 64 * k
    assert np.array_equal(raw.cpu().numpy(), want_raw)
    nn_a, nn_b = ref.pack_operands(a_q, b_q, bits=4, layout="nn")
    want = oracle_native.dense_int4_nn(nn_a, nn_b, sa, sb, m=m, n=n, k=k, epilogue=1 if epilogue == "relu2" else 0)
    assert np.array_equal(bf16_bits(torch, out), want)


def test_fp6_large_k_swiglu(device):
    """The fused SwiGLU tile over two K slices (K = 262144 + 128): raw up and
    gate sums exact, the output within 2 bf16 ulp of the oracle."""
    m, n = 256, 128
    k = kt.FP6_MAX_K + 128
    a_q, b_q = _large_k_case(stable_seed("large-k-swiglu"), m=m, b_cols=2 * n, k=k)
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=4, layout="nn")
    r = ref.rng(6)
    sa = ref.uniform_bf16(r, (m,), 0.0005, 0.002)
    sb = ref.uniform_bf16(r, (2 * n,), 0.0005, 0.002)
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL)
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=spec, epilogue=shk.Epilogue.SWIGLU, m=m,
                                         n=n, k=k)
    assert kt.TABLE[kernel.table_index].operand_format == kt.OPERANDS_FP6
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    print(f"case fp6 large K swiglu shape=({m},{n},{k})", flush=True)
    out = shk.fused_swiglu_up_gate(a, b, a_scale=ta, b_scale=tb)
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), ref.int_matmul(a_q, b_q))
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, a_scale=sa, b_scale=sb, epilogue="swiglu")
    assert max_ulp(bf16_bits(torch, out), want) <= ULP_TOL


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("epilogue", ["none", "swiglu"])
def test_fp6_converted_operands_are_reusable(layout, epilogue, device):
    """convert(B) once, then convert(A) + GEMM for two different A: each
    result equals the one-call launch bit for bit."""
    m, n, k = 512, 256, 384
    swiglu = epilogue == "swiglu"
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL)
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=spec, epilogue=shk.Epilogue(epilogue),
                                         m=m, n=n, k=k, layout=shk.GemmLayout(layout))
    assert kt.TABLE[kernel.table_index].operand_format == kt.OPERANDS_FP6
    _, _, _, b_arg, _, sb = dense_case(11, bits=4, layout=layout, m=m, n=n, k=k, subchannel=None, swiglu=swiglu)
    b = to_dev(torch, b_arg, device)
    tb = to_dev(torch, sb, device)
    work = native.gemm_workspace(kernel, m, n, k, device=device)
    print(f"case fp6 reuse {layout} {epilogue}", flush=True)
    native.convert_operand(kernel, 1, b, m=m, n=n, k=k, workspace=work)
    for seed in (12, 13):
        _, _, a_arg, _, sa, _ = dense_case(seed, bits=4, layout=layout, m=m, n=n, k=k, subchannel=None, swiglu=swiglu)
        a = to_dev(torch, a_arg, device)
        ta = to_dev(torch, sa, device)
        native.convert_operand(kernel, 0, a, m=m, n=n, k=k, workspace=work)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        native.launch_converted(kernel, m=m, n=n, k=k, workspace=work, a_scale=ta, b_scale=tb, out=out)
        direct = shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(torch, out), bf16_bits(torch, direct))


def _one_kernel_per_family():
    seen, out = set(), []
    for kernel in _UNSPLIT:
        key = (kernel.a_dtype, kernel.layout, kernel.epilogue, kernel.scale.mode)
        if key not in seen:
            seen.add(key)
            out.append(kernel)
    return out


@pytest.mark.parametrize("kernel", _one_kernel_per_family(), ids=lambda k: k.kernel_id)
def test_torch_gemm_custom_op_matches_oracle(kernel, device):
    """torch_gemm (the registered custom op, reference torch_ops.py) against
    the package's reference math, eagerly and traced by torch.compile through
    the fake implementation, as the reference checks it against
    explicit_mm(use_reference=True) (tests/test_native_generated.py:111-139):
    bit for bit, SwiGLU within 2 bf16 ulp; and bit for bit against
    explicit_mm."""
    bits, layout, sub, epi = _kernel_params(kernel)
    shape = representative_generation_shape(kernel)
    seed = stable_seed("custom-op", kernel.kernel_id)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=shape.m, n=shape.n, k=shape.k,
                                                 subchannel=sub, swiglu=epi == "swiglu")
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    print(f"case {kernel.kernel_id} shape=({shape.m},{shape.n},{shape.k})", flush=True)
    want = shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    got = shk.torch_gemm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch._dynamo.reset()  # each case compiles the same lambda for another kernel
    traced = torch.compile(lambda *t: shk.torch_gemm(t[0], t[1], kernel=kernel, a_scale=t[2], b_scale=t[3]),
                           backend="eager", fullgraph=True)(a, b, ta, tb)
    torch.cuda.synchronize()
    oracle = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, layout=layout, a_scale=sa, b_scale=sb,
                                     subchannel=sub, epilogue=epi)
    for out in (got, traced):
        assert out.dtype == torch.bfloat16 and tuple(out.shape) == (shape.m, shape.n)
        if epi == "swiglu":
            assert max_ulp(bf16_bits(torch, out), oracle) <= ULP_TOL
        else:
            assert np.array_equal(bf16_bits(torch, out), oracle)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))


_PERSISTENT = [k for k in _UNSPLIT if k.schedule is shk.KernelSchedule.PERSISTENT]


@pytest.mark.parametrize("kernel", _PERSISTENT, ids=lambda k: k.kernel_id)
def test_persistent_kernels_loop_over_tiles(kernel, device):
    """Persistent schedule (reference KernelSchedule.PERSISTENT): at 4096 x
    8192 every workgroup takes two or more tiles (256 x 256 tiles: 512 for
    256 resident workgroups; 128 x 128 and 64 x 64 tiles: 2048 and 8192).
    The output equals the standard schedule's bit for bit, the raw int32
    accumulators equal the oracle's integer matmul, and (NN) the bf16 output
    equals the oracle's whole dense path."""
    bits, layout, sub, epi = _kernel_params(kernel)
    m, n, k = 4096, 8192, 512
    seed = stable_seed("persistent", kernel.kernel_id)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=False)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    standard = shk.default_registry.select(dtype=kernel.a_dtype, scale=kernel.scale, epilogue=kernel.epilogue,
                                           layout=kernel.layout, m=m, n=n, k=k)
    print(f"case {kernel.kernel_id} vs {standard.kernel_id} shape=({m},{n},{k})", flush=True)
    got = shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    want = shk.explicit_mm(a, b, kernel=standard, a_scale=ta, b_scale=tb)
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    from oracle import native as oracle_native

    assert np.array_equal(raw.cpu().numpy(), oracle_native.matmul_i8(a_q, b_q))
    if layout == "nn":
        oracle = oracle_native.dense_int4_nn(a_arg, b_arg, sa, sb, m=m, n=n, k=k, subchannel=sub or 0, epilogue=0)
        assert np.array_equal(bf16_bits(torch, got), oracle)


@pytest.mark.parametrize("scale", ["pc", "sc32", "sc64", "sc128", "sc256"])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_mm_persistent_schedule_matches_oracle(scale, layout, device):
    """mm(schedule=KernelSchedule.PERSISTENT) (reference api.py:119-164)."""
    m, n, k = 512, 768, 512
    sub = None if scale == "pc" else int(scale[2:])
    seed = stable_seed("mm-persistent", scale, layout)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=4, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=False)
    spec = shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL) if sub is None else shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, sub)
    print(f"case mm persistent {scale} {layout}", flush=True)
    out = shk.mm(to_dev(torch, a_arg, device), to_dev(torch, b_arg, device), a_scale=to_dev(torch, sa, device),
                 b_scale=to_dev(torch, sb, device), layout=shk.GemmLayout(layout), scale=spec,
                 schedule=shk.KernelSchedule.PERSISTENT)
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=4, layout=layout, a_scale=sa, b_scale=sb, subchannel=sub,
                                   epilogue="none")
    assert np.array_equal(bf16_bits(torch, out), want)
