"""Split-K table kernels (reference registry.py:96-108 SPLIT_K 2/4/8, float32
output zeroed before the launch, native.py:739-740).

Each K slice sums its integer products exactly and adds its scaled fp32
partial into the output, so:
  * with unit scales the output is the exact int32 product (every partial is
    an integer below 2^24 in magnitude, and so is every sum of them): this
    pins the slice offsets of both operands bit for bit;
  * with random scales the output is the oracle's scaled product up to fp32
    rounding of at most 8 partial sums: |got - want| <= 1e-5 * bound, where
    bound is the oracle's scaled product of the operands' magnitudes;
  * subchannel slices start at their first scale group.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from tests._util import dense_case, stable_seed, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

import amd_strix_halo_kernels as shk  # noqa: E402

_SPLIT = tuple(k for k in shk.default_registry.all() if k.tile.split_k > 1)
ONE_BF16 = 0x3F80


def _sub_of(kernel):
    if kernel.scale.mode is not shk.ScaleMode.SUBCHANNEL:
        return None
    return kernel.scale.subchannel_size


def _run(kernel, a_arg, b_arg, sa, sb, device):
    out = shk.explicit_mm(to_dev(torch, a_arg, device), to_dev(torch, b_arg, device), kernel=kernel,
                          a_scale=to_dev(torch, sa, device), b_scale=to_dev(torch, sb, device))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    return out.cpu().numpy()


def test_split_entries_cover_the_reference_families():
    fams = {(k.a_dtype, k.scale.mode, k.layout, k.tile.split_k) for k in _SPLIT}
    for layout in (shk.GemmLayout.NN, shk.GemmLayout.NT, shk.GemmLayout.TN):
        for split in (2, 4, 8):
            assert (shk.OperandDType.INT4, shk.ScaleMode.PER_CHANNEL, layout, split) in fams
            assert (shk.OperandDType.INT4, shk.ScaleMode.SUBCHANNEL, layout, split) in fams
            assert (shk.OperandDType.INT8, shk.ScaleMode.PER_CHANNEL, layout, split) in fams
            assert (shk.OperandDType.INT8, shk.ScaleMode.SUBCHANNEL, layout, split) in fams
    assert all(k.output_dtype == "float32" and k.epilogue is shk.Epilogue.NONE for k in _SPLIT)


@pytest.mark.parametrize("kernel", _SPLIT, ids=lambda k: k.kernel_id)
@pytest.mark.parametrize("blocks", [1, 3])
def test_split_k_matches_oracle(kernel, blocks, device):
    """`blocks` K blocks (or scale groups) per slice; one is the shortest
    slice a split entry accepts (K = BLOCK_K * SPLIT_K), where each slice's
    pipeline runs a single stage."""
    bits = 4 if kernel.a_dtype is shk.OperandDType.INT4 else 8
    sub = _sub_of(kernel)
    m, n = 2 * kernel.tile.block_m, 2 * kernel.tile.block_n
    # whole groups per slice
    k = blocks * kernel.tile.block_k * kernel.tile.split_k
    if sub:
        k = blocks * kernel.tile.split_k * max(sub, kernel.tile.block_k)
    seed = stable_seed("splitk", kernel.kernel_id, blocks)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=kernel.layout.value, m=m, n=n, k=k,
                                                 subchannel=sub, swiglu=False)
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)

    # unit scales: the exact integer product
    ones_a = np.full(sa.shape, ONE_BF16, dtype=np.uint16)
    ones_b = np.full(sb.shape, ONE_BF16, dtype=np.uint16)
    exact = _run(kernel, a_arg, b_arg, ones_a, ones_b, device)
    assert np.array_equal(exact, ref.int_matmul(a_q, b_q).astype(np.float32))

    got = _run(kernel, a_arg, b_arg, sa, sb, device)
    want = ref.scaled_mm(a_q, b_q, sa, sb, subchannel=sub)
    bound = ref.scaled_mm(np.abs(a_q.astype(np.int32)), np.abs(b_q.astype(np.int32)), sa & 0x7FFF, sb & 0x7FFF, subchannel=sub)
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * bound.astype(np.float64) + 1e-30)


@pytest.mark.parametrize("split", [2, 8])
def test_split_k_large_k(split, device):
    """int4 per-channel K of about 2^18, twice what one unsplit accumulator
    of the int8 engines holds: each slice's int32 sum stays exact (K /
    SPLIT_K < 131072; split 2: K = 262016, split 8: K = 262144).  Row 0 of A
    and column 0 of B hold -8, so out[0, 0] = 64 * K, up to 2^24.
    Unit scales give the exact integer product (every partial sum of the
    slices is an integer of magnitude <= 2^24); random scales stay within the
    fp32 bound of the other split tests.  The order of the slices' atomic
    adds varies from run to run, so those results may differ in the last
    bits between runs (the tolerance covers it)."""
    kernel = next(k for k in _SPLIT if k.tile.split_k == split and k.scale.mode is shk.ScaleMode.PER_CHANNEL
                  and k.a_dtype is shk.OperandDType.INT4 and k.layout is shk.GemmLayout.NN)
    m, n = kernel.tile.block_m, kernel.tile.block_n
    k = 262144 if split == 8 else 2 * (131072 - 64)
    r = ref.rng(stable_seed("splitk-large", split))
    a_q = ref.randint4(r, (m, k))
    b_q = ref.randint4(r, (k, n))
    a_q[0, :] = -8
    b_q[:, 0] = -8
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=4, layout="nn")
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    ones_a = np.full((m,), ONE_BF16, dtype=np.uint16)
    ones_b = np.full((n,), ONE_BF16, dtype=np.uint16)
    exact = _run(kernel, a_arg, b_arg, ones_a, ones_b, device)
    prod = ref.int_matmul(a_q, b_q)
    assert prod[0, 0] == 64 * k
    assert np.array_equal(exact, prod.astype(np.float32))
    sa = ref.uniform_bf16(r, (m,), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (n,), 0.005, 0.02)
    got = _run(kernel, a_arg, b_arg, sa, sb, device)
    want = ref.scaled_mm(a_q, b_q, sa, sb, subchannel=None)
    bound = ref.scaled_mm(np.abs(a_q.astype(np.int32)), np.abs(b_q.astype(np.int32)), sa, sb, subchannel=None)
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * bound.astype(np.float64) + 1e-30)


def test_split_k_rejects_shapes_and_modes_it_cannot_run(device):
    kernel = next(k for k in _SPLIT if k.tile.split_k == 8 and k.scale.mode is shk.ScaleMode.PER_CHANNEL
                  and k.a_dtype is shk.OperandDType.INT4 and k.layout is shk.GemmLayout.NN)
    m, n, k = 256, 256, 256  # K = 256 < BLOCK_K * 8
    a = torch.zeros((m, k // 2), dtype=torch.uint8, device=device)
    b = torch.zeros((k // 2, n), dtype=torch.uint8, device=device)
    sa = torch.ones(m, dtype=torch.bfloat16, device=device)
    sb = torch.ones(n, dtype=torch.bfloat16, device=device)
    with pytest.raises(Exception, match="SPLIT_K"):
        shk.explicit_mm(a, b, kernel=kernel, a_scale=sa, b_scale=sb)
