"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Every oracle function is checked against something other than a retyping of
its own formula:

* known answers from the reference's tests (pack/unpack, the integer matmul,
  calculate_group_info, the TOPS definition);
* golden vectors written by the reference package itself
  (tests/golden/reference_vectors.npz, from tests/golden/make_golden.py):
  reference_mm for int4/int8 x NN/NT/TN x pc/sc32/sc64/sc128 x
  none/relu2/swiglu, and calculate_group_info's torch branch;
* brute force on tiny inputs (nibble loops, int64 triple loops, row
  ownership of the task list);
* closed forms and invariants (bf16 rounding vs torch's conversion, unit
  scales, a single subchannel group equals per-channel, layout equivalence,
  a one-group ragged call equals the dense call, empty groups give zeros);
* the C restatement against the numpy one (bit for bit).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import ref

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---------------------------------------------------------------------------
# known answers from the reference's tests


def test_pack_unpack_known_answers():
    # tests/test_quant.py:34-38
    x = np.array([[-8, -1, 0, 7], [3, -4, 5, -6]], dtype=np.int8)
    p = ref.pack_int4_k_major(x)
    assert p.dtype == np.uint8
    assert np.array_equal(ref.unpack_int4_k_major(p), x)
    # byte = (odd << 4) | (even & 0xF)
    assert p.tolist() == [[0xF8, 0x70], [0xC3, 0xA5]]
    # tests/test_quant.py:41-45: odd K is zero-padded
    assert ref.unpack_int4_k_major(ref.pack_int4_k_major(np.array([[1, -2, 3]], np.int8))).tolist() == [[1, -2, 3, 0]]


def test_integer_matmul_known_answer():
    # tests/test_quant.py:56-76
    a = np.array([[1, -2, 3, -4], [5, 6, -7, 0]], dtype=np.int8)
    b = np.array([[1, 2], [-3, 4], [5, -6], [7, 0]], dtype=np.int8)
    assert ref.int_matmul(a, b).tolist() == [[-6, -24], [-48, 76]]
    ap, bp = ref.pack_operands(a, b, bits=4, layout="nn")
    out = ref.reference_gemm(ap, bp, bits=4, layout="nn")
    assert out.tolist() == [[-6.0, -24.0], [-48.0, 76.0]]


def test_group_info_known_answers():
    # tests/test_ragged_dot.py:120-131
    info = ref.calculate_group_info(np.array([17, 31, 24]), 32, align_tile=8)
    assert info.num_tasks == 3
    assert info.group_id.tolist() == [0, 1, 2]
    assert info.block_start.tolist() == [0, 16, 48]
    assert info.actual_start.tolist() == [0, 17, 48]
    assert info.actual_end.tolist() == [17, 48, 72]
    assert info.start_within_block.tolist() == [0, 1, 0]
    assert info.actual_size.tolist() == [17, 31, 24]
    # tests/test_ragged_dot.py:134-144
    info = ref.calculate_group_info(np.array([2, 0, 7]), 16, tid_size=4, align_tile=8)
    assert info.num_tasks == 2
    assert info.group_id.tolist() == [0, 2, 0, 0]
    assert info.block_start.tolist() == [0, 0, 0, 0]
    assert info.actual_start.tolist() == [0, 2, 0, 0]
    assert info.actual_end.tolist() == [2, 9, 0, 0]
    assert info.actual_size.tolist() == [2, 7, 0, 0]
    # tests/test_ragged_dot.py:147-151
    with pytest.raises(ValueError, match="tid_size must be at least 3"):
        ref.calculate_group_info(np.array([17, 31, 24]), 32, tid_size=2, align_tile=8)


def test_tops_known_answer():
    # tests/test_benchmarking.py:50-53
    assert ref.tops_for_runtime(1024, 1024, 1024, 1.0) == pytest.approx(2.147483648)


# ---------------------------------------------------------------------------
# golden vectors from the reference package


def test_dense_reference_matches_reference_package_bit_for_bit(golden):
    cases = [str(c) for c in golden["dense_cases"]]
    assert len(cases) == 72
    worst = {}
    for name in cases:
        bits = int(name[1])
        _, layout, scale, epi = name.split("_")
        sub = None if scale == "pc" else int(scale[2:])
        got = ref.reference_gemm_bf16(golden[f"{name}.a"], golden[f"{name}.b"], bits=bits, layout=layout,
                                      a_scale=golden[f"{name}.a_scale"], b_scale=golden[f"{name}.b_scale"],
                                      subchannel=sub, epilogue=epi)
        want = golden[f"{name}.out"]
        assert got.shape == want.shape, name
        d = ref.bf16_ulp_diff(got, want)
        worst[name] = int(d.max())
        if epi == "swiglu":
            # exp() of numpy and torch may differ by an ulp; after the bf16
            # cast that is at most one bf16 ulp.
            assert d.max() <= 1, name
        else:
            assert np.array_equal(got, want), name
    assert sum(v == 0 for v in worst.values()) >= 48


def test_group_info_matches_reference_package(golden):
    for key in golden["group_info_cases"]:
        key = str(key)
        sizes = golden[f"{key}.sizes"]
        tile, tid, align, num = (int(v) for v in golden[f"{key}.params"])
        info = ref.calculate_group_info(sizes, tile, tid_size=None if tid < 0 else tid, align_tile=align)
        assert info.num_tasks == num
        got = np.stack([info.group_id, info.block_start, info.actual_start, info.actual_end,
                        info.start_within_block, info.actual_size])
        assert np.array_equal(got, golden[f"{key}.fields"]), key


# ---------------------------------------------------------------------------
# brute force


def test_unpack_every_byte_brute_force():
    p = np.arange(256, dtype=np.uint8).reshape(1, 256)
    u = ref.unpack_int4_k_major(p)
    for v in range(256):
        lo, hi = v & 15, v >> 4
        assert u[0, 2 * v] == (lo - 16 if lo > 7 else lo)
        assert u[0, 2 * v + 1] == (hi - 16 if hi > 7 else hi)
    assert np.array_equal(ref.pack_int4_k_major(u), p)


@pytest.mark.parametrize("shape", [(3, 5, 7), (16, 9, 33), (1, 1, 1)])
def test_int_matmul_brute_force(shape):
    m, n, k = shape
    r = ref.rng(m * 100 + n * 10 + k)
    a = ref.randint8(r, (m, k))
    b = ref.randint8(r, (k, n))
    want = np.zeros((m, n), dtype=np.int64)
    for i in range(m):
        for j in range(n):
            s = 0
            for kk in range(k):
                s += int(a[i, kk]) * int(b[kk, j])
            want[i, j] = s
    assert np.array_equal(ref.int_matmul(a, b), want)


def test_group_info_rows_owned_exactly_once():
    r = ref.rng(5)
    for _ in range(50):
        g = int(r.integers(1, 10))
        sizes = r.integers(0, 90, size=g)
        tile = int(r.choice([16, 32, 64]))
        align = int(r.choice([1, 2, 4, 8, 16]))
        info = ref.calculate_group_info(sizes, tile, align_tile=align)
        owner = np.full(int(sizes.sum()), -1)
        starts = np.concatenate([[0], np.cumsum(sizes)])
        for t in range(info.num_tasks):
            gid = info.group_id[t]
            a0, a1 = info.actual_start[t], info.actual_end[t]
            assert starts[gid] <= a0 < a1 <= starts[gid + 1]
            assert info.block_start[t] % align == 0 or info.block_start[t] >= starts[gid] - align
            assert info.block_start[t] <= a0 and a1 <= info.block_start[t] + tile
            assert (owner[a0:a1] == -1).all()
            owner[a0:a1] = gid
        assert (owner >= 0).all()


# ---------------------------------------------------------------------------
# closed forms and invariants


def test_bf16_round_matches_torch_conversion():
    torch = pytest.importorskip("torch")
    r = ref.rng(11)
    x = np.concatenate([
        r.standard_normal(20000).astype(np.float32) * 10.0 ** r.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 3.0e38, -3.0e38, 1.0e-40, np.inf, -np.inf], np.float32),
        # exact ties: the low 16 bits are 0x8000
        (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ]).astype(np.float32)
    got = ref.bf16_round(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_unit_scales_reproduce_the_integer_result():
    r = ref.rng(3)
    a, b = ref.randint4(r, (24, 64)), ref.randint4(r, (64, 40))
    ap, bp = ref.pack_operands(a, b, bits=4, layout="nn")
    ones_a = ref.bf16_from_f32(np.ones(24))
    ones_b = ref.bf16_from_f32(np.ones(40))
    out = ref.reference_gemm(ap, bp, bits=4, a_scale=ones_a, b_scale=ones_b)
    assert np.array_equal(out, ref.int_matmul(a, b).astype(np.float32))


def test_one_subchannel_group_equals_per_channel():
    r = ref.rng(4)
    a, b = ref.randint4(r, (8, 64)), ref.randint4(r, (64, 16))
    ap, bp = ref.pack_operands(a, b, bits=4, layout="nn")
    sa = ref.uniform_bf16(r, (8,), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (16,), 0.005, 0.02)
    pc = ref.reference_gemm(ap, bp, bits=4, a_scale=sa, b_scale=sb)
    sc = ref.reference_gemm(ap, bp, bits=4, a_scale=sa[:, None], b_scale=sb[None, :], subchannel=64)
    assert np.array_equal(pc, sc)


def test_scale_order_is_a_then_b():
    # (acc * sa) * sb and acc * (sa * sb) round differently for these values;
    # the golden vectors fix the first, this pins that the oracle keeps it.
    acc = np.array([[7]], dtype=np.int8)
    one = np.array([[1]], dtype=np.int8)
    sa = ref.bf16_from_f32(np.array([0.0117], np.float32))
    sb = ref.bf16_from_f32(np.array([0.0193], np.float32))
    fa, fb = ref.bf16_to_f32(sa)[0], ref.bf16_to_f32(sb)[0]
    got = ref.scaled_mm(acc, one, sa, sb, subchannel=None)[0, 0]
    assert got == np.float32(np.float32(7.0 * fa) * fb)


@pytest.mark.parametrize("bits", [4, 8])
def test_layouts_are_equivalent(bits):
    r = ref.rng(bits)
    a = ref.randint4(r, (16, 32)) if bits == 4 else ref.randint8(r, (16, 32))
    b = ref.randint4(r, (32, 24)) if bits == 4 else ref.randint8(r, (32, 24))
    outs = []
    for layout in ("nn", "nt", "tn"):
        ap, bp = ref.pack_operands(a, b, bits=bits, layout=layout)
        outs.append(ref.reference_gemm(ap, bp, bits=bits, layout=layout))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_relu2_and_swiglu_closed_forms():
    x = np.array([[-2.0, 0.0, 3.0, 0.0, 5.0, -5.0]], np.float32)
    assert ref.relu2(x).tolist() == [[0.0, 0.0, 9.0, 0.0, 25.0, 0.0]]
    s = ref.swiglu(x)  # up = [-2, 0, 3], gate = [0, 5, -5]
    assert s[0, 0] == 0.0  # gate 0 -> silu 0
    assert s[0, 1] == 0.0  # up 0
    assert s[0, 2] == pytest.approx(3.0 * (-5.0 / (1.0 + np.exp(5.0))), rel=1e-6)


def test_ragged_single_group_equals_dense():
    r = ref.rng(21)
    a = ref.randint4(r, (40, 64))
    b = ref.randint4(r, (1, 64, 24))
    sa = ref.uniform_bf16(r, (40,), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (1, 24), 0.005, 0.02)
    out = ref.ragged_fwd_reference(a, b, np.array([40]), sa, sb)
    dense = ref.scaled_mm(a, b[0], sa, sb[0], subchannel=None)
    assert np.array_equal(out, dense)


def test_ragged_bwd_empty_and_full_groups():
    r = ref.rng(22)
    a = ref.randint4(r, (3, 8, 39))
    b = ref.randint4(r, (3, 39, 12))
    sa = ref.uniform_bf16(r, (3, 8), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (3, 12), 0.005, 0.02)
    out = ref.ragged_bwd_reference(a, b, np.array([5, 0, 39]), sa, sb)
    assert (out[1] == 0).all()
    assert np.array_equal(out[2], ref.scaled_mm(a[2], b[2], sa[2], sb[2], subchannel=None))
    assert np.array_equal(out[0], ref.scaled_mm(a[0, :, :5], b[0, :5], sa[0], sb[0], subchannel=None))


def _f32(x) -> np.float32:
    return np.float32(x)


def _bf(bits) -> np.float32:
    return ref.bf16_to_f32(np.uint16(bits))[()] if np.ndim(bits) == 0 else ref.bf16_to_f32(bits)


@pytest.mark.parametrize("subchannel", [None, 4])
def test_ragged_fwd_reference_brute_force_over_groups(subchannel):
    """Element by element over five groups, one empty and one of a single
    row: row i belongs to the group whose cumulative row span holds it, and
    out[i, j] is (float(sum_k a[i,k] b[g,k,j]) * a_scale[i]) * b_scale[g, j]
    (per-channel) or the K-ordered fp32 sum of the per-group products with
    the last group partial (subchannel S = 4, K = 10), as the reference's
    grouped references compute them (tests/test_ragged_dot.py:19-51)."""
    r = ref.rng(41)
    sizes = np.array([3, 0, 5, 1, 4])
    m, k, n, groups = int(sizes.sum()), 10, 5, sizes.size
    a_q = ref.randint4(r, (m, k))
    b_q = ref.randint4(r, (groups, k, n))
    if subchannel:
        cols = -(-k // subchannel)
        sa = ref.uniform_bf16(r, (m, cols), 0.01, 1.0)
        sb = ref.uniform_bf16(r, (groups, cols, n), 0.01, 1.0)
    else:
        sa = ref.uniform_bf16(r, (m,), 0.01, 1.0)
        sb = ref.uniform_bf16(r, (groups, n), 0.01, 1.0)
    got = ref.ragged_fwd_reference(a_q, b_q, sizes, sa, sb, subchannel=subchannel)
    owner = []
    for g, sz in enumerate(sizes.tolist()):
        owner += [g] * sz
    for i in range(m):
        g = owner[i]
        for j in range(n):
            if not subchannel:
                acc = sum(int(a_q[i, kk]) * int(b_q[g, kk, j]) for kk in range(k))
                v = _f32(_f32(acc) * _bf(sa[i]))
                v = _f32(v * _bf(sb[g, j]))
            else:
                v = _f32(0.0)
                for s, k0 in enumerate(range(0, k, subchannel)):
                    acc = sum(int(a_q[i, kk]) * int(b_q[g, kk, j]) for kk in range(k0, min(k0 + subchannel, k)))
                    p = _f32(_f32(acc) * _bf(sa[i, s]))
                    p = _f32(p * _bf(sb[g, s, j]))
                    v = _f32(v + p)
            assert got[i, j].view(np.uint32) == v.view(np.uint32), (i, j, g)


def test_ragged_bwd_reference_subchannel():
    """Subchannel backward: a full-length group equals the dense subchannel
    product (scaled_mm, pinned by the reference's golden vectors); a group
    truncated inside a scale group sums only the scale groups that start
    below its length, the last one cut at the length; an empty group is zero
    (tests/test_ragged_dot.py:99-117)."""
    r = ref.rng(42)
    groups, rows, kcap, cols, sub = 3, 6, 24, 7, 8
    a_q = ref.randint4(r, (groups, rows, kcap))
    b_q = ref.randint4(r, (groups, kcap, cols))
    sa = ref.uniform_bf16(r, (groups, rows, kcap // sub), 0.01, 1.0)
    sb = ref.uniform_bf16(r, (groups, kcap // sub, cols), 0.01, 1.0)
    sizes = np.array([kcap, 13, 0])
    got = ref.ragged_bwd_reference(a_q, b_q, sizes, sa, sb, subchannel=sub)
    assert np.array_equal(got[0], ref.scaled_mm(a_q[0], b_q[0], sa[0], sb[0], subchannel=sub))
    assert (got[2] == 0).all()
    gk = int(sizes[1])
    for i in range(rows):
        for j in range(cols):
            v = _f32(0.0)
            for s, k0 in enumerate(range(0, kcap, sub)):
                k1 = min(k0 + sub, gk)
                if k1 <= k0:
                    continue
                acc = sum(int(a_q[1, i, kk]) * int(b_q[1, kk, j]) for kk in range(k0, k1))
                p = _f32(_f32(acc) * _bf(sa[1, i, s]))
                p = _f32(p * _bf(sb[1, s, j]))
                v = _f32(v + p)
            assert got[1, i, j].view(np.uint32) == v.view(np.uint32), (i, j)
    # the second scale group is cut at 13: K values 13..15 must not count
    cut = a_q.copy()
    cut[1, :, 13:] = 0
    assert np.array_equal(got[1], ref.scaled_mm(cut[1], b_q[1], sa[1], sb[1], subchannel=sub))


def test_bf16_ulp_diff_closed_forms():
    """Distances on the bf16 line: adjacent values are 1 apart on either
    side of zero, +0 and -0 coincide, a pair straddling zero is the sum of
    the magnitudes' distances from zero, a binade holds 128 steps, and the
    distance is symmetric."""
    d = ref.bf16_ulp_diff
    assert d(np.uint16(0x3F80), np.uint16(0x3F81)) == 1      # 1.0, next bf16
    assert d(np.uint16(0xBF80), np.uint16(0xBF81)) == 1      # -1.0, next below
    assert d(np.uint16(0x007F), np.uint16(0x0080)) == 1      # largest subnormal, smallest normal
    assert d(np.uint16(0x0000), np.uint16(0x8000)) == 0      # +0, -0
    assert d(np.uint16(0x0003), np.uint16(0x8002)) == 5      # 3 ulps above zero, 2 below
    assert d(np.uint16(0x3F80), np.uint16(0x4000)) == 128    # 1.0 to 2.0
    assert d(np.uint16(0x3F80), np.uint16(0xBF80)) == 2 * 0x3F80
    a = np.array([0x1234, 0x8001, 0x7F7F], dtype=np.uint16)
    b = np.array([0x1236, 0x0001, 0x7F7E], dtype=np.uint16)
    assert d(a, b).tolist() == [2, 2, 1]
    assert np.array_equal(d(a, b), d(b, a))
    assert (d(a, a) == 0).all()


# ---------------------------------------------------------------------------
# C restatement vs numpy restatement


def test_c_oracle_matches_numpy_oracle():
    from oracle import native

    if not native.available():
        from oracle import build as obuild

        obuild.build(verbose=False)
    r = ref.rng(31)
    m, n, k = 48, 80, 512
    a, b = ref.randint4(r, (m, k)), ref.randint4(r, (k, n))
    ap, bp = ref.pack_operands(a, b, bits=4, layout="nn")
    assert np.array_equal(native.matmul_i8(a, b), ref.int_matmul(a, b))
    for sub, epi in ((0, 0), (0, 1), (64, 0), (256, 1)):
        if sub:
            sa = ref.uniform_bf16(r, (m, k // sub), 0.005, 0.02)
            sb = ref.uniform_bf16(r, (k // sub, n), 0.005, 0.02)
        else:
            sa = ref.uniform_bf16(r, (m,), 0.005, 0.02)
            sb = ref.uniform_bf16(r, (n,), 0.005, 0.02)
        want = ref.reference_gemm_bf16(ap, bp, bits=4, a_scale=sa, b_scale=sb, subchannel=sub or None,
                                       epilogue="relu2" if epi else "none")
        got = native.dense_int4_nn(ap, bp, sa, sb, m=m, n=n, k=k, subchannel=sub, epilogue=epi)
        assert np.array_equal(got, want), (sub, epi)


def test_device_fake_quant_closed_forms():
    """fake_quant_int_device: for power-of-two scales the reciprocal is
    exact, so it must equal the CPU division form everywhere; ties round half
    to even; NaN gives 0 and infinities clamp.  (Its reciprocal rule for
    other scales is pinned against torch on the GPU, tests/test_gpu_quant.py.)"""
    r = ref.rng(77)
    x = (r.standard_normal(200_000) * 6).astype(np.float32)
    ties = (np.arange(-20, 20) + 0.5).astype(np.float32)
    for scale in (0.125, 0.5, 2.0, 1.0 / 64):
        for bits in (4, 8):
            assert np.array_equal(ref.fake_quant_int_device(x * scale, bits=bits, scale=scale),
                                  ref.fake_quant_int(x * scale, bits=bits, scale=scale))
        got = ref.fake_quant_int_device(ties * np.float32(scale), bits=8, scale=scale)
        assert np.array_equal(got, np.rint(ties).astype(np.int8))  # half to even: 0.5 -> 0, 1.5 -> 2
        assert np.all(got % 2 == 0)
    special = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e30, -1e30], dtype=np.float32)
    assert ref.fake_quant_int_device(special, bits=4, scale=0.1).tolist() == [0, 7, -8, 0, 0, 7, -8]
    assert ref.fake_quant_int_device(special, bits=8, scale=3.0).tolist() == [0, 127, -128, 0, 0, 127, -128]
    # the reciprocal is rounded once from double: 1/0.017 in float32 differs from 1/float32(0.017)
    assert np.float32(1.0 / 0.017) != np.float32(1.0) / np.float32(0.017)
