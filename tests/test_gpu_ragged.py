"""GPU parity of the ragged path (calculate_group_info, ragged_dot_int4,
ragged_dot_int4_bwd) against the CPU oracle.

The cases mirror the reference's tests/test_ragged_dot.py (:154-586): every
layout, per-channel and subchannel-32 scales, split_k 1 and 2, empty groups,
odd K with garbage in the padding, and the even-K fast path; plus the
C5 MoE benchmark shape at full size.  Per-channel results are bit-identical to
the oracle (same op order, exact int32 sums); subchannel split-K adds fp32
partials in another order and is held to a relative 1e-5.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest

from oracle import ref
from tests._util import bf16_bits, max_ulp, stable_seed, to_dev

torch = pytest.importorskip("torch")

import amd_strix_halo_kernels as shk  # noqa: E402

pytestmark = pytest.mark.gpu

LAYOUTS = [shk.GemmLayout.NN, shk.GemmLayout.NT, shk.GemmLayout.TN, shk.GemmLayout.TT]
SCALES = [shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL), shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 32)]


def _pack_fwd(a_q, b_q, layout):
    """Physical forward operands (test_ragged_dot.py:54-65)."""
    lhs = ref.pack_int4_k_major(a_q)
    if layout in (shk.GemmLayout.TN, shk.GemmLayout.TT):
        lhs = np.ascontiguousarray(lhs.T)
    rhs = []
    for g in range(b_q.shape[0]):
        p = ref.pack_int4_k_major(b_q[g].T)
        rhs.append(p if layout in (shk.GemmLayout.NT, shk.GemmLayout.TT) else np.ascontiguousarray(p.T))
    return lhs, np.ascontiguousarray(np.stack(rhs))


def _pack_bwd(a_q, b_q, layout):
    """Physical backward operands (test_ragged_dot.py:68-81)."""
    lhs, rhs = [], []
    for g in range(a_q.shape[0]):
        l = ref.pack_int4_k_major(a_q[g])
        lhs.append(np.ascontiguousarray(l.T) if layout in (shk.GemmLayout.TN, shk.GemmLayout.TT) else l)
        r = ref.pack_int4_k_major(b_q[g].T)
        rhs.append(r if layout in (shk.GemmLayout.NT, shk.GemmLayout.TT) else np.ascontiguousarray(r.T))
    return np.ascontiguousarray(np.stack(lhs)), np.ascontiguousarray(np.stack(rhs))


# ---------------------------------------------------------------------------
# task list


@pytest.mark.parametrize(
    "sizes,tile,tid_size",
    [([512] * 8, 64, None), ([300, 0, 1000, 17, 2779], 64, None), ([1] * 16, 32, None), ([4096], 128, None),
     ([7, 9, 0, 40], 16, None), ([512] * 8, 64, 600), ([17, 31, 24], 32, None), ([2, 0, 7], 16, 4),
     ([0, 0, 0], 16, None), ([0, 0, 0], 16, 5)],
)
def test_group_info_device_matches_oracle(sizes, tile, tid_size, device):
    gs = torch.tensor(sizes, dtype=torch.int32, device=device)
    info = shk.calculate_group_info(gs, tile, tid_size=tid_size)
    want = ref.calculate_group_info(np.array(sizes), tile, tid_size=tid_size)
    assert info.num_tasks == want.num_tasks
    for f in ("group_id", "block_start", "actual_start", "actual_end", "start_within_block", "actual_size"):
        got = getattr(info, f)
        assert got.is_cuda and got.dtype == torch.int64
        assert np.array_equal(got.cpu().numpy(), getattr(want, f)), f


def test_group_info_device_random_against_oracle(device):
    r = ref.rng(77)
    for _ in range(40):
        g = int(r.integers(1, 40))
        sizes = r.integers(0, 300, size=g)
        tile = int(r.choice([16, 32, 64, 128]))
        align = int(r.choice([1, 2, 4, 8]))
        info = shk.calculate_group_info(torch.tensor(sizes, device=device), tile, align_tile=align)
        want = ref.calculate_group_info(sizes, tile, align_tile=align)
        assert info.num_tasks == want.num_tasks
        assert np.array_equal(info.actual_end.cpu().numpy(), want.actual_end)
        assert np.array_equal(info.block_start.cpu().numpy(), want.block_start)
        assert np.array_equal(info.group_id.cpu().numpy(), want.group_id)


# ---------------------------------------------------------------------------
# forward


def _fwd_case(seed, m, k, n, sizes, scale, *, std=0.1):
    r = ref.rng(seed)
    groups = len(sizes)
    a_q = ref.randint4(r, (m, k))
    b_q = ref.randint4(r, (groups, k, n))
    if scale.mode is shk.ScaleMode.PER_CHANNEL:
        sa = ref.uniform_bf16(r, (m,), 0.008, 0.012)
        sb = ref.uniform_bf16(r, (groups, n), 0.009, 0.011)
    else:
        cols = -(-k // scale.subchannel_size)
        sa = ref.uniform_bf16(r, (m, cols), 0.008, 0.012)
        sb = ref.uniform_bf16(r, (groups, cols, n), 0.009, 0.011)
    return a_q, b_q, sa, sb


def _run_fwd(device, a_q, b_q, sizes, sa, sb, scale, layout, config, output_dtype):
    lhs, rhs = _pack_fwd(a_q, b_q, layout)
    out = shk.ragged_dot_int4(
        to_dev(torch, lhs, device), to_dev(torch, rhs, device), torch.tensor(sizes, dtype=torch.int32, device=device),
        a_scale=to_dev(torch, sa, device), b_scale=to_dev(torch, sb, device), scale=scale, config=config,
        layout=layout, output_dtype=output_dtype)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("output_dtype", ["float32", "bfloat16"])
def test_ragged_fwd_small_reference_case(output_dtype, device):
    """test_ragged_dot.py:240-303: m=9, k=32, n=16, sizes [2, 0, 7]."""
    scale = SCALES[0]
    sizes = [2, 0, 7]
    a_q, b_q, sa, sb = _fwd_case(19, 9, 32, 16, sizes, scale)
    cfg = shk.RaggedDotConfig(block_m=16, block_n=16, block_k=32, group_size_tasks=4, num_warps=4, num_stages=3)
    dt = getattr(torch, output_dtype)
    out = _run_fwd(device, a_q, b_q, sizes, sa, sb, scale, shk.GemmLayout.NN, cfg, dt)
    want = ref.ragged_fwd_reference(a_q, b_q, np.array(sizes), sa, sb)
    if output_dtype == "float32":
        assert np.array_equal(out.cpu().numpy(), want)
    else:
        assert np.array_equal(bf16_bits(torch, out), ref.bf16_round(want))


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("scale", SCALES, ids=lambda s: s.label)
@pytest.mark.parametrize("block_m", [16, 32, 64, 128])
def test_ragged_fwd_all_layouts(layout, scale, block_m, device):
    """test_ragged_dot.py:306-368: m=17, k=64, n=24, sizes [5, 0, 12]."""
    sizes = [5, 0, 12]
    a_q, b_q, sa, sb = _fwd_case(stable_seed("fwd", layout.value, scale.label, block_m), 17, 64, 24, sizes, scale)
    cfg = shk.RaggedDotConfig(block_m=block_m, block_n=16, block_k=32, group_size_tasks=2)
    out = _run_fwd(device, a_q, b_q, sizes, sa, sb, scale, layout, cfg, torch.float32)
    want = ref.ragged_fwd_reference(a_q, b_q, np.array(sizes), sa, sb,
                                    subchannel=scale.subchannel_size)
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("scale", [SCALES[0], SCALES[1], shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 64),
                                   shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 256)], ids=lambda s: s.label)
def test_ragged_fwd_even_k_and_larger(scale, device):
    """test_ragged_dot.py:448-513 (even K) plus a multi-stage K and N tail."""
    for m, k, n, sizes in ((33, 64, 24, [5, 12, 16]), (300, 512, 200, [100, 0, 37, 163])):
        if scale.subchannel_size and k % scale.subchannel_size and scale.subchannel_size > k:
            continue
        a_q, b_q, sa, sb = _fwd_case(stable_seed("even", m, scale.label), m, k, n, sizes, scale)
        out = _run_fwd(device, a_q, b_q, sizes, sa, sb, scale, shk.GemmLayout.NN, shk.RaggedDotConfig(),
                       torch.bfloat16)
        want = ref.ragged_fwd_reference(a_q, b_q, np.array(sizes), sa, sb, subchannel=scale.subchannel_size)
        assert np.array_equal(bf16_bits(torch, out), ref.bf16_round(want))


# fp6 forward (k_f6ragged.hip): every layout and output mode, through the
# native entry (128-row tasks), on shapes that exercise the row and column
# masks, K padded to 128 and the byte-wise operand loads (K/2 or M not a
# multiple of 16)
FP6_FWD_SHAPES = [(17, 64, 24, [5, 0, 12]), (300, 200, 40, [100, 0, 37, 163]),
                  (640, 384, 264, [1, 300, 0, 339]), (96, 256, 8, [96])]


def _run_fwd_native(device, a_q, b_q, sizes, sa, sb, layout, block_m, out_mode, fp6=False, subchannel=None):
    from amd_strix_halo_kernels import kernel_table as kt
    from amd_strix_halo_kernels import native
    lhs, rhs = _pack_fwd(a_q, b_q, layout)
    m, n = a_q.shape[0], b_q.shape[2]
    dt = {kt.OUT_BF16: torch.bfloat16, kt.OUT_F32: torch.float32, kt.OUT_I32: torch.int32}[out_mode]
    out = torch.full((m, n), 7, dtype=dt, device=device)
    native.launch_ragged_fwd(
        to_dev(torch, lhs, device), to_dev(torch, rhs, device), torch.tensor(sizes, dtype=torch.int32, device=device),
        a_scale=to_dev(torch, sa, device), b_scale=to_dev(torch, sb, device), out=out, layout=layout,
        subchannel=subchannel,
        block_m=block_m, align_tile=32 if fp6 else 8, rows=m, cols=n, k_packed=a_q.shape[1] // 2,
        out_mode=out_mode, fp6=fp6)
    torch.cuda.synchronize()
    return out


def _ragged_int_reference(a_q, b_q, sizes):
    out = np.zeros((a_q.shape[0], b_q.shape[2]), dtype=np.int64)
    start = 0
    for g, size in enumerate(sizes):
        out[start:start + size] = ref.int_matmul(a_q[start:start + size], b_q[g])
        start += size
    return out


@pytest.mark.parametrize("groups,align", [(5, 32), (37, 64), (1100, 32)])
@pytest.mark.parametrize("fp6", [True, False], ids=["fp6", "packed"])
def test_grouped_forward_builds_the_oracle_task_list(groups, align, fp6, device):
    """amd_strix_halo_kernels_launch_ragged_fwd_grouped: the task list it
    leaves in the caller's buffer (built inside the fp6 conversion launch for
    up to 1024 groups, by the stand-alone launch otherwise) is the oracle's
    calculate_group_info, and the output is the oracle's forward."""
    import ctypes

    from amd_strix_halo_kernels import kernel_table as kt
    from amd_strix_halo_kernels import native
    r = ref.rng(stable_seed("grouped", groups, align, fp6))
    sizes = r.integers(0, 90, size=groups)
    sizes[r.integers(0, groups)] = 0
    m, k, n = int(sizes.sum()) + 3, 128, 64
    a_q, b_q, sa, sb = _fwd_case(stable_seed("grouped-op", groups), m, k, n, list(sizes), SCALES[0])
    tile = kt.RAGGED_FP6_BLOCK_M if fp6 else 64
    desc = kt.find_ragged(kt.FAMILY_RAGGED_FWD, layout=kt.LAYOUT_NN, subchannel=None, block_m=tile, fp6=fp6)
    lib = native.load_dispatch_library()
    lhs, rhs = _pack_fwd(a_q, b_q, shk.GemmLayout.NN)
    lhs_d, rhs_d = to_dev(torch, lhs, device), to_dev(torch, rhs, device)
    sa_d, sb_d = to_dev(torch, sa, device), to_dev(torch, sb, device)
    gs = torch.tensor(sizes, dtype=torch.int32, device=device)
    cap = kt.ragged_task_capacity(m, groups, tile)
    tasks = torch.full((cap, 4), -5, dtype=torch.int32, device=device)
    count = torch.full((4,), -5, dtype=torch.int32, device=device)
    nbytes = desc.ragged_workspace_bytes(m, n, k // 2, groups)
    work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
    out = torch.full((m, n), 7, dtype=torch.float32, device=device)
    print(f"case grouped fwd groups={groups} align={align} fp6={fp6} m={m}", flush=True)
    rc = lib.amd_strix_halo_kernels_launch_ragged_fwd_grouped(
        desc.index, 0, torch.cuda.current_stream().cuda_stream, lhs_d.data_ptr(), rhs_d.data_ptr(), sa_d.data_ptr(),
        sb_d.data_ptr(), gs.data_ptr(), align, tasks.data_ptr(), count.data_ptr(), cap, out.data_ptr(), m, n, k // 2,
        groups, 0, kt.OUT_F32, work.data_ptr() if nbytes else None, ctypes.c_uint64(nbytes))
    assert rc == 0, native._library_last_error(lib)
    torch.cuda.synchronize()
    want = ref.calculate_group_info(sizes, tile, align_tile=align)
    got = tasks.cpu().numpy()
    assert int(count[0]) == want.num_tasks
    t = want.num_tasks
    for col, f in enumerate(("group_id", "block_start", "actual_start", "actual_end")):
        assert np.array_equal(got[:t, col], getattr(want, f)[:t]), f
    assert not got[t:].any()
    res = out.cpu().numpy()
    assert np.array_equal(res[:m - 3], ref.ragged_fwd_reference(a_q, b_q, sizes, sa, sb)[:m - 3])
    assert (res[m - 3:] == 7).all()  # rows past the groups are not written


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("shape", FP6_FWD_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}x{s[2]}")
def test_ragged_fwd_fp6_all_layouts_and_modes(layout, shape, device):
    from amd_strix_halo_kernels import kernel_table as kt
    m, k, n, sizes = shape
    a_q, b_q, sa, sb = _fwd_case(stable_seed("fp6fwd", layout.value, m), m, k, n, sizes, SCALES[0])
    print(f"case fp6 fwd {layout.value} {shape}", flush=True)
    want = ref.ragged_fwd_reference(a_q, b_q, np.array(sizes), sa, sb)
    got = _run_fwd_native(device, a_q, b_q, sizes, sa, sb, layout, kt.RAGGED_FP6_BLOCK_M, kt.OUT_F32, fp6=True)
    assert np.array_equal(got.cpu().numpy(), want)
    got = _run_fwd_native(device, a_q, b_q, sizes, sa, sb, layout, kt.RAGGED_FP6_BLOCK_M, kt.OUT_BF16, fp6=True)
    assert np.array_equal(bf16_bits(torch, got), ref.bf16_round(want))
    got = _run_fwd_native(device, a_q, b_q, sizes, sa, sb, layout, kt.RAGGED_FP6_BLOCK_M, kt.OUT_I32, fp6=True)
    assert np.array_equal(got.cpu().numpy().astype(np.int64), _ragged_int_reference(a_q, b_q, sizes))


# fp6 subchannel forward (the 128 x 128 subchannel tile on the task list):
# M * ceil(K/S) even (and ceil(K/32) even for groups of 32); row and column
# masks, groups that span several tiles and tiles that span two groups' rows,
# K not a multiple of 128 or of the group size (the last group ends at K)
FP6_SUB_SHAPES = [(17, 512, 24, [5, 0, 12]), (300, 512, 40, [100, 0, 37, 163]),
                  (640, 384, 264, [1, 300, 0, 339]), (96, 1024, 8, [96]), (40, 200, 24, [10, 30]),
                  (64, 2880, 40, [20, 0, 44]), (130, 96, 16, [65, 65])]


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("subchannel", [32, 64, 128, 256])
def test_ragged_fwd_fp6_subchannel(layout, subchannel, device):
    """Every group size and layout in fp32 (bit-exact: the oracle's group
    order and per-group rounding), bf16 (the fp32 result rounded once) and
    int32 (the exact sums over all K)."""
    from amd_strix_halo_kernels import kernel_table as kt
    spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, subchannel)
    for m, k, n, sizes in FP6_SUB_SHAPES:
        cols = -(-k // subchannel)
        if m * cols % 2 or (subchannel == 32 and cols % 2):
            assert not kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_FWD, subchannel=subchannel, m=m, n=n, k_packed=k // 2)
            continue
        a_q, b_q, sa, sb = _fwd_case(stable_seed("fp6sub", layout.value, subchannel, m), m, k, n, sizes, spec)
        if m == 300:
            # zero and tiny scales: the tile's folds in the reference's operation order
            sa[::7, 0] = 0
            sb[:, -1, ::5] = 0x1C80  # 2^-70
        print(f"case fp6 sub fwd {layout.value} S={subchannel} {(m, k, n, sizes)}", flush=True)
        want = ref.ragged_fwd_reference(a_q, b_q, np.array(sizes), sa, sb, subchannel=subchannel)
        run = functools.partial(_run_fwd_native, device, a_q, b_q, sizes, sa, sb, layout, kt.RAGGED_FP6_BLOCK_M,
                                fp6=True, subchannel=subchannel)
        got = run(kt.OUT_F32)
        assert np.array_equal(got.cpu().numpy(), want)
        got = run(kt.OUT_BF16)
        assert np.array_equal(bf16_bits(torch, got), ref.bf16_round(want))
        got = run(kt.OUT_I32)
        assert np.array_equal(got.cpu().numpy().astype(np.int64), _ragged_int_reference(a_q, b_q, sizes))


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("block_m", [16, 32, 64, 128])
def test_ragged_fwd_packed_per_channel_kernels(layout, block_m, device):
    """The int8-MFMA forward kernels, which the API uses for shapes the fp6
    entry does not take, on the fp6 shapes."""
    from amd_strix_halo_kernels import kernel_table as kt
    m, k, n, sizes = FP6_FWD_SHAPES[1]
    a_q, b_q, sa, sb = _fwd_case(stable_seed("pkfwd", layout.value, block_m), m, k, n, sizes, SCALES[0])
    want = ref.ragged_fwd_reference(a_q, b_q, np.array(sizes), sa, sb)
    got = _run_fwd_native(device, a_q, b_q, sizes, sa, sb, layout, block_m, kt.OUT_F32)
    assert np.array_equal(got.cpu().numpy(), want)


def test_config_c5_forward_full(device):
    """C5: G=8, M=8192, K=2048, N=1408, multinomial group sizes with an empty group."""
    r = ref.rng(5)
    sizes = ref.multinomial_group_sizes(r, 8192, 8)
    assert (sizes == 0).any() and sizes.sum() == 8192
    a_q = ref.randint4(r, (8192, 2048))
    b_q = ref.randint4(r, (8, 2048, 1408))
    sa = ref.uniform_bf16(r, (8192,), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (8, 1408), 0.005, 0.02)
    out = _run_fwd(device, a_q, b_q, sizes.tolist(), sa, sb, SCALES[0], shk.GemmLayout.NN, shk.RaggedDotConfig(),
                   torch.bfloat16)
    want = ref.ragged_fwd_reference(a_q, b_q, sizes, sa, sb)
    assert np.array_equal(bf16_bits(torch, out), ref.bf16_round(want))


@pytest.mark.parametrize("subchannel", [32, 128])
def test_config_c5_forward_full_subchannel(subchannel, device):
    """C5 with scale groups of 32 and 128 on the fp6 subchannel tile: every
    output bit-exact in bf16 (the groups folded in order)."""
    from amd_strix_halo_kernels import kernel_table as kt
    r = ref.rng(50 + subchannel)
    sizes = ref.multinomial_group_sizes(r, 8192, 8)
    cols = 2048 // subchannel
    a_q = ref.randint4(r, (8192, 2048))
    b_q = ref.randint4(r, (8, 2048, 1408))
    sa = ref.uniform_bf16(r, (8192, cols), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (8, cols, 1408), 0.005, 0.02)
    assert kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_FWD, subchannel=subchannel, m=8192, n=1408, k_packed=1024)
    print(f"case C5 forward full subchannel {subchannel}", flush=True)
    spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, subchannel)
    out = _run_fwd(device, a_q, b_q, sizes.tolist(), sa, sb, spec, shk.GemmLayout.NN, shk.RaggedDotConfig(),
                   torch.bfloat16)
    want = ref.ragged_fwd_reference(a_q, b_q, sizes, sa, sb, subchannel=subchannel)
    assert np.array_equal(bf16_bits(torch, out), ref.bf16_round(want))


# ---------------------------------------------------------------------------
# backward


def _bwd_case(seed, groups, m, kcap, n, scale):
    r = ref.rng(seed)
    a_q = ref.randint4(r, (groups, m, kcap))
    b_q = ref.randint4(r, (groups, kcap, n))
    if scale.mode is shk.ScaleMode.PER_CHANNEL:
        sa = ref.uniform_bf16(r, (groups, m), 0.008, 0.012)
        sb = ref.uniform_bf16(r, (groups, n), 0.009, 0.011)
    else:
        cols = -(-kcap // scale.subchannel_size)
        sa = ref.uniform_bf16(r, (groups, m, cols), 0.008, 0.012)
        sb = ref.uniform_bf16(r, (groups, cols, n), 0.009, 0.011)
    return a_q, b_q, sa, sb


def _run_bwd(device, a_q, b_q, sizes, sa, sb, scale, layout, split_k):
    lhs, rhs = _pack_bwd(a_q, b_q, layout)
    out = shk.ragged_dot_int4_bwd(
        to_dev(torch, lhs, device), to_dev(torch, rhs, device), torch.tensor(sizes, dtype=torch.int32, device=device),
        a_scale=to_dev(torch, sa, device), b_scale=to_dev(torch, sb, device), scale=scale,
        config=shk.RaggedBwdDotConfig(block_m=16, block_n=16, block_k=16, split_k=split_k), layout=layout)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check_bwd(got, want, scale, split_k):
    if scale.mode is shk.ScaleMode.SUBCHANNEL and split_k > 1:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-7)
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("scale", SCALES, ids=lambda s: s.label)
@pytest.mark.parametrize("split_k", [1, 2])
def test_ragged_bwd_tile_aligned(layout, scale, split_k, device):
    """test_ragged_dot.py:371-445: G=3, m=16, K cap 32, n=20, sizes [32, 0, 32]."""
    sizes = [32, 0, 32]
    a_q, b_q, sa, sb = _bwd_case(stable_seed("bwd-al", layout.value, scale.label, split_k), 3, 16, 32, 20, scale)
    got = _run_bwd(device, a_q, b_q, sizes, sa, sb, scale, layout, split_k)
    want = ref.ragged_bwd_reference(a_q, b_q, np.array(sizes), sa, sb, subchannel=scale.subchannel_size)
    _check_bwd(got, want, scale, split_k)


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("scale", SCALES, ids=lambda s: s.label)
@pytest.mark.parametrize("split_k", [1, 2])
def test_ragged_bwd_odd_k_garbage_padding(layout, scale, split_k, device):
    """test_ragged_dot.py:516-586: K cap 39, sizes [5, 0, 37]; the padding
    beyond each group's K holds random values that must not contribute."""
    sizes = [5, 0, 37]
    a_q, b_q, sa, sb = _bwd_case(stable_seed("bwd-odd", layout.value, scale.label, split_k), 3, 16, 39, 20, scale)
    got = _run_bwd(device, a_q, b_q, sizes, sa, sb, scale, layout, split_k)
    want = ref.ragged_bwd_reference(a_q, b_q, np.array(sizes), sa, sb, subchannel=scale.subchannel_size)
    _check_bwd(got, want, scale, split_k)


@pytest.mark.parametrize("split_k", [1, 3])
@pytest.mark.parametrize("scale", [SCALES[0], shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 128),
                                   shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 256)], ids=lambda s: s.label)
def test_ragged_bwd_multi_stage(scale, split_k, device):
    sizes = [700, 0, 1, 1023, 512]
    a_q, b_q, sa, sb = _bwd_case(stable_seed("bwd-ms", scale.label, split_k), 5, 200, 1024, 136, scale)
    got = _run_bwd(device, a_q, b_q, sizes, sa, sb, scale, shk.GemmLayout.NN, split_k)
    want = ref.ragged_bwd_reference(a_q, b_q, np.array(sizes), sa, sb, subchannel=scale.subchannel_size)
    _check_bwd(got, want, scale, split_k)


# fp6 backward: every layout, odd and tile-crossing K capacities with
# random values past each group's length, empty and one-row groups, M and N
# not multiples of 32
# (groups, M, K capacity, N, group sizes).  The last four split each group's
# tile grid into XCD regions: 4 x 2 with 1 and 3 column tiles (regions of 0
# and 1, 1 and 2 columns), 4 x 2 with 2, and 2 x 4 with 4.
FP6_BWD_SHAPES = [(3, 48, 39, 24, [5, 0, 37]), (5, 200, 1024, 136, [700, 0, 1, 1023, 512]),
                  (2, 264, 300, 40, [300, 129]), (3, 512, 72, 96, [40, 0, 72]), (2, 512, 136, 296, [136, 77]),
                  (2, 1024, 64, 256, [64, 1]), (4, 256, 40, 512, [0, 40, 13, 2])]


def _bwd_raw_garbage_ws(device, a_q, b_q, sizes, sa, sb, layout, subchannel):
    """The fp6 backward's raw int32 sums through the C ABI, with a workspace
    that starts as garbage: the GEMM reads only blocks the conversion wrote."""
    import ctypes

    from amd_strix_halo_kernels import kernel_table as kt
    from amd_strix_halo_kernels import native
    groups, m, n = a_q.shape[0], a_q.shape[1], b_q.shape[2]
    lhs, rhs = _pack_bwd(a_q, b_q, layout)
    kp = lhs.shape[-1] if layout in (shk.GemmLayout.NN, shk.GemmLayout.NT) else lhs.shape[1]
    desc = kt.find_ragged(kt.FAMILY_RAGGED_BWD, layout=kt.LAYOUT_CODES[layout.value], subchannel=subchannel, fp6=True)
    nbytes = desc.ragged_workspace_bytes(m, n, kp, groups)
    work = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=device)
    raw = torch.full((groups, m, n), 7, dtype=torch.int32, device=device)
    lhs_d, rhs_d = to_dev(torch, lhs, device), to_dev(torch, rhs, device)
    sa_d, sb_d = to_dev(torch, sa, device), to_dev(torch, sb, device)
    gs = torch.tensor(sizes, dtype=torch.int32, device=device)
    lib = native.load_dispatch_library()
    rc = lib.amd_strix_halo_kernels_launch_ragged_bwd_ws(
        desc.index, 0, torch.cuda.current_stream().cuda_stream, lhs_d.data_ptr(), rhs_d.data_ptr(), sa_d.data_ptr(),
        sb_d.data_ptr(), gs.data_ptr(), raw.data_ptr(), m, n, kp, groups, subchannel or 0, 1, kt.OUT_I32,
        work.data_ptr(), ctypes.c_uint64(nbytes))
    assert rc == 0, native._library_last_error(lib)
    torch.cuda.synchronize()
    return raw.cpu().numpy().astype(np.int64)


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("shape", FP6_BWD_SHAPES, ids=lambda s: f"g{s[0]}_{s[1]}x{s[2]}x{s[3]}")
def test_ragged_bwd_fp6_all_layouts(layout, shape, device):
    groups, m, kcap, n, sizes = shape
    a_q, b_q, sa, sb = _bwd_case(stable_seed("fp6bwd", layout.value, m), groups, m, kcap, n, SCALES[0])
    print(f"case fp6 bwd {layout.value} {shape}", flush=True)
    want = ref.ragged_bwd_reference(a_q, b_q, np.array(sizes), sa, sb)
    for split_k in (1, 2):  # the fp6 entry computes each output whole either way
        got = _run_bwd(device, a_q, b_q, sizes, sa, sb, SCALES[0], layout, split_k)
        assert np.array_equal(got, want)
    want_i = np.stack([ref.int_matmul(a_q[g][:, :sizes[g]], b_q[g][:sizes[g]]) for g in range(groups)])
    assert np.array_equal(_bwd_raw_garbage_ws(device, a_q, b_q, sizes, sa, sb, layout, None), want_i)


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda l: l.value)
@pytest.mark.parametrize("subchannel", [32, 64, 128, 256])
def test_ragged_bwd_fp6_subchannel(layout, subchannel, device):
    """The fp6 subchannel backward (groups of 32 to 256, K padded to 256):
    every group's scale groups up to its length folded in order, bit-exact
    for split_k 1 and 2 (each output is computed whole), and the raw int32
    sums; one shape with zero and tiny scales (the folds in the reference's
    operation order).  The scales of groups past each length are NaN: the
    reference never reads them, and neither may the kernel."""
    from amd_strix_halo_kernels import kernel_table as kt
    spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, subchannel)
    for shape in FP6_BWD_SHAPES + [(2, 33, 256, 40, [256, 100]), (3, 64, 256, 24, [33, 97, 200])]:
        groups, m, kcap, n, sizes = shape
        kp = -(-kcap // 2)
        cols = -(-2 * kp // subchannel)
        if not kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_BWD, subchannel=subchannel, m=m, n=n, k_packed=kp):
            assert m * cols % 2 or (subchannel == 32 and cols % 2)
            continue
        a_q, b_q, sa, sb = _bwd_case(stable_seed("fp6subbwd", layout.value, subchannel, m), groups, m, kcap, n, spec)
        if m == 264:
            sa[:, ::5, 0] = 0
            sb[:, -1, ::3] = 0x1C80  # 2^-70
        for g, size in enumerate(sizes):
            used = -(-size // subchannel)
            sa[g, :, used:] = 0x7FC0  # NaN
            sb[g, used:, :] = 0x7FC0
        print(f"case fp6 sub bwd {layout.value} S={subchannel} {shape}", flush=True)
        want = ref.ragged_bwd_reference(a_q, b_q, np.array(sizes), sa, sb, subchannel=subchannel)
        for split_k in (1, 2):
            got = _run_bwd(device, a_q, b_q, sizes, sa, sb, spec, layout, split_k)
            assert np.array_equal(got, want)
        want_i = np.stack([ref.int_matmul(a_q[g][:, :sizes[g]], b_q[g][:sizes[g]]) for g in range(groups)])
        assert np.array_equal(_bwd_raw_garbage_ws(device, a_q, b_q, sizes, sa, sb, layout, subchannel), want_i)


def test_config_c5_backward_full(device):
    """C5 backward: dW[g] = X_g^T dY_g, lhs [8, 2048, cap/2], rhs [8, cap/2, 1408]."""
    r = ref.rng(55)
    sizes = ref.multinomial_group_sizes(r, 8192, 8)
    cap = int(sizes.max()) + (int(sizes.max()) % 2)
    a_q = ref.randint4(r, (8, 2048, cap))
    b_q = ref.randint4(r, (8, cap, 1408))
    sa = ref.uniform_bf16(r, (8, 2048), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (8, 1408), 0.005, 0.02)
    got = _run_bwd(device, a_q, b_q, sizes.tolist(), sa, sb, SCALES[0], shk.GemmLayout.NN, 1)
    want = ref.ragged_bwd_reference(a_q, b_q, sizes, sa, sb)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("subchannel", [32, 128])
def test_config_c5_backward_full_subchannel(subchannel, device):
    """The C5 backward with scale groups of 32 and 128 on the fp6 subchannel
    tile (K capacity rounded up to 64): all of dW bit-exact, each group's
    scale groups past its length unread (NaN here)."""
    from amd_strix_halo_kernels import kernel_table as kt
    r = ref.rng(550 + subchannel)
    sizes = ref.multinomial_group_sizes(r, 8192, 8)
    cap = -(-int(sizes.max()) // 64) * 64
    cols = -(-cap // subchannel)
    a_q = ref.randint4(r, (8, 2048, cap))
    b_q = ref.randint4(r, (8, cap, 1408))
    sa = ref.uniform_bf16(r, (8, 2048, cols), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (8, cols, 1408), 0.005, 0.02)
    for g, size in enumerate(sizes.tolist()):
        used = -(-size // subchannel)
        sa[g, :, used:] = 0x7FC0
        sb[g, used:, :] = 0x7FC0
    assert kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_BWD, subchannel=subchannel, m=2048, n=1408, k_packed=cap // 2)
    print(f"case C5 backward full subchannel {subchannel}", flush=True)
    spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, subchannel)
    got = _run_bwd(device, a_q, b_q, sizes.tolist(), sa, sb, spec, shk.GemmLayout.NN, 1)
    want = ref.ragged_bwd_reference(a_q, b_q, sizes, sa, sb, subchannel=subchannel)
    assert np.array_equal(got, want)


def test_ragged_errors(device):
    gs = torch.tensor([4, 4], device=device, dtype=torch.int32)
    lhs = torch.zeros((8, 16), device=device, dtype=torch.uint8)
    rhs = torch.zeros((2, 16, 8), device=device, dtype=torch.uint8)
    with pytest.raises(ValueError, match="weight-matched layout"):
        shk.ragged_dot_int4(lhs, rhs, gs, a_scale=torch.ones((8, 1), device=device, dtype=torch.bfloat16),
                            b_scale=torch.ones((2, 8, 1), device=device, dtype=torch.bfloat16),
                            scale=shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, 32))
    with pytest.raises(ValueError, match="sum\\(group_sizes\\) must equal lhs rows 8"):
        shk.ragged_dot_int4(lhs, rhs, torch.tensor([4, 5], device=device))
    with pytest.raises(ValueError, match="non-negative"):
        shk.ragged_dot_int4(lhs, rhs, torch.tensor([12, -4], device=device))
    with pytest.raises(ValueError, match="logical padded K 32"):
        shk.ragged_dot_int4_bwd(torch.zeros((2, 8, 16), device=device, dtype=torch.uint8),
                                torch.zeros((2, 16, 8), device=device, dtype=torch.uint8),
                                torch.tensor([33, 0], device=device))
