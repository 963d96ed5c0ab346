"""Skinny dense tiles (block_m 16 / 32 / 64, block_k 32; csrc/shk_skinny.h)
against the CPU oracle.

The reference registers 16- and 32-row variants of every dense tile family
(registry.py:29, 48-77) and takes int4 per-channel / SwiGLU K in multiples of
32 (registry.py:112-176); its own test selects them at M = 16 and 32
(tests/test_registry.py:206-227).  These tests run decode-sized shapes
through the public calls and the skinny table entries: bf16 outputs
bit-exact against the oracle (within 2 ulp for SwiGLU), int32 accumulators
bit-exact, including the path that splits a tile's K over several
workgroups and adds their exact int32 partials.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from tests._util import bf16_bits, dense_case, max_ulp, stable_seed, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

import amd_strix_halo_kernels as shk  # noqa: E402
from amd_strix_halo_kernels import kernel_table as kt  # noqa: E402
from amd_strix_halo_kernels import native  # noqa: E402

ULP_TOL = 2


def _spec(sub):
    return shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL) if sub is None else shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, sub)


def _dtype(bits):
    return shk.OperandDType.INT4 if bits == 4 else shk.OperandDType.INT8


def _check(got_bits, a_arg, b_arg, *, bits, layout, sa, sb, sub, epilogue):
    want = ref.reference_gemm_bf16(a_arg, b_arg, bits=bits, layout=layout, a_scale=sa, b_scale=sb,
                                   subchannel=sub, epilogue=epilogue)
    if epilogue == "swiglu":
        assert max_ulp(got_bits, want) <= ULP_TOL
    else:
        assert np.array_equal(got_bits, want)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("scale", ["pc", "sc32"])
@pytest.mark.parametrize("epilogue", ["none", "relu2", "swiglu"])
@pytest.mark.parametrize("m", [16, 32, 48])
@pytest.mark.parametrize("k", [32, 96])
def test_decode_shapes_through_the_public_calls(bits, layout, scale, epilogue, m, k, device):
    """M = 16, 32, 48 and K = 32, 96 select a skinny tile (no other tile
    accepts them) and match the oracle; the selected kernel's raw int32
    output equals the integer matmul."""
    n = 128
    sub = None if scale == "pc" else int(scale[2:])
    seed = stable_seed("skinny-api", bits, layout, scale, epilogue, m, k)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=sub,
                                                 swiglu=epilogue == "swiglu")
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    lay = shk.GemmLayout(layout)
    epi = shk.Epilogue(epilogue)
    kernel = shk.default_registry.select(dtype=_dtype(bits), scale=_spec(sub), epilogue=epi, m=m, n=n, k=k,
                                         layout=lay)
    assert kt.TABLE[kernel.table_index].operand_format == kt.OPERANDS_STREAM
    assert m % kernel.tile.block_m == 0 and kernel.tile.block_m == (16 if m == 48 else m)
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    if epilogue == "swiglu":
        out = shk.fused_swiglu_up_gate(a, b, a_scale=ta, b_scale=tb, dtype=_dtype(bits), layout=lay, scale=_spec(sub))
    else:
        out = shk.mm(a, b, a_scale=ta, b_scale=tb, dtype=_dtype(bits), layout=lay, scale=_spec(sub), epilogue=epi)
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (m, n)
    assert np.array_equal(raw.cpu().numpy(), ref.int_matmul(a_q, b_q))
    _check(bf16_bits(torch, out), a_arg, b_arg, bits=bits, layout=layout, sa=sa, sb=sb, sub=sub, epilogue=epilogue)


def _stream_kernel(bits, layout, r, *, sub=None, epilogue="none", schedule=shk.KernelSchedule.STANDARD, split=1):
    for kern in shk.default_registry.all():
        d = kt.TABLE[kern.table_index]
        if (d.is_stream and d.dtype_bits == bits and kern.layout.value == layout and d.block_m == r
                and kern.scale == _spec(sub) and kern.epilogue.value == epilogue and kern.schedule is schedule
                and kern.tile.split_k == split):
            return kern
    raise LookupError((bits, layout, r, sub, epilogue, schedule, split))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("r", [16, 32, 64])
@pytest.mark.parametrize("epilogue", ["none", "swiglu"])
def test_split_k_over_workgroups_is_exact(bits, layout, r, epilogue, device):
    """A shape with few tiles and a long K: the launcher splits each tile's
    K over several workgroups (the last to arrive adds the exact int32
    partials).  Every output equals the oracle's, and a second and third
    call reuse the per-stream workspace (its counters were left zero)."""
    m, n, k = r, 128, 8192 + 32
    desc = kt.TABLE[_stream_kernel(bits, layout, r, epilogue=epilogue).table_index]
    assert kt.sk_split_count(desc, m, n, k) > 1
    seed = stable_seed("skinny-split", bits, layout, r, epilogue)
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=m, n=n, k=k, subchannel=None,
                                                 swiglu=epilogue == "swiglu")
    kernel = _stream_kernel(bits, layout, r, epilogue=epilogue)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    print(f"case {kernel.kernel_id} shape=({m},{n},{k}) splits={kt.sk_split_count(desc, m, n, k)}", flush=True)
    outs = [shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb) for _ in range(3)]
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), ref.int_matmul(a_q, b_q))
    first = bf16_bits(torch, outs[0])
    for o in outs[1:]:
        assert np.array_equal(bf16_bits(torch, o), first)
    _check(first, a_arg, b_arg, bits=bits, layout=layout, sa=sa, sb=sb, sub=None, epilogue=epilogue)


def test_split_launches_of_different_shapes_share_the_workspace(device):
    """Split launches of several shapes in a row on one stream share its
    workspace.  The counters of a shape with more tiles lie where a shape
    with fewer tiles kept its partials, so each launch must leave all of the
    workspace it used zero: every output is exact and the workspace reads
    all zero after every call."""
    shapes = [(16, 128, 8192 + 32), (16, 8192, 8192), (32, 256, 4096), (16, 4096, 8192), (16, 128, 8192 + 32)]
    key = (device.index or 0, torch.cuda.current_stream(device).cuda_stream)
    for i, (m, n, k) in enumerate(shapes):
        kernel = _stream_kernel(4, "nn", m)
        assert kt.sk_split_count(kt.TABLE[kernel.table_index], m, n, k) > 1
        a_q, b_q, a_arg, b_arg, sa, sb = dense_case(stable_seed("skinny-reuse", i), bits=4, layout="nn", m=m, n=n,
                                                     k=k, subchannel=None, swiglu=False)
        a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
        ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
        print(f"case {kernel.kernel_id} shape=({m},{n},{k}) splits="
              f"{kt.sk_split_count(kt.TABLE[kernel.table_index], m, n, k)}", flush=True)
        raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
        torch.cuda.synchronize()
        assert np.array_equal(raw.cpu().numpy(), ref.int_matmul(a_q, b_q)), (m, n, k)
        assert int(native._SPLIT_WORKSPACES[key].count_nonzero()) == 0, (m, n, k)


def test_headline_skinny_shape_every_output(device):
    """M = 16, N = K = 8192 int4 per-channel (the skinny bench line): every
    output bit-exact, on the split path (2 workgroups per tile)."""
    m, n, k = 16, 8192, 8192
    seed = stable_seed("skinny-headline")
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=4, layout="nn", m=m, n=n, k=k, subchannel=None,
                                                 swiglu=False)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=_spec(None), epilogue=shk.Epilogue.NONE,
                                         m=m, n=n, k=k)
    assert kernel.tile.block_m == 16 and kt.sk_split_count(kt.TABLE[kernel.table_index], m, n, k) == 2
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    out = shk.mm(a, b, a_scale=ta, b_scale=tb)
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), ref.int_matmul(a_q, b_q))
    _check(bf16_bits(torch, out), a_arg, b_arg, bits=4, layout="nn", sa=sa, sb=sb, sub=None, epilogue="none")


def test_int4_long_k_needs_the_split_and_stays_exact(device):
    """int4 waves hold 256 * sum in int32, so one wave takes at most 1023
    stages of 128 K: K = 4 * 1023 * 128 + 128 needs two workgroups per tile
    even for a single tile.  Row 0 of A and column 0 of B hold -8, so
    out[0, 0] = 64 * K.  Without a workspace the C ABI refuses that K."""
    m, n = 16, 64
    k = 4 * 1023 * 128 + 128
    kernel = _stream_kernel(4, "nn", 16)
    desc = kt.TABLE[kernel.table_index]
    assert kt.sk_split_count(desc, m, n, k, with_workspace=False) == 0
    assert kt.sk_split_count(desc, m, n, k) >= 2
    r = ref.rng(stable_seed("skinny-long-k"))
    a_q = ref.randint4(r, (m, k))
    b_q = ref.randint4(r, (k, n))
    a_q[0, :] = -8
    b_q[:, 0] = -8
    a_arg, b_arg = ref.pack_operands(a_q, b_q, bits=4, layout="nn")
    sa = ref.uniform_bf16(r, (m,), 0.005, 0.02)
    sb = ref.uniform_bf16(r, (n,), 0.005, 0.02)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    print(f"case {kernel.kernel_id} shape=({m},{n},{k})", flush=True)
    out = shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
    torch.cuda.synchronize()
    prod = ref.int_matmul(a_q, b_q)
    assert prod[0, 0] == 64 * k
    assert np.array_equal(raw.cpu().numpy(), prod)
    _check(bf16_bits(torch, out), a_arg, b_arg, bits=4, layout="nn", sa=sa, sb=sb, sub=None, epilogue="none")
    lib = native.load_dispatch_library()
    c = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    rc = lib.amd_strix_halo_kernels_launch_gemm(kernel.table_index, 0, 0, a.data_ptr(), b.data_ptr(), ta.data_ptr(),
                                                tb.data_ptr(), c.data_ptr(), m, n, k, 0, kt.EPILOGUE_NONE, kt.OUT_BF16)
    assert rc == 1 and b"needs a workspace" in lib.amd_strix_halo_kernels_last_error()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("sub", [32, 64, 128, 256])
@pytest.mark.parametrize("r", [16, 32, 64])
def test_subchannel_groups_fold_in_order(bits, layout, sub, r, device):
    """Subchannel skinny tiles add every group's scaled partial in group
    order (api.py:311-325): bit-exact for 1, 3, 9 and 37 groups of each size
    (37: several rounds of the four waves' group chunks, the last one
    partial), with scales over three decades."""
    n = 128
    for groups in (1, 3, 9, 37):
        k = groups * sub
        seed = stable_seed("skinny-sc", bits, layout, sub, r, groups)
        a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=r, n=n, k=k, subchannel=sub,
                                                     swiglu=False, scale_lo=1e-4, scale_hi=0.1)
        kernel = _stream_kernel(bits, layout, r, sub=sub)
        a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
        ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
        print(f"case {kernel.kernel_id} shape=({r},{n},{k})", flush=True)
        out = shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
        raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
        torch.cuda.synchronize()
        assert np.array_equal(raw.cpu().numpy(), ref.int_matmul(a_q, b_q))
        _check(bf16_bits(torch, out), a_arg, b_arg, bits=bits, layout=layout, sa=sa, sb=sb, sub=sub,
               epilogue="none")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("sub", [32, 128])
@pytest.mark.parametrize("r", [16, 32])
def test_subchannel_swiglu_groups_fold_in_order(bits, layout, sub, r, device):
    """The SwiGLU subchannel skinny tiles (up and gate columns, two column
    tiles per wave): 3 and 37 groups, int32 sums exact, outputs within 2 ulp."""
    n = 64
    for groups in (3, 37):
        k = groups * sub
        seed = stable_seed("skinny-sc-swiglu", bits, layout, sub, r, groups)
        a_q, b_q, a_arg, b_arg, sa, sb = dense_case(seed, bits=bits, layout=layout, m=r, n=n, k=k, subchannel=sub,
                                                     swiglu=True, scale_lo=1e-4, scale_hi=0.1)
        kernel = _stream_kernel(bits, layout, r, sub=sub, epilogue="swiglu")
        a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
        ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
        print(f"case {kernel.kernel_id} shape=({r},{n},{k})", flush=True)
        out = shk.explicit_mm(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
        raw = native.launch_generated_kernel_i32(a, b, kernel=kernel, a_scale=ta, b_scale=tb)
        torch.cuda.synchronize()
        assert np.array_equal(raw.cpu().numpy(), ref.int_matmul(a_q, b_q))
        _check(bf16_bits(torch, out), a_arg, b_arg, bits=bits, layout=layout, sa=sa, sb=sb, sub=sub,
               epilogue="swiglu")


def test_subchannel_a_scale_at_a_two_byte_offset(device):
    """The subchannel scale loads read dwords: an a_scale tensor that starts
    2 bytes past a 4-byte boundary (a view at element 1) still gives every
    row its own group scales."""
    m, n, k, sub = 16, 64, 96, 32
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(stable_seed("skinny-mis"), bits=4, layout="nn", m=m, n=n, k=k,
                                                 subchannel=sub, swiglu=False)
    kernel = _stream_kernel(4, "nn", 16, sub=sub)
    backing = to_dev(torch, np.concatenate([np.zeros(1, np.uint16), sa.reshape(-1)]), device)
    ta = backing[1:].view(m, k // sub)
    assert ta.data_ptr() % 4 == 2
    out = shk.explicit_mm(to_dev(torch, a_arg, device), to_dev(torch, b_arg, device), kernel=kernel, a_scale=ta,
                          b_scale=to_dev(torch, sb, device))
    torch.cuda.synchronize()
    _check(bf16_bits(torch, out), a_arg, b_arg, bits=4, layout="nn", sa=sa, sb=sb, sub=sub, epilogue="none")


@pytest.mark.parametrize("sub", [None, 64])
def test_persistent_skinny_tiles(sub, device):
    """mm(schedule=PERSISTENT) at M = 16: the persistent launch strides over
    (split, tile) units and matches the standard schedule bit for bit."""
    m, n, k = 16, 4096, 4096
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(stable_seed("skinny-persistent", sub), bits=4, layout="nn", m=m, n=n,
                                                 k=k, subchannel=sub, swiglu=False)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    out_p = shk.mm(a, b, a_scale=ta, b_scale=tb, scale=_spec(sub), schedule=shk.KernelSchedule.PERSISTENT)
    out_s = shk.mm(a, b, a_scale=ta, b_scale=tb, scale=_spec(sub))
    torch.cuda.synchronize()
    got = bf16_bits(torch, out_p)
    assert np.array_equal(got, bf16_bits(torch, out_s))
    _check(got, a_arg, b_arg, bits=4, layout="nn", sa=sa, sb=sb, sub=sub, epilogue="none")


def test_split_launches_replay_in_a_graph(device):
    """A split skinny launch captured in a HIP graph and replayed: the
    counters it leaves at zero let every replay finish the same way.  Eager
    work and synchronizations run between the replays, and every replay is
    checked against the eager result."""
    m, n, k = 16, 1024, 8192
    a_q, b_q, a_arg, b_arg, sa, sb = dense_case(stable_seed("skinny-graph"), bits=4, layout="nn", m=m, n=n, k=k,
                                                 subchannel=None, swiglu=False)
    a, b = to_dev(torch, a_arg, device), to_dev(torch, b_arg, device)
    ta, tb = to_dev(torch, sa, device), to_dev(torch, sb, device)
    kernel = _stream_kernel(4, "nn", 16)
    assert kt.sk_split_count(kt.TABLE[kernel.table_index], m, n, k) > 1
    out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm-up: the stream's workspace is allocated and zeroed
        native.launch_generated_kernel(a, b, kernel=kernel, a_scale=ta, b_scale=tb, c=out)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    eager = bf16_bits(torch, out)
    _check(eager, a_arg, b_arg, bits=4, layout="nn", sa=sa, sb=sb, sub=None, epilogue="none")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        native.launch_generated_kernel(a, b, kernel=kernel, a_scale=ta, b_scale=tb, c=out)
    for i in range(3):
        out.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(torch, out), eager), f"replay {i}"
        shk.mm(a, b, a_scale=ta, b_scale=tb)  # eager work between replays
        torch.cuda.synchronize()
