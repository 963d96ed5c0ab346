"""GPU parity of the device quantization and int4 packing.

The reference's fake_quant_int and pack_int4_k_major (quant.py:14-51) are
torch element-wise code, so on a CUDA tensor the reference's result is what
torch computes on the GPU.  The public functions run the library's one-pass
HIP kernel on CUDA tensors; every case compares its output bit for bit

* with the reference's formula evaluated by torch on the same CUDA tensor, and
* with the oracle (``fake_quant_int_device``, ``pack_int4_k_major``) on the
  CPU, which pins the oracle's rule for torch's GPU division on this hardware.

Cases cover float32 / float16 / bfloat16 sources, scales whose reciprocal is
and is not exact, odd row and column counts, strided and misaligned views,
batched tensors, NaN / +-inf / ties, both packing axes, the full C2 operand
size, and an mm() call on the packed operands.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ref
from tests._util import stable_seed

torch = pytest.importorskip("torch")

import amd_strix_halo_kernels as shk  # noqa: E402

pytestmark = pytest.mark.gpu

DTYPES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
SHAPES = [(1, 1), (3, 5), (7, 33), (2, 16), (64, 1000), (513, 257), (128, 4096)]
SCALES = [0.1, 0.017, 0.001, 3.7, 0.125]


def _ref_codes(x, bits, scale):
    """The reference's fake_quant_int formula (quant.py:26-29), run by torch."""
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return torch.clamp(torch.round(x.float() / scale), lo, hi).to(torch.int8)


def _ref_pack(q):
    """The reference's pack_int4_k_major formula (quant.py:32-38), run by torch."""
    if q.shape[-1] % 2:
        q = torch.nn.functional.pad(q, (0, 1))
    even = q[..., 0::2].to(torch.int16) & 0xF
    odd = q[..., 1::2].to(torch.int16) & 0xF
    return ((odd << 4) | even).to(torch.uint8).contiguous()


def _values(shape, scale, bits, seed, dtype, device):
    """Values spanning the code range and past it, with special values."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * (scale * (1 << (bits - 1)) * 0.6)
    flat = x.view(-1)
    special = torch.tensor([float("nan"), float("inf"), float("-inf"), 0.0, -0.0, 0.5 * scale, 1.5 * scale,
                            -2.5 * scale, 1e30, -1e30])
    n = min(flat.numel(), special.numel())
    flat[:n] = special[:n]
    return x.to(dtype).to(device)


@pytest.mark.parametrize("dtype", list(DTYPES), ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("scale", SCALES, ids=str)
@pytest.mark.parametrize("bits", [4, 8])
def test_fake_quant_int_matches_torch_on_the_gpu(dtype, shape, scale, bits, device):
    x = _values(shape, scale, bits, stable_seed("fake_quant", dtype, shape, scale, bits), DTYPES[dtype], device)
    print(f"case fake_quant {dtype} {shape} scale={scale} bits={bits}", flush=True)
    got = shk.fake_quant_int(x, bits=bits, scale=scale)
    want = _ref_codes(x, bits, scale)
    torch.cuda.synchronize()
    assert got.dtype == torch.int8 and got.shape == x.shape
    assert torch.equal(got, want)
    assert np.array_equal(got.cpu().numpy(), ref.fake_quant_int_device(x.float().cpu().numpy(), bits=bits,
                                                                       scale=scale))


@pytest.mark.parametrize("shape", [(1, 1), (1, 2), (5, 7), (3, 4, 9), (2, 3, 64), (300, 1001)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", ["int8", "int32", "uint8"])
def test_pack_int4_k_major_matches_torch_on_the_gpu(shape, dtype, device):
    g = torch.Generator().manual_seed(sum(shape) * 7 + len(dtype))
    codes = torch.randint(-8, 8, shape, generator=g, dtype=torch.int32)
    if dtype == "int32":
        codes.view(-1)[::11] += 16 * torch.randint(-5, 5, codes.view(-1)[::11].shape, generator=g, dtype=torch.int32)
    q = codes.to(getattr(torch, dtype) if dtype != "uint8" else torch.int32)
    if dtype == "uint8":
        q = (q & 0xFF).to(torch.uint8)
    q = q.to(device)
    print(f"case pack {dtype} {shape}", flush=True)
    got = shk.pack_int4_k_major(q)
    want = _ref_pack(q)
    torch.cuda.synchronize()
    assert got.dtype == torch.uint8 and tuple(got.shape) == tuple(want.shape)
    assert torch.equal(got, want)
    assert np.array_equal(got.cpu().numpy(), ref.pack_int4_k_major(q.cpu().numpy().astype(np.int64).astype(np.int8)))


@pytest.mark.parametrize("axis", [-1, -2])
@pytest.mark.parametrize("shape", [(4, 6), (5, 7), (33, 130), (3, 5, 7), (2, 6, 40), (1024, 1024)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_quantize_pack_int4_both_axes(axis, shape, dtype, device):
    scale = 0.017
    x = _values(shape, scale, 4, sum(shape) + axis, DTYPES[dtype], device)
    print(f"case quantize_pack axis={axis} {dtype} {shape}", flush=True)
    got = shk.quantize_pack_int4(x, scale=scale, axis=axis)
    q = _ref_codes(x, 4, scale)
    want = _ref_pack(q) if axis == -1 else _ref_pack(q.transpose(-1, -2)).transpose(-1, -2).contiguous()
    torch.cuda.synchronize()
    assert tuple(got.shape) == tuple(want.shape)
    assert torch.equal(got, want)


def test_views_strided_and_misaligned(device):
    """A row-strided view and a view starting one element past an aligned
    address (the element-wise load path) quantize like torch."""
    base = _values((65, 131), 0.1, 4, 5, torch.bfloat16, device)
    for view in (base[1:, 3:], base[:, ::1][2:40, 1:100], base.t()[:50, :60]):
        print(f"case view {tuple(view.shape)} strides {view.stride()}", flush=True)
        assert torch.equal(shk.fake_quant_int(view, bits=4, scale=0.1), _ref_codes(view, 4, 0.1))
        assert torch.equal(shk.quantize_pack_int4(view, scale=0.1), _ref_pack(_ref_codes(view, 4, 0.1)))


def test_c2_operand_size(device):
    """The full C2 operands: 8192 x 8192 bf16 values packed along each axis."""
    g = torch.Generator(device=device).manual_seed(9)
    x = (torch.randn((8192, 8192), generator=g, device=device) * 0.05).to(torch.bfloat16)
    print("case c2 size", flush=True)
    q = _ref_codes(x, 4, 0.01)
    assert torch.equal(shk.quantize_pack_int4(x, scale=0.01), _ref_pack(q))
    assert torch.equal(shk.quantize_pack_int4(x, scale=0.01, axis=-2), _ref_pack(q.t()).t().contiguous())


def test_packed_operands_feed_mm(device):
    """Operands quantized and packed on the device give mm() the same result
    as operands packed by the reference formulas (README quick start)."""
    g = torch.Generator(device=device).manual_seed(3)
    m, n, k = 512, 512, 1024
    a = (torch.randn((m, k), generator=g, device=device) * 0.1).to(torch.bfloat16)
    b = (torch.randn((k, n), generator=g, device=device) * 0.1).to(torch.bfloat16)
    sa = torch.full((m,), 0.01, device=device, dtype=torch.bfloat16)
    sb = torch.full((n,), 0.02, device=device, dtype=torch.bfloat16)
    print("case packed operands into mm", flush=True)
    a_dev, b_dev = shk.quantize_pack_int4(a, scale=0.1), shk.quantize_pack_int4(b, scale=0.1, axis=-2)
    a_ref = _ref_pack(_ref_codes(a, 4, 0.1))
    b_ref = _ref_pack(_ref_codes(b, 4, 0.1).t()).t().contiguous()
    assert torch.equal(a_dev, a_ref) and torch.equal(b_dev, b_ref)
    got = shk.mm(a_dev, b_dev, a_scale=sa, b_scale=sb)
    want = shk.mm(a_ref, b_ref, a_scale=sa, b_scale=sb)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
