"""Writes tests/golden/reference_vectors.npz from the reference's own CPU path.

The oracle's scaling / epilogue op order and its task-list builder are checked
bit for bit against vectors produced by the reference package itself:
``amd_strix_halo_kernels.api.reference_mm`` (api.py:257-325) through
``mm`` / ``fused_swiglu_up_gate`` with ``use_reference=True``, and the torch
branch of ``calculate_group_info`` (ragged.py:307-323).  Run in a container
that has the reference checkout; the GPU box never runs this script.

    python tests/golden/make_golden.py /root/reference

Only inputs and outputs are stored (packed operands, bf16 bit patterns, group
sizes and task arrays); nothing of the reference's source is kept.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np


def _seed(text: str) -> int:
    return int.from_bytes(hashlib.sha256(text.encode()).digest()[:4], "little")


def main(reference_root: str) -> None:
    sys.path.insert(0, str(Path(reference_root) / "src"))
    import torch
    from amd_strix_halo_kernels import (  # the reference package
        Epilogue,
        GemmLayout,
        OperandDType,
        ScaleMode,
        ScaleSpec,
        calculate_group_info,
        fused_swiglu_up_gate,
        mm,
    )
    from amd_strix_halo_kernels.quant import fake_quant_int, pack_int4_k_major

    out: dict[str, np.ndarray] = {}
    cases = []
    shapes = {4: (16, 32, 128), 8: (16, 32, 128)}
    for bits in (4, 8):
        dtype = OperandDType.INT4 if bits == 4 else OperandDType.INT8
        for layout in ("nn", "nt", "tn"):
            for scale in ("pc", "sc32", "sc64", "sc128"):
                for epilogue in ("none", "relu2", "swiglu"):
                    name = f"b{bits}_{layout}_{scale}_{epilogue}"
                    g = torch.Generator().manual_seed(_seed(name))
                    m, n, k = shapes[bits]
                    b_cols = 2 * n if epilogue == "swiglu" else n
                    a = torch.randn((m, k), generator=g, dtype=torch.float32).to(torch.bfloat16) * 0.1
                    b = torch.randn((k, b_cols), generator=g, dtype=torch.float32).to(torch.bfloat16) * 0.1
                    a_q = fake_quant_int(a, bits=bits, scale=0.02 if bits == 8 else 0.1)
                    b_q = fake_quant_int(b, bits=bits, scale=0.02 if bits == 8 else 0.1)
                    spec = ScaleSpec(ScaleMode.PER_CHANNEL) if scale == "pc" else ScaleSpec(
                        ScaleMode.SUBCHANNEL, int(scale[2:]))
                    if scale == "pc":
                        sa = (torch.rand((m,), generator=g) * 0.015 + 0.005).to(torch.bfloat16)
                        sb = (torch.rand((b_cols,), generator=g) * 0.015 + 0.005).to(torch.bfloat16)
                    else:
                        cols = -(-k // spec.subchannel_size)
                        sa = (torch.rand((m, cols), generator=g) * 0.015 + 0.005).to(torch.bfloat16)
                        sb = (torch.rand((cols, b_cols), generator=g) * 0.015 + 0.005).to(torch.bfloat16)
                    a_t = layout == "tn"
                    b_t = layout == "nt"
                    if bits == 4:
                        a_arg = pack_int4_k_major(a_q)
                        a_arg = a_arg.transpose(0, 1).contiguous() if a_t else a_arg
                        b_arg = pack_int4_k_major(b_q.transpose(0, 1))
                        b_arg = b_arg if b_t else b_arg.transpose(0, 1).contiguous()
                    else:
                        a_arg = a_q.transpose(0, 1).contiguous() if a_t else a_q
                        b_arg = b_q.transpose(0, 1).contiguous() if b_t else b_q
                    lay = GemmLayout(layout)
                    if epilogue == "swiglu":
                        res = fused_swiglu_up_gate(a_arg, b_arg, a_scale=sa, b_scale=sb, dtype=dtype, layout=lay,
                                                   scale=spec, use_reference=True)
                    else:
                        res = mm(a_arg, b_arg, a_scale=sa, b_scale=sb, dtype=dtype, layout=lay, scale=spec,
                                 epilogue=Epilogue(epilogue), use_reference=True)
                    out[f"{name}.a"] = a_arg.numpy()
                    out[f"{name}.b"] = b_arg.numpy()
                    out[f"{name}.a_scale"] = sa.view(torch.int16).numpy().view(np.uint16)
                    out[f"{name}.b_scale"] = sb.view(torch.int16).numpy().view(np.uint16)
                    out[f"{name}.out"] = res.view(torch.int16).numpy().view(np.uint16)
                    cases.append(name)
    out["dense_cases"] = np.array(cases)

    gi_cases = []
    rng = np.random.default_rng(_seed("group-info"))
    specs = [([17, 31, 24], 32, None, 8), ([2, 0, 7], 16, 4, 8), ([300, 0, 1000, 17, 2779], 64, None, 8),
             ([1] * 16, 32, None, 8), ([7, 9, 0, 40], 16, None, 8), ([512] * 8, 64, 600, 8)]
    for i in range(6):
        sizes = rng.integers(0, 200, size=int(rng.integers(1, 12))).tolist()
        specs.append((sizes, int(rng.choice([16, 32, 64, 128])), None, int(rng.choice([4, 8, 16]))))
    for i, (sizes, tile, tid, align) in enumerate(specs):
        if tile % align:
            align = 8
        info = calculate_group_info(torch.tensor(sizes, dtype=torch.int32), tile, tid_size=tid, align_tile=align,
                                    allow_triton=False)
        key = f"gi{i}"
        out[f"{key}.sizes"] = np.array(sizes, dtype=np.int64)
        out[f"{key}.params"] = np.array([tile, -1 if tid is None else tid, align, info.num_tasks], dtype=np.int64)
        out[f"{key}.fields"] = np.stack([t.numpy() for t in (info.group_id, info.block_start, info.actual_start,
                                                             info.actual_end, info.start_within_block,
                                                             info.actual_size)])
        gi_cases.append(key)
    out["group_info_cases"] = np.array(gi_cases)
    dst = Path(__file__).resolve().parent / "reference_vectors.npz"
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({len(cases)} dense cases, {len(gi_cases)} group-info cases)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
