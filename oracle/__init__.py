"""CPU oracle for the quantized GEMM hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the numerical semantics of the reference's
torch path so that the gfx950 HIP kernels can be checked against it.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it, and only as the checker / CPU baseline.  The product
package (``amd_strix_halo_kernels``) never imports, links or executes
anything from here.

Contents
--------
``ref``      numpy restatement (pack/unpack, fake quantization, exact integer
             matmul, per-channel / subchannel scaling in the reference's op
             order, ReLU2 / SwiGLU epilogues, bf16 rounding, layouts, the
             ragged task list and the grouped ragged forward / backward,
             TOPS accounting, seeded config inputs).
``native``   ctypes loader of ``oracle.c`` (multithreaded exact int32
             matmul and the whole dense int4 NN path), used where numpy's
             integer matmul is too slow and as the CPU baseline.

Every function cites the reference file:line it follows (paths relative to
the reference repository root).  How each function is pinned (known answers
from the reference's tests, brute force, closed forms, invariants) is listed in
``tests/test_oracle.py``.
"""
