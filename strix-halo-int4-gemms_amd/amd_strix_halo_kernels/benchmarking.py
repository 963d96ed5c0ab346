"""Throughput accounting of the reference (benchmarking.py:104-111).

TOPS = 2*M*N*K / seconds / 1e12; a fused SwiGLU call counts both GEMMs
(2*M*(2D)*K, autotune.py:971-976); the ragged backward counts
K = sum(group_sizes).
"""

from __future__ import annotations


def gemm_ops(m: int, n: int, k: int) -> int:
    return 2 * int(m) * int(n) * int(k)


def tops_for_runtime(m: int, n: int, k: int, runtime_ms: float) -> float:
    if runtime_ms <= 0:
        raise ValueError("runtime_ms must be positive")
    return gemm_ops(m, n, k) / (runtime_ms * 1.0e-3) / 1.0e12
