"""Benchmark records, the JSON benchmark database and device timing.

The record and database types keep the reference's schema
(benchmarking.py:13-99), so a database file written by either side loads in
the other: ``{"records": [{"kernel_id", "shape": {"m", "n", "k"},
"runtime_ms", "tops", "iterations", "warmup", "success", "max_abs_diff",
"max_rel_diff", "notes", "metadata"}]}``.

Throughput accounting follows benchmarking.py:102-111: TOPS = 2*M*N*K /
seconds / 1e12.  A fused SwiGLU call counts both GEMMs (autotune.py:971-976);
the ragged backward counts K = sum(group_sizes).

Device timing: the reference samples with ``triton.testing.do_bench``
(benchmarking.py:138-152), which this image does not have.
``device_event_samples`` does the same job with HIP events recorded on the
current stream around every call: a short estimate sets the number of warm-up
and timed calls from ``warmup_ms`` / ``rep_ms``, and a 256 MiB buffer is
rewritten before every timed call so that no call starts with its operands in
the L2 caches or the last-level cache (as do_bench does).  The reference's
names ``triton_do_bench_samples`` and ``benchmark_triton_callable`` are
aliases of the HIP-event functions.
"""

from __future__ import annotations

import json
import statistics
import time
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any, Callable, Iterable

from .metadata import KernelMetadata

TIMING_BACKEND = "hip_events"
CACHE_FLUSH_BYTES = 256 << 20
MAX_TIMED_CALLS = 10_000


@dataclass(frozen=True, slots=True)
class BenchmarkShape:
    m: int
    n: int
    k: int

    def to_dict(self) -> dict[str, int]:
        return {"m": self.m, "n": self.n, "k": self.k}

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "BenchmarkShape":
        return cls(m=int(data["m"]), n=int(data["n"]), k=int(data["k"]))


@dataclass(frozen=True, slots=True)
class BenchmarkRecord:
    kernel_id: str
    shape: BenchmarkShape
    runtime_ms: float
    tops: float
    iterations: int
    warmup: int
    success: bool = True
    max_abs_diff: float | None = None
    max_rel_diff: float | None = None
    notes: str = ""
    metadata: dict[str, Any] = field(default_factory=dict)

    def to_dict(self) -> dict[str, Any]:
        out = asdict(self)
        out["shape"] = self.shape.to_dict()
        return out

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "BenchmarkRecord":
        def opt_float(key: str) -> float | None:
            value = data.get(key)
            return None if value is None else float(value)

        return cls(
            kernel_id=str(data["kernel_id"]),
            shape=BenchmarkShape.from_dict(data["shape"]),
            runtime_ms=float(data["runtime_ms"]),
            tops=float(data["tops"]),
            iterations=int(data["iterations"]),
            warmup=int(data["warmup"]),
            success=bool(data.get("success", True)),
            max_abs_diff=opt_float("max_abs_diff"),
            max_rel_diff=opt_float("max_rel_diff"),
            notes=str(data.get("notes", "")),
            metadata=dict(data.get("metadata", {})),
        )


class BenchmarkDatabase:
    """An append-only list of records with the lookups autotuning needs."""

    def __init__(self, records: Iterable[BenchmarkRecord] = ()) -> None:
        self._records: list[BenchmarkRecord] = list(records)

    def add(self, record: BenchmarkRecord) -> None:
        self._records.append(record)

    def records(self) -> tuple[BenchmarkRecord, ...]:
        return tuple(self._records)

    def matching_records(self, kernel: KernelMetadata, shape: BenchmarkShape) -> tuple[BenchmarkRecord, ...]:
        """Successful records of ``kernel`` at exactly ``shape``."""
        return tuple(r for r in self._records if r.success and r.kernel_id == kernel.kernel_id and r.shape == shape)

    def best_record(self, kernel: KernelMetadata, shape: BenchmarkShape) -> BenchmarkRecord | None:
        found = self.matching_records(kernel, shape)
        return max(found, key=lambda r: r.tops) if found else None

    def to_dict(self) -> dict[str, Any]:
        return {"records": [r.to_dict() for r in self._records]}

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "BenchmarkDatabase":
        return cls(BenchmarkRecord.from_dict(r) for r in data.get("records", []))

    @classmethod
    def load(cls, path: Path | str) -> "BenchmarkDatabase":
        return cls.from_dict(json.loads(Path(path).read_text()))

    def save(self, path: Path | str) -> None:
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(self.to_dict(), indent=2, sort_keys=True) + "\n")


def gemm_ops(shape: BenchmarkShape) -> int:
    return 2 * int(shape.m) * int(shape.n) * int(shape.k)


def tops_for_runtime(shape: BenchmarkShape, runtime_ms: float) -> float:
    if runtime_ms <= 0:
        raise ValueError("runtime_ms must be positive")
    return gemm_ops(shape) / (runtime_ms * 1.0e-3) / 1.0e12


def _quantile(sorted_values: list[float], q: float) -> float:
    """Linear interpolation between the two nearest ranks (numpy's default)."""
    if not 0.0 <= q <= 1.0:
        raise ValueError("quantile must be between 0 and 1")
    pos = q * (len(sorted_values) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(sorted_values) - 1)
    frac = pos - lo
    return sorted_values[lo] + frac * (sorted_values[hi] - sorted_values[lo])


def summarize_runtime_samples(samples_ms: Iterable[float]) -> dict[str, float | int]:
    """Summary statistics of per-call times; non-positive samples are dropped
    and counted (benchmarking.py:125-135 keys)."""
    raw = [float(s) for s in samples_ms]
    if not raw:
        raise ValueError("at least one runtime sample is required")
    kept = sorted(s for s in raw if s > 0.0)
    if not kept:
        raise ValueError("at least one positive runtime sample is required")
    return {
        "sample_count": len(kept),
        "raw_sample_count": len(raw),
        "dropped_nonpositive_sample_count": len(raw) - len(kept),
        "runtime_ms_min": kept[0],
        "runtime_ms_p20": _quantile(kept, 0.20),
        "runtime_ms_median": statistics.median(kept),
        "runtime_ms_mean": statistics.mean(kept),
        "runtime_ms_p80": _quantile(kept, 0.80),
        "runtime_ms_max": kept[-1],
    }


def device_event_samples(
    fn: Callable[[], Any],
    *,
    warmup_ms: int = 25,
    rep_ms: int = 100,
    flush_cache: bool = True,
) -> tuple[float, ...]:
    """Per-call device times in ms of ``fn`` on the current stream."""
    if warmup_ms < 0:
        raise ValueError("warmup_ms must be non-negative")
    if rep_ms <= 0:
        raise ValueError("rep_ms must be positive")
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("device timing requires a GPU")
    flush = torch.empty(CACHE_FLUSH_BYTES // 4, dtype=torch.int32, device="cuda") if flush_cache else None
    fn()
    torch.cuda.synchronize()
    # estimate one call from five back-to-back calls
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(5):
        if flush is not None:
            flush.zero_()
        fn()
    t1.record()
    torch.cuda.synchronize()
    estimate = max(t0.elapsed_time(t1) / 5.0, 1.0e-3)
    n_warm = max(1, int(warmup_ms / estimate))
    n_rep = min(MAX_TIMED_CALLS, max(1, int(rep_ms / estimate)))
    for _ in range(n_warm):
        fn()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    for i in range(n_rep):
        if flush is not None:
            flush.zero_()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return tuple(float(s.elapsed_time(e)) for s, e in zip(starts, ends))


def benchmark_device_callable(
    *,
    kernel: KernelMetadata,
    shape: BenchmarkShape,
    fn: Callable[[], Any],
    warmup_ms: int = 25,
    rep_ms: int = 100,
    metadata: dict[str, Any] | None = None,
    notes: str = "",
) -> BenchmarkRecord:
    """One record from HIP-event samples; runtime is the median sample
    (benchmarking.py:155-186)."""
    summary = summarize_runtime_samples(device_event_samples(fn, warmup_ms=warmup_ms, rep_ms=rep_ms))
    runtime = float(summary["runtime_ms_median"])
    meta: dict[str, Any] = {"timing_backend": TIMING_BACKEND, "timing_return_mode": "all",
                            "warmup_ms": warmup_ms, "rep_ms": rep_ms, **summary}
    meta.update(metadata or {})
    return BenchmarkRecord(kernel_id=kernel.kernel_id, shape=shape, runtime_ms=runtime,
                           tops=tops_for_runtime(shape, runtime), iterations=int(summary["sample_count"]),
                           warmup=warmup_ms, metadata=meta, notes=notes)


# The reference's names for the device timing functions.
triton_do_bench_samples = device_event_samples
benchmark_triton_callable = benchmark_device_callable


def benchmark_callable(
    *,
    kernel: KernelMetadata,
    shape: BenchmarkShape,
    fn: Callable[[], Any],
    warmup: int = 5,
    iterations: int = 20,
    synchronize: Callable[[], Any] | None = None,
    metadata: dict[str, Any] | None = None,
    notes: str = "",
) -> BenchmarkRecord:
    """Wall-clock mean over ``iterations`` calls (benchmarking.py:189-234);
    pass ``synchronize`` for device work."""
    if warmup < 0:
        raise ValueError("warmup must be non-negative")
    if iterations <= 0:
        raise ValueError("iterations must be positive")
    for _ in range(warmup):
        fn()
    if synchronize is not None:
        synchronize()
    start = time.perf_counter()
    for _ in range(iterations):
        fn()
    if synchronize is not None:
        synchronize()
    runtime = (time.perf_counter() - start) * 1.0e3 / iterations
    return BenchmarkRecord(kernel_id=kernel.kernel_id, shape=shape, runtime_ms=runtime,
                           tops=tops_for_runtime(shape, runtime), iterations=iterations, warmup=warmup,
                           metadata=dict(metadata or {}), notes=notes)
