"""Autotuning over the gfx950 kernel table and the ragged-dot launch configs.

Same entry points, arguments, results and database records as the
reference's autotune.py:
  * ``autotune`` (autotune.py:144-220) times every registry kernel that
    matches the request and supports the shape, keeps the best by TOPS and
    appends the records to a ``BenchmarkDatabase`` (saved when a path is
    given);
  * ``autotune_ragged_dot`` (autotune.py:251-381) does the same for
    ``ragged_dot_int4`` / ``ragged_dot_int4_bwd`` launch configs, recording a
    failed candidate as an unsuccessful record when ``continue_on_error``.

Differences that follow from the MI355X build:
  * every table kernel takes its shape at run time, so there is no per-shape
    artifact: ``generated_shape_for_kernel`` returns None and
    ``require_exact_generated_shape`` reduces to ``kernel_supports_shape``;
  * timing uses HIP events (``benchmarking.device_event_samples``) in place
    of triton's do_bench; the records say so in ``timing_backend``;
  * the default ragged candidates are the configs that select distinct
    gfx950 kernels: one forward config per compiled row-tile height of the
    packed kernels, plus block_m 256, which asks for the fp6 kernel (block_m
    64, the default config, also takes the fp6 kernel where that kernel
    applies), and one backward config per split-K factor.
    Configs that differ only in fields the gfx950 launch ignores (block_n,
    block_k, warps, stages) would time the same kernel twice.
Operands are synthetic, seeded from the kernel id and shape: uniform int4
(or int8) codes and the reference's linspace bf16 scales
(autotune.py:551-594, 818-829).  Packing happens before timing.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from enum import Enum
from pathlib import Path
from typing import Any, Callable, Iterable, Sequence

from . import kernel_table as kt
from .benchmarking import (
    TIMING_BACKEND,
    BenchmarkDatabase,
    BenchmarkRecord,
    BenchmarkShape,
    benchmark_device_callable,
    device_event_samples,
    summarize_runtime_samples,
    tops_for_runtime,
)
from .heuristics import kernel_supports_shape
from .metadata import Epilogue, GemmLayout, KernelMetadata, KernelSchedule, OperandDType, ScaleMode, ScaleSpec
from .ragged import RaggedBwdDotConfig, RaggedDotConfig, ragged_dot_int4, ragged_dot_int4_bwd
from .registry import KernelRegistry, default_registry

BenchmarkRunner = Callable[[KernelMetadata, BenchmarkShape], BenchmarkRecord]
RaggedBenchmarkRunner = Callable[["RaggedAutotuneCandidate", BenchmarkShape], BenchmarkRecord]


class RaggedDotMode(str, Enum):
    """Ragged int4 dot family to autotune."""

    FWD = "fwd"
    BWD = "bwd"


def ragged_config_label(config: RaggedDotConfig | RaggedBwdDotConfig) -> str:
    """The config part of a ragged record's kernel id (ragged_artifacts.py:18-22 format)."""
    head = f"BM{config.block_m}_BN{config.block_n}_BK{config.block_k}"
    if isinstance(config, RaggedDotConfig):
        return f"{head}_GST{config.group_size_tasks}_W{config.num_warps}_S{config.num_stages}"
    return f"{head}_W{config.num_warps}_S{config.num_stages}_SK{config.split_k}"


@dataclass(frozen=True, slots=True)
class AutotuneResult:
    shape: BenchmarkShape
    candidates: tuple[KernelMetadata, ...]
    records: tuple[BenchmarkRecord, ...]
    best_kernel: KernelMetadata
    best_record: BenchmarkRecord
    benchmark_db: BenchmarkDatabase


@dataclass(frozen=True, slots=True)
class RaggedAutotuneCandidate:
    """One ragged-dot launch config."""

    mode: RaggedDotMode
    layout: GemmLayout
    scale: ScaleSpec
    config: RaggedDotConfig | RaggedBwdDotConfig

    @property
    def config_label(self) -> str:
        return ragged_config_label(self.config)

    @property
    def kernel_id(self) -> str:
        return (f"ragged_dot_int4_{self.mode.value}_{self.layout.value}_"
                f"{self.scale.label.lower()}_{self.config_label.lower()}")


@dataclass(frozen=True, slots=True)
class RaggedAutotuneResult:
    shape: BenchmarkShape
    mode: RaggedDotMode
    layout: GemmLayout
    scale: ScaleSpec
    group_sizes: tuple[int, ...]
    candidates: tuple[RaggedAutotuneCandidate, ...]
    records: tuple[BenchmarkRecord, ...]
    best_candidate: RaggedAutotuneCandidate
    best_record: BenchmarkRecord
    benchmark_db: BenchmarkDatabase


def generated_shape_for_kernel(kernel: KernelMetadata, *, root: str | Path | None = None) -> BenchmarkShape | None:
    """None: gfx950 table kernels are not specialised to a generation shape."""
    del kernel, root
    return None


def artifact_supports_shape(kernel: KernelMetadata, shape: BenchmarkShape, *, root: str | Path | None = None) -> bool:
    del root
    return kernel_supports_shape(kernel, m=shape.m, n=shape.n, k=shape.k)


def find_autotune_candidates(
    *,
    m: int,
    n: int,
    k: int,
    dtype: OperandDType,
    layout: GemmLayout = GemmLayout.NN,
    scale: ScaleSpec,
    epilogue: Epilogue,
    schedule: KernelSchedule = KernelSchedule.STANDARD,
    registry: KernelRegistry = default_registry,
    root: str | Path | None = None,
    require_exact_generated_shape: bool = True,
) -> tuple[KernelMetadata, ...]:
    """Registry kernels of the request that support (m, n, k) (autotune.py:115-141)."""
    del root, require_exact_generated_shape
    return tuple(
        kern for kern in registry.all()
        if kern.a_dtype is dtype and kern.b_dtype is dtype and kern.layout is layout and kern.scale == scale
        and kern.epilogue is epilogue and kern.schedule is schedule
        and kernel_supports_shape(kern, m=m, n=n, k=k)
    )


def _load_db(benchmark_db: BenchmarkDatabase | None, path: str | Path | None) -> BenchmarkDatabase | None:
    if benchmark_db is None and path is not None and Path(path).exists():
        return BenchmarkDatabase.load(Path(path))
    return benchmark_db


def _finish(existing: BenchmarkDatabase | None, records: Sequence[BenchmarkRecord],
            path: str | Path | None, what: str) -> tuple[BenchmarkRecord, BenchmarkDatabase]:
    good = [r for r in records if r.success]
    if not good:
        raise RuntimeError(f"{what} produced no successful benchmark records")
    best = max(good, key=lambda r: r.tops)
    db = BenchmarkDatabase((*(existing.records() if existing is not None else ()), *records))
    if path is not None:
        db.save(Path(path))
    return best, db


def autotune(
    *,
    m: int,
    n: int,
    k: int,
    dtype: OperandDType,
    layout: GemmLayout = GemmLayout.NN,
    scale: ScaleSpec,
    epilogue: Epilogue,
    schedule: KernelSchedule = KernelSchedule.STANDARD,
    registry: KernelRegistry = default_registry,
    benchmark_db: BenchmarkDatabase | None = None,
    benchmark_db_path: str | Path | None = None,
    root: str | Path | None = None,
    library_path: str | Path | None = None,
    warmup_ms: int = 25,
    rep_ms: int = 100,
    validate: bool = False,
    benchmark_runner: BenchmarkRunner | None = None,
) -> AutotuneResult:
    shape = BenchmarkShape(m, n, k)
    candidates = find_autotune_candidates(m=m, n=n, k=k, dtype=dtype, layout=layout, scale=scale,
                                          epilogue=epilogue, schedule=schedule, registry=registry, root=root)
    if not candidates:
        raise LookupError(
            f"no pregenerated kernels match dtype={dtype.value}, layout={layout.value}, scale={scale.label}, "
            f"epilogue={epilogue.value}, schedule={schedule.value}, shape=({m}, {n}, {k})")
    existing = _load_db(benchmark_db, benchmark_db_path)
    runner = benchmark_runner or (lambda kern, s: _benchmark_native_kernel(
        kern, s, root=root, library_path=library_path, warmup_ms=warmup_ms, rep_ms=rep_ms, validate=validate))
    records = tuple(runner(kern, shape) for kern in candidates)
    if not records:
        raise RuntimeError("autotune produced no benchmark records")
    best, db = _finish(existing, records, benchmark_db_path, "autotune")
    best_kernel = next(kern for kern in candidates if kern.kernel_id == best.kernel_id)
    return AutotuneResult(shape=shape, candidates=candidates, records=records, best_kernel=best_kernel,
                          best_record=best, benchmark_db=db)


def default_ragged_dot_candidates(
    mode: RaggedDotMode,
    *,
    layout: GemmLayout = GemmLayout.NN,
    scale: ScaleSpec = ScaleSpec(ScaleMode.PER_CHANNEL),
    split_ks: Iterable[int] = (1, 2),
) -> tuple[RaggedAutotuneCandidate, ...]:
    """One config per distinct gfx950 ragged kernel (see the module docstring)."""
    mode = _check_ragged_mode(mode)
    layout = _check_layout(layout)
    split_ks = tuple(split_ks)
    if mode is RaggedDotMode.FWD:
        heights = sorted(set(kt.RAGGED_FWD_BLOCK_M) | {kt.RAGGED_FP6_CONFIG_BLOCK_M})
        configs = [RaggedDotConfig(block_m=bm, align_tile=min(8, bm)) for bm in heights]
    else:
        configs = [RaggedBwdDotConfig(split_k=int(sk)) for sk in split_ks]
    return tuple(RaggedAutotuneCandidate(mode=mode, layout=layout, scale=scale, config=c) for c in configs)


def autotune_ragged_dot(
    *,
    mode: RaggedDotMode,
    m: int,
    n: int,
    k: int,
    k_capacity: int | None = None,
    group_sizes: Sequence[int] | Any | None = None,
    groups: int = 8,
    layout: GemmLayout = GemmLayout.NN,
    scale: ScaleSpec = ScaleSpec(ScaleMode.PER_CHANNEL),
    candidates: Iterable[RaggedAutotuneCandidate | RaggedDotConfig | RaggedBwdDotConfig] | None = None,
    split_ks: Iterable[int] = (1, 2),
    benchmark_db: BenchmarkDatabase | None = None,
    benchmark_db_path: str | Path | None = None,
    warmup_ms: int = 25,
    rep_ms: int = 100,
    continue_on_error: bool = True,
    benchmark_runner: RaggedBenchmarkRunner | None = None,
) -> RaggedAutotuneResult:
    """Times ragged-dot configs at one shape.

    FWD: ``group_sizes`` partitions the M rows.  BWD: ``group_sizes``
    partitions the logical K; every group's operands are padded to
    ``k_capacity`` (default max(group_sizes)).  Without ``group_sizes`` the
    total is split over ``groups`` as evenly as possible.
    """
    if m <= 0 or n <= 0 or k <= 0:
        raise ValueError("m, n, and k must be positive")
    if warmup_ms < 0:
        raise ValueError("warmup_ms must be non-negative")
    if rep_ms <= 0:
        raise ValueError("rep_ms must be positive")
    mode = _check_ragged_mode(mode)
    layout = _check_layout(layout)
    sizes = _normalize_ragged_group_sizes(mode=mode, group_sizes=group_sizes, groups=groups, m=m, k=k)
    capacity = _normalize_ragged_k_capacity(mode=mode, k=k, k_capacity=k_capacity, group_sizes=sizes)
    shape = BenchmarkShape(m=m, n=n, k=k)
    cands = _normalize_ragged_candidates(mode=mode, layout=layout, scale=scale, candidates=candidates,
                                         split_ks=split_ks)
    if not cands:
        raise LookupError(f"no ragged-dot autotune candidates for mode={mode.value}, layout={layout.value}")
    existing = _load_db(benchmark_db, benchmark_db_path)
    runner = benchmark_runner or (lambda cand, s: _benchmark_ragged_candidate(
        cand, s, m=m, n=n, k_capacity=capacity, group_sizes=sizes, warmup_ms=warmup_ms, rep_ms=rep_ms))
    records: list[BenchmarkRecord] = []
    for cand in cands:
        try:
            record = runner(cand, shape)
        except Exception as exc:  # noqa: BLE001 - recorded as a failed candidate
            if not continue_on_error:
                raise
            record = BenchmarkRecord(
                kernel_id=cand.kernel_id, shape=shape, runtime_ms=float("inf"), tops=0.0, iterations=0,
                warmup=warmup_ms, success=False, notes="ragged-dot autotune candidate failed",
                metadata={"error": repr(exc), **_ragged_record_metadata(
                    cand, group_sizes=sizes, k_capacity=capacity, warmup_ms=warmup_ms, rep_ms=rep_ms)})
        records.append(record)
    best, db = _finish(existing, records, benchmark_db_path, "ragged-dot autotune")
    best_cand = next(c for c in cands if c.kernel_id == best.kernel_id)
    return RaggedAutotuneResult(shape=shape, mode=mode, layout=layout, scale=scale, group_sizes=sizes,
                                candidates=cands, records=tuple(records), best_candidate=best_cand,
                                best_record=best, benchmark_db=db)


# --------------------------------------------------------------------------
# argument checks


def _stable_seed(value: str) -> int:
    return int.from_bytes(hashlib.sha256(value.encode()).digest()[:4], "little")


def _check_layout(layout: GemmLayout) -> GemmLayout:
    if type(layout) is not GemmLayout:
        raise TypeError(f"layout must be a GemmLayout, got {type(layout).__name__}")
    return layout


def _check_ragged_mode(mode: RaggedDotMode) -> RaggedDotMode:
    if type(mode) is not RaggedDotMode:
        raise TypeError(f"mode must be a RaggedDotMode, got {type(mode).__name__}")
    return mode


def _balanced_sizes(total: int, groups: int) -> tuple[int, ...]:
    if groups <= 0:
        raise ValueError("groups must be positive")
    q, r = divmod(total, groups)
    return tuple(q + (g < r) for g in range(groups))


def _normalize_ragged_group_sizes(*, mode: RaggedDotMode, group_sizes: Any, groups: int, m: int,
                                  k: int) -> tuple[int, ...]:
    if group_sizes is None:
        sizes = _balanced_sizes(m if mode is RaggedDotMode.FWD else k, groups)
    else:
        host = group_sizes
        for step in ("detach", "cpu", "tolist"):
            if hasattr(host, step):
                host = getattr(host, step)()
        sizes = tuple(int(v) for v in host)
    if not sizes:
        raise ValueError("group_sizes must contain at least one group")
    if any(v < 0 for v in sizes):
        raise ValueError("group_sizes must be non-negative")
    if mode is RaggedDotMode.FWD and sum(sizes) != m:
        raise ValueError(f"forward group_sizes must sum to M={m}; got {sum(sizes)}")
    if mode is RaggedDotMode.BWD and sum(sizes) != k:
        raise ValueError(f"backward group_sizes must sum to K={k}; got {sum(sizes)}")
    return sizes


def _normalize_ragged_k_capacity(*, mode: RaggedDotMode, k: int, k_capacity: int | None,
                                 group_sizes: tuple[int, ...]) -> int:
    if mode is RaggedDotMode.FWD:
        if k_capacity is not None and k_capacity != k:
            raise ValueError("k_capacity is only configurable for backward ragged dot")
        return k
    largest = max(group_sizes)
    capacity = largest if k_capacity is None else int(k_capacity)
    if capacity <= 0:
        raise ValueError("k_capacity must be positive")
    if capacity < largest:
        raise ValueError(f"backward k_capacity must be >= max(group_sizes)={largest}; got {capacity}")
    return capacity


def _normalize_ragged_candidates(*, mode: RaggedDotMode, layout: GemmLayout, scale: ScaleSpec,
                                 candidates: Any, split_ks: Iterable[int]) -> tuple[RaggedAutotuneCandidate, ...]:
    if candidates is None:
        return default_ragged_dot_candidates(mode, layout=layout, scale=scale, split_ks=split_ks)
    want = RaggedDotConfig if mode is RaggedDotMode.FWD else RaggedBwdDotConfig
    out = []
    for cand in candidates:
        if isinstance(cand, RaggedAutotuneCandidate):
            if cand.mode is not mode:
                raise ValueError(f"candidate mode {cand.mode.value} does not match requested {mode.value}")
            if cand.layout is not layout:
                raise ValueError(f"candidate layout {cand.layout.value} does not match requested {layout.value}")
            if cand.scale != scale:
                raise ValueError(f"candidate scale {cand.scale.label} does not match requested {scale.label}")
            if not isinstance(cand.config, want):
                raise TypeError(f"{mode.value} ragged-dot candidates must use {want.__name__}")
            out.append(cand)
        elif isinstance(cand, want):
            out.append(RaggedAutotuneCandidate(mode=mode, layout=layout, scale=scale, config=cand))
        else:
            raise TypeError(f"unsupported ragged autotune candidate {cand!r}")
    return tuple(out)


# --------------------------------------------------------------------------
# synthetic operands and timing


def _torch_gpu() -> Any:
    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("torch is required for autotuning") from exc
    if not torch.cuda.is_available() or torch.version.hip is None:
        raise RuntimeError("autotuning requires a ROCm torch GPU device")
    return torch


def _pack_rows(torch: Any, codes: Any) -> Any:
    from .quant import pack_int4_k_major

    return pack_int4_k_major(codes.contiguous())


def _rhs_operand(torch: Any, b_q: Any, *, int4: bool, b_trans: bool) -> Any:
    """B codes [.., K, N] in the layout's storage: K-major packed [.., N, K/2]
    for NT, [.., K/2, N] for NN (int8 codes: the same without packing)."""
    kn = b_q.transpose(-1, -2).contiguous()
    stored = _pack_rows(torch, kn) if int4 else kn
    return stored if b_trans else stored.transpose(-1, -2).contiguous()


def _lhs_operand(torch: Any, a_q: Any, *, int4: bool, a_trans: bool) -> Any:
    stored = _pack_rows(torch, a_q) if int4 else a_q.contiguous()
    return stored.transpose(-1, -2).contiguous() if a_trans else stored


def _linspace_scales(torch: Any, *, rows: int, cols: int, k: int, scale: ScaleSpec, groups: int | None,
                     ragged_fwd: bool = False) -> tuple[Any, Any]:
    """The reference's synthetic bf16 scales (autotune.py:551-594, 818-829)."""
    lead = () if groups is None else (groups,)
    a_lead = () if ragged_fwd else lead
    bf16 = dict(device="cuda", dtype=torch.bfloat16)
    if scale.mode is ScaleMode.PER_CHANNEL:
        a_n = rows * (1 if not a_lead else groups)
        a = torch.linspace(0.75, 1.25, a_n, **bf16).reshape(*a_lead, rows)
        b = torch.linspace(1.10, 0.90, cols * (groups or 1), **bf16).reshape(*lead, cols)
        return a, b
    sc = -(-k // (scale.subchannel_size or 1))
    a = torch.linspace(0.80, 1.20, rows * sc * (1 if not a_lead else groups), **bf16).reshape(*a_lead, rows, sc)
    b = torch.linspace(1.15, 0.85, sc * cols * (groups or 1), **bf16).reshape(*lead, sc, cols)
    return a, b


def _validation_tolerances(kernel: KernelMetadata) -> tuple[float, float]:
    """(rtol, atol) of autotune.py:829-834."""
    if kernel.output_dtype == "bfloat16":
        return 8.0e-3, 1.0e-2
    return 1.0e-4, (1.0e-2 if kernel.epilogue in {Epilogue.RELU2, Epilogue.SWIGLU} else 1.0e-3)


def _benchmark_native_kernel(kernel: KernelMetadata, shape: BenchmarkShape, *, root: str | Path | None,
                             library_path: str | Path | None, warmup_ms: int, rep_ms: int,
                             validate: bool) -> BenchmarkRecord:
    """Times one table kernel on synthetic operands (autotune.py:837-924)."""
    torch = _torch_gpu()
    from .api import explicit_mm
    from .native import _output_torch_dtype, launch_generated_kernel

    gen = torch.Generator(device="cuda")
    gen.manual_seed(_stable_seed(f"{kernel.kernel_id}-{shape.m},{shape.n},{shape.k}"))
    int4 = kernel.a_dtype is OperandDType.INT4
    lim = 8 if int4 else 128
    b_cols = 2 * shape.n if kernel.epilogue is Epilogue.SWIGLU else shape.n
    a_q = torch.randint(-lim, lim, (shape.m, shape.k), device="cuda", dtype=torch.int8, generator=gen)
    b_q = torch.randint(-lim, lim, (shape.k, b_cols), device="cuda", dtype=torch.int8, generator=gen)
    a = _lhs_operand(torch, a_q, int4=int4, a_trans=kernel.layout in {GemmLayout.TN, GemmLayout.TT})
    b = _rhs_operand(torch, b_q, int4=int4, b_trans=kernel.layout in {GemmLayout.NT, GemmLayout.TT})
    del a_q, b_q
    a_scale, b_scale = _linspace_scales(torch, rows=shape.m, cols=b_cols, k=shape.k, scale=kernel.scale, groups=None)
    c = torch.empty((shape.m, shape.n), device="cuda", dtype=_output_torch_dtype(torch, kernel))

    def run() -> Any:
        return launch_generated_kernel(a, b, kernel=kernel, a_scale=a_scale, b_scale=b_scale, c=c,
                                       root=root, library_path=library_path)

    max_abs = max_rel = None
    if validate:
        # the reference math multiplies int32 matrices, which torch runs on the CPU only
        expected = explicit_mm(a.cpu(), b.cpu(), kernel=kernel, a_scale=a_scale.cpu(), b_scale=b_scale.cpu(),
                               use_reference=True).float()
        actual = run().float().cpu()
        rtol, atol = _validation_tolerances(kernel)
        torch.testing.assert_close(actual, expected, rtol=rtol, atol=atol)
        diff = (actual - expected).abs()
        max_abs = float(diff.max())
        max_rel = float((diff / expected.abs().clamp(min=1.0e-3)).max())
    record = benchmark_device_callable(
        kernel=kernel, shape=shape, fn=run, warmup_ms=warmup_ms, rep_ms=rep_ms,
        notes="autotuned gfx950 table kernel; HIP-event device timing; packing excluded",
        metadata={"arch": kernel.arch, "dtype": kernel.a_dtype.value, "layout": kernel.layout.value,
                  "scale": kernel.scale.label, "epilogue": kernel.epilogue.value,
                  "output_dtype": kernel.output_dtype, "tile": kernel.tile.label, "even_k": kernel.tile.even_k,
                  "split_k": kernel.tile.split_k, "schedule": kernel.schedule.value, "validated": validate,
                  "torch_version": str(torch.__version__), "torch_hip": str(torch.version.hip),
                  "device": torch.cuda.get_device_name()})
    # a SwiGLU call computes two GEMMs of N columns each (autotune.py:971-976)
    factor = 2.0 if kernel.epilogue is Epilogue.SWIGLU else 1.0
    return BenchmarkRecord(kernel_id=record.kernel_id, shape=record.shape, runtime_ms=record.runtime_ms,
                           tops=record.tops * factor, iterations=record.iterations, warmup=record.warmup,
                           success=record.success, max_abs_diff=max_abs, max_rel_diff=max_rel,
                           notes=record.notes, metadata=record.metadata)


def _ragged_config_dict(config: RaggedDotConfig | RaggedBwdDotConfig) -> dict[str, Any]:
    fields = ("block_m", "block_n", "block_k", "align_tile", "group_size_tasks", "split_k",
              "enable_even_k_fast_path", "num_warps", "num_stages")
    return {f: getattr(config, f) for f in fields if hasattr(config, f)}


def _ragged_record_metadata(cand: RaggedAutotuneCandidate, *, group_sizes: tuple[int, ...], k_capacity: int,
                            warmup_ms: int, rep_ms: int) -> dict[str, Any]:
    return {"mode": cand.mode.value, "layout": cand.layout.value, "scale": cand.scale.label,
            "groups": len(group_sizes), "group_sizes": list(group_sizes), "logical_k_capacity": k_capacity,
            "config": _ragged_config_dict(cand.config), "config_label": cand.config_label, "dtype": "int4",
            "path": f"gfx950_ragged_dot_{cand.mode.value}", "timing_backend": TIMING_BACKEND,
            "warmup_ms": warmup_ms, "rep_ms": rep_ms}


def _benchmark_ragged_candidate(cand: RaggedAutotuneCandidate, shape: BenchmarkShape, *, m: int, n: int,
                                k_capacity: int, group_sizes: tuple[int, ...], warmup_ms: int,
                                rep_ms: int) -> BenchmarkRecord:
    """Times one ragged config on synthetic operands (autotune.py:704-800)."""
    torch = _torch_gpu()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(_stable_seed(f"{cand.kernel_id}-{m},{n},{k_capacity}-{group_sizes}"))
    groups = len(group_sizes)
    fwd = cand.mode is RaggedDotMode.FWD
    a_trans = cand.layout in {GemmLayout.TN, GemmLayout.TT}
    b_trans = cand.layout in {GemmLayout.NT, GemmLayout.TT}
    a_shape = (m, k_capacity) if fwd else (groups, m, k_capacity)
    a_q = torch.randint(-8, 8, a_shape, device="cuda", dtype=torch.int8, generator=gen)
    b_q = torch.randint(-8, 8, (groups, k_capacity, n), device="cuda", dtype=torch.int8, generator=gen)
    lhs = _lhs_operand(torch, a_q, int4=True, a_trans=a_trans)
    rhs = _rhs_operand(torch, b_q, int4=True, b_trans=b_trans)
    del a_q, b_q
    a_scale, b_scale = _linspace_scales(torch, rows=m, cols=n, k=k_capacity, scale=cand.scale, groups=groups,
                                        ragged_fwd=fwd)
    gs = torch.tensor(group_sizes, device="cuda", dtype=torch.int32)
    out = torch.empty((m, n) if fwd else (groups, m, n), device="cuda",
                      dtype=torch.bfloat16 if fwd else torch.float32)
    fn = ragged_dot_int4 if fwd else ragged_dot_int4_bwd

    def run() -> Any:
        return fn(lhs, rhs, gs, a_scale=a_scale, b_scale=b_scale, scale=cand.scale, config=cand.config,
                  layout=cand.layout, out=out)

    run()
    torch.cuda.synchronize()
    summary = summarize_runtime_samples(device_event_samples(run, warmup_ms=warmup_ms, rep_ms=rep_ms))
    runtime = float(summary["runtime_ms_median"])
    meta = {**_ragged_record_metadata(cand, group_sizes=group_sizes, k_capacity=k_capacity, warmup_ms=warmup_ms,
                                      rep_ms=rep_ms),
            "output_dtype": "bfloat16" if fwd else "float32", "input_distribution": "random_int4_uniform",
            "torch_version": str(torch.__version__), "torch_hip": str(torch.version.hip),
            "device": torch.cuda.get_device_name(), **summary}
    return BenchmarkRecord(kernel_id=cand.kernel_id, shape=shape, runtime_ms=runtime,
                           tops=tops_for_runtime(shape, runtime), iterations=int(summary["sample_count"]),
                           warmup=warmup_ms, metadata=meta,
                           notes="prepacked operands; BF16 scales; quantization/packing excluded from timing")
