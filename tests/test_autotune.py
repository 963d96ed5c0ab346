"""Benchmark database, heuristics and autotune host logic (no GPU).

Cases follow the reference's tests/test_benchmarking.py:50-127 and
tests/test_autotune.py:151-380: the database JSON round trip drops failed
records from lookups, an exact-shape record outranks the static score, the
autotuner keeps the best record and feeds it back to the heuristic, and the
ragged autotuner checks group sizes / candidate modes and keeps failed
candidates.  Timing runs through injected runners, so nothing here touches a
GPU.
"""

from __future__ import annotations

import json

import pytest

import amd_strix_halo_kernels as shk
from amd_strix_halo_kernels.metadata import (
    Epilogue,
    GemmLayout,
    KernelMetadata,
    OperandDType,
    ScaleMode,
    ScaleSpec,
    TileConfig,
)
from amd_strix_halo_kernels.ragged import RaggedBwdDotConfig, RaggedDotConfig
from amd_strix_halo_kernels.registry import KernelRegistry

PC = ScaleSpec(ScaleMode.PER_CHANNEL)


def _kernel(kid: str, tile: TileConfig, *, epilogue: Epilogue = Epilogue.NONE, tops: float | None = None):
    return KernelMetadata(kernel_id=kid, arch="gfx950", a_dtype=OperandDType.INT4, b_dtype=OperandDType.INT4,
                          acc_dtype="int32", output_dtype="bfloat16", scale_dtype="bfloat16", scale=PC,
                          epilogue=epilogue, tile=tile, triton_kernel_name=kid, measured_tops=tops)


def _tile(bm=64, bn=256, bk=64, even_k=True, split_k=1):
    return TileConfig(bm, bn, bk, 8, 8, 3, 0, even_k, split_k)


def _rec(kid, shape, tops, success=True):
    return shk.BenchmarkRecord(kid, shape, runtime_ms=1.0, tops=tops, iterations=4, warmup=1, success=success)


def test_tops_for_runtime_counts_two_ops_per_mac():
    assert shk.gemm_ops(shk.BenchmarkShape(2, 3, 5)) == 60
    # 2 * 1024**3 ops in 1 ms
    assert shk.tops_for_runtime(shk.BenchmarkShape(1024, 1024, 1024), 1.0) == pytest.approx(2.147483648)
    with pytest.raises(ValueError):
        shk.tops_for_runtime(shk.BenchmarkShape(1, 1, 1), 0.0)


def test_summary_quantiles_interpolate_between_ranks():
    s = shk.summarize_runtime_samples([4.0, 1.0, 2.0, 8.0, -1.0, 0.0])
    assert s["raw_sample_count"] == 6 and s["sample_count"] == 4
    assert s["dropped_nonpositive_sample_count"] == 2
    assert (s["runtime_ms_min"], s["runtime_ms_max"]) == (1.0, 8.0)
    assert s["runtime_ms_median"] == 3.0 and s["runtime_ms_mean"] == 3.75
    # sorted [1, 2, 4, 8]: p20 at rank 0.6 -> 1.6, p80 at rank 2.4 -> 5.6
    assert s["runtime_ms_p20"] == pytest.approx(1.6)
    assert s["runtime_ms_p80"] == pytest.approx(5.6)
    with pytest.raises(ValueError):
        shk.summarize_runtime_samples([])
    with pytest.raises(ValueError):
        shk.summarize_runtime_samples([0.0, -2.0])


def test_database_round_trip_keeps_reference_schema(tmp_path):
    shape = shk.BenchmarkShape(64, 512, 64)
    good = _rec("k", shape, 17.0)
    failed = _rec("k", shape, 99.0, success=False)
    other_shape = _rec("k", shk.BenchmarkShape(64, 512, 128), 50.0)
    db = shk.BenchmarkDatabase([good, failed, other_shape])
    path = tmp_path / "sub" / "bench.json"
    db.save(path)
    raw = json.loads(path.read_text())
    assert sorted(raw["records"][0]) == sorted([
        "kernel_id", "shape", "runtime_ms", "tops", "iterations", "warmup", "success", "max_abs_diff",
        "max_rel_diff", "notes", "metadata"])
    assert raw["records"][0]["shape"] == {"m": 64, "n": 512, "k": 64}
    loaded = shk.BenchmarkDatabase.load(path)
    assert loaded.records() == db.records()
    kern = _kernel("k", _tile())
    assert loaded.matching_records(kern, shape) == (good,)
    assert loaded.best_record(kern, shape) == good
    assert loaded.best_record(_kernel("absent", _tile()), shape) is None


def test_heuristic_prefers_exact_shape_record_and_rejects_unsupported_shapes():
    fast = _kernel("fast", _tile(bn=512), tops=100.0)
    slow = _kernel("slow", _tile(bn=256), tops=50.0)
    registry = KernelRegistry([fast, slow])
    shape = shk.BenchmarkShape(64, 512, 64)
    req = dict(m=64, n=512, k=64, dtype=OperandDType.INT4, scale=PC, epilogue=Epilogue.NONE, registry=registry)
    assert shk.choose_kernel(**req) == fast
    db = shk.BenchmarkDatabase([_rec("fast", shape, 4.0), _rec("slow", shape, 8.0)])
    assert shk.choose_kernel(**req, benchmark_db=db) == slow
    masked = _kernel("masked", _tile(even_k=False))
    assert not shk.kernel_supports_shape(masked, m=64, n=512, k=128)
    assert shk.estimate_kernel_score(masked, m=64, n=512, k=128) == float("-inf")
    assert not shk.kernel_supports_shape(fast, m=65, n=512, k=64)
    assert not shk.kernel_supports_shape(fast, m=64, n=513, k=64)
    split = _kernel("split", _tile(split_k=2), epilogue=Epilogue.SWIGLU)
    assert not shk.kernel_supports_shape(split, m=64, n=256, k=256)
    with pytest.raises(LookupError):
        shk.choose_kernel(m=65, n=512, k=64, dtype=OperandDType.INT4, scale=PC, epilogue=Epilogue.NONE,
                          registry=registry)


def test_autotune_keeps_best_and_feeds_the_heuristic(tmp_path):
    shape = shk.BenchmarkShape(4096, 4096, 4096)
    a = _kernel("a", _tile(bn=512), tops=500.0)
    b = _kernel("b", _tile(bn=256), tops=10.0)
    registry = KernelRegistry([a, b])
    path = tmp_path / "db.json"
    shk.BenchmarkDatabase([_rec("older", shape, 1.0)]).save(path)
    seen = []

    def runner(kern, tuned):
        seen.append((kern.kernel_id, tuned))
        return _rec(kern.kernel_id, tuned, 60.0 if kern.kernel_id == "a" else 65.0)

    result = shk.autotune(m=4096, n=4096, k=4096, dtype=OperandDType.INT4, scale=PC, epilogue=Epilogue.NONE,
                          registry=registry, benchmark_db_path=path, benchmark_runner=runner)
    assert seen == [("a", shape), ("b", shape)]
    assert result.best_kernel == b and result.best_record.tops == 65.0
    assert result.candidates == (a, b)
    # earlier records are kept and the new ones appended
    assert [r.kernel_id for r in shk.BenchmarkDatabase.load(path).records()] == ["older", "a", "b"]
    assert shk.choose_kernel(m=4096, n=4096, k=4096, dtype=OperandDType.INT4, scale=PC, epilogue=Epilogue.NONE,
                             registry=registry, benchmark_db=result.benchmark_db) == b
    assert shk.generated_shape_for_kernel(a) is None
    with pytest.raises(LookupError):
        shk.autotune(m=100, n=4096, k=4096, dtype=OperandDType.INT4, scale=PC, epilogue=Epilogue.NONE,
                     registry=registry, benchmark_runner=runner)
    with pytest.raises(RuntimeError):
        shk.autotune(m=4096, n=4096, k=4096, dtype=OperandDType.INT4, scale=PC, epilogue=Epilogue.NONE,
                     registry=registry, benchmark_runner=lambda k, s: _rec(k.kernel_id, s, 1.0, success=False))


def test_default_registry_candidates_cover_the_table():
    cands = shk.find_autotune_candidates(m=8192, n=8192, k=8192, dtype=OperandDType.INT4, scale=PC,
                                         epilogue=Epilogue.NONE)
    assert len(cands) >= 2
    assert all(shk.kernel_supports_shape(c, m=8192, n=8192, k=8192) for c in cands)
    assert len({c.kernel_id for c in cands}) == len(cands)


def test_ragged_candidates_and_labels():
    fwd = shk.default_ragged_dot_candidates(shk.RaggedDotMode.FWD)
    assert fwd and all(isinstance(c.config, RaggedDotConfig) for c in fwd)
    assert len({c.kernel_id for c in fwd}) == len(fwd)
    bwd = shk.default_ragged_dot_candidates(shk.RaggedDotMode.BWD, layout=GemmLayout.TN, split_ks=(1, 2, 4))
    assert [c.config.split_k for c in bwd] == [1, 2, 4]
    assert all(c.layout is GemmLayout.TN for c in bwd)
    cfg = RaggedDotConfig(block_m=32, block_n=128, block_k=64, group_size_tasks=2, num_warps=4, num_stages=3)
    assert shk.ragged_config_label(cfg) == "BM32_BN128_BK64_GST2_W4_S3"
    bcfg = RaggedBwdDotConfig(block_m=16, block_n=64, block_k=32, split_k=2, num_warps=4, num_stages=2)
    assert shk.ragged_config_label(bcfg) == "BM16_BN64_BK32_W4_S2_SK2"
    cand = shk.RaggedAutotuneCandidate(shk.RaggedDotMode.BWD, GemmLayout.NN, ScaleSpec(ScaleMode.SUBCHANNEL, 32),
                                       bcfg)
    assert cand.kernel_id == "ragged_dot_int4_bwd_nn_sc32_bm16_bn64_bk32_w4_s2_sk2"
    with pytest.raises(TypeError):
        shk.default_ragged_dot_candidates("fwd")


def test_ragged_autotune_shapes_group_sizes_and_failures(tmp_path):
    cfg = RaggedBwdDotConfig(split_k=2)

    def runner(cand, tuned):
        assert cand.mode is shk.RaggedDotMode.BWD and tuned == shk.BenchmarkShape(32, 96, 39)
        return _rec(cand.kernel_id, tuned, 9.0)

    res = shk.autotune_ragged_dot(mode=shk.RaggedDotMode.BWD, m=32, n=96, k=39, group_sizes=(7, 0, 32),
                                  layout=GemmLayout.TN, candidates=(cfg,), benchmark_runner=runner)
    assert res.group_sizes == (7, 0, 32) and res.best_candidate.config == cfg

    # balanced default partition of M over the groups
    got = {}

    def fwd_runner(cand, tuned):
        got["n"] = got.get("n", 0) + 1
        if cand.config.block_m == 16:
            raise RuntimeError("no such launch")
        return _rec(cand.kernel_id, tuned, float(cand.config.block_m))

    path = tmp_path / "ragged.json"
    res = shk.autotune_ragged_dot(mode=shk.RaggedDotMode.FWD, m=10, n=64, k=64, groups=3,
                                  benchmark_runner=fwd_runner, benchmark_db_path=path)
    assert res.group_sizes == (4, 3, 3)
    assert got["n"] == len(res.candidates)
    failed = [r for r in res.records if not r.success]
    assert len(failed) == 1 and "no such launch" in failed[0].metadata["error"]
    assert res.best_record.tops == max(float(c.config.block_m) for c in res.candidates)
    assert len(shk.BenchmarkDatabase.load(path).records()) == len(res.candidates)
    with pytest.raises(RuntimeError, match="no such launch"):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.FWD, m=10, n=64, k=64, groups=3,
                                benchmark_runner=fwd_runner, continue_on_error=False)

    base = dict(n=64, k=64, benchmark_runner=runner)
    with pytest.raises(ValueError, match="sum to M"):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.FWD, m=10, group_sizes=(4, 4), **base)
    with pytest.raises(ValueError, match="sum to K"):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.BWD, m=10, group_sizes=(4, 4), **base)
    with pytest.raises(ValueError, match="non-negative"):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.FWD, m=10, group_sizes=(12, -2), **base)
    with pytest.raises(ValueError, match="k_capacity"):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.BWD, m=10, group_sizes=(40, 24), k_capacity=32, **base)
    with pytest.raises(ValueError, match="only configurable"):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.FWD, m=10, k_capacity=128, **base)
    with pytest.raises(TypeError):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.FWD, m=10, candidates=(cfg,), **base)
    wrong_layout = shk.RaggedAutotuneCandidate(shk.RaggedDotMode.FWD, GemmLayout.NT, PC, RaggedDotConfig())
    with pytest.raises(ValueError, match="layout"):
        shk.autotune_ragged_dot(mode=shk.RaggedDotMode.FWD, m=10, candidates=(wrong_layout,), **base)
