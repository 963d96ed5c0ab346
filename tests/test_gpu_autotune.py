"""Autotuning on the GPU: every candidate kernel runs, validates against the
package's reference math (``explicit_mm(use_reference=True)``) and gets a
HIP-event timed record; the ragged autotuner times every default config."""

from __future__ import annotations

import pytest

import amd_strix_halo_kernels as shk
from amd_strix_halo_kernels.metadata import Epilogue, GemmLayout, OperandDType, ScaleMode, ScaleSpec

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _print_case(*parts) -> None:
    print("case:", *parts, flush=True)


def test_device_event_samples_time_a_known_copy():
    x = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    samples = shk.device_event_samples(lambda: y.copy_(x), warmup_ms=2, rep_ms=10)
    assert samples and all(s > 0 for s in samples)
    # 128 MiB of traffic cannot beat 8 TB/s
    assert min(samples) > (128 << 20) / 8.0e12 * 1.0e3


@pytest.mark.parametrize("dtype,scale,epilogue,layout", [
    (OperandDType.INT4, ScaleSpec(ScaleMode.PER_CHANNEL), Epilogue.NONE, GemmLayout.NN),
    (OperandDType.INT4, ScaleSpec(ScaleMode.PER_CHANNEL), Epilogue.SWIGLU, GemmLayout.NT),
    (OperandDType.INT4, ScaleSpec(ScaleMode.SUBCHANNEL, 128), Epilogue.NONE, GemmLayout.TN),
    (OperandDType.INT8, ScaleSpec(ScaleMode.PER_CHANNEL), Epilogue.RELU2, GemmLayout.NN),
])
def test_autotune_validates_and_times_every_candidate(tmp_path, dtype, scale, epilogue, layout):
    m, n, k = 512, 512, 1024
    _print_case("autotune", dtype.value, scale.label, epilogue.value, layout.value, (m, n, k))
    path = tmp_path / "db.json"
    res = shk.autotune(m=m, n=n, k=k, dtype=dtype, layout=layout, scale=scale, epilogue=epilogue,
                       warmup_ms=2, rep_ms=5, validate=True, benchmark_db_path=path)
    assert len(res.records) == len(res.candidates) >= 1
    for rec in res.records:
        assert rec.success and rec.runtime_ms > 0 and rec.tops > 0
        assert rec.metadata["validated"] and rec.metadata["timing_backend"] == "hip_events"
        assert rec.max_abs_diff is not None
    assert res.best_record.tops == max(r.tops for r in res.records)
    loaded = shk.BenchmarkDatabase.load(path)
    assert loaded.best_record(res.best_kernel, res.shape) == res.best_record
    assert shk.choose_kernel(m=m, n=n, k=k, dtype=dtype, layout=layout, scale=scale, epilogue=epilogue,
                             benchmark_db=loaded) == res.best_kernel


@pytest.mark.parametrize("mode,scale", [
    (shk.RaggedDotMode.FWD, ScaleSpec(ScaleMode.PER_CHANNEL)),
    (shk.RaggedDotMode.FWD, ScaleSpec(ScaleMode.SUBCHANNEL, 128)),
    (shk.RaggedDotMode.BWD, ScaleSpec(ScaleMode.PER_CHANNEL)),
])
def test_ragged_autotune_times_every_default_config(mode, scale):
    m, n, k = 1024, 512, 1024
    _print_case("ragged autotune", mode.value, scale.label, (m, n, k))
    res = shk.autotune_ragged_dot(mode=mode, m=m, n=n, k=k, groups=4, scale=scale, warmup_ms=2, rep_ms=5,
                                  continue_on_error=False)
    assert len(res.records) == len(res.candidates) >= 2
    assert all(r.success and r.tops > 0 for r in res.records)
    assert res.best_record.tops == max(r.tops for r in res.records)
    assert sum(res.group_sizes) == (m if mode is shk.RaggedDotMode.FWD else k)
