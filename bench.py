"""Benchmark of the gfx950 quantized GEMM path on one MI355X.

Headline metric: int4 x int4 per-channel GEMM TOPS at
M=N=K=8192 (config C2) through ``amd_strix_halo_kernels.mm``, as a fraction of
the gfx950 dense int8 MFMA peak.  Secondary lines in the same JSON object:
C3 (int4 subchannel-256 ReLU2, 4096x16384x4096), C4 (int8 fused SwiGLU,
4096 x 11008 x 4096, TOPS count up + gate), C5 (ragged MoE forward and
K-ragged backward, G=8, M=8192, K=2048, N=1408; also with scale groups
of 128 on the fp6 subchannel tile), the C2 persistent schedule,
the device quantize-and-pack of a C2-sized bf16 operand (GB/s against HBM),
and the decode-sized skinny GEMM (int4 per-channel and with scale groups of
128, M=16, N=K=8192; GB/s against HBM, weights streamed from HBM and
MALL-resident).

    python bench.py [--steps K] [--warmup W] [--no-secondary] [--no-cpu-baseline]
                    [--only c2|c3|c4|c5|c5_sc|c2p|quant|skinny|skinny_sc]

A step is one API call over operands already resident in HBM; the timed region
is exactly K steps bracketed by a device synchronisation on both sides.
Kernel durations come from HIP events recorded around every launch on the
stream the kernel runs on (torch's current stream).  C2 runs on the fp6 path
(two operand conversions, then the GEMM); the same three launches are also
made through the split C ABI with an event between each, which gives the GEMM
kernel's own duration for the roofline (fp6 MFMA peak) beside the whole
call's throughput (`value`, also reported against the int8 MFMA peak).  The
headline is the steady state (no cache flush between steps; C2's operands fit
the 256 MB MALL), after `preload_calls` untimed calls; beside it the line
carries the baseline's method (event median over K reps with the MALL
flushed before each: `flushed_event_median_ms`) and the wall time per call
right after an idle second (`idle_start_ms`).  The CPU baselines: C2 times
the repository's C oracle (unpack -> int32 matmul -> scale -> bf16) on a
bounded row slice; C3 and C4 time the torch reference path
(use_reference=True) on a row sample, C5 the grouped torch references of the
reference's tests on the whole call, all on the host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "strix-halo-int4-gemms_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "int4 GEMM TOPS @8192³ (% gfx950 int8 MFMA peak); fused SwiGLU TOPS"
INT8_MFMA_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, published
FP6_MFMA_PEAK_TFLOPS = 10100.0  # MI355X dense fp6/fp4 MFMA, published
HBM_PEAK_GBS = 8000.0
COPY_BYTES = 256 << 20
TRAFFIC_FILE = ROOT / "profiles" / "f6_gemm_c2_8192_traffic.txt"


def _measured_traffic():
    """HBM bytes per C2 launch from the committed FETCH_SIZE / WRITE_SIZE
    profile (scaled by the copy-kernel calibration), or None."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        return None
    return None


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _time_steps(torch, fn, steps: int, warmup: int):
    """Runs fn warmup + steps times; returns (wall ms/step, mean and median
    device ms per call) (see _time_steps_device)."""
    wall_ms, _, mean, median = _time_steps_device(torch, fn, steps, warmup)
    return wall_ms, mean, median


def _time_steps_device(torch, fn, steps: int, warmup: int):
    """Runs fn warmup + steps times; returns (wall ms/step, device ms/step,
    mean and median device ms per call).

    The timed loop issues the K calls back to back, as a caller's loop does,
    bracketed by synchronize: an event recorded between two calls adds a gap
    of ~11 us on the GPU (kernel trace of C2: 0 us from one call's last
    kernel to the next call's first without events, 11.5 us with a pair), so
    the device time per step comes from one event pair around the whole
    loop, and the per-call events run in a second pass of the same K calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    first, last = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    first.record()
    for _ in range(steps):
        fn()
    last.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    device_ms = first.elapsed_time(last) / steps
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    kern = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    kern.sort()
    return wall_ms, device_ms, sum(kern) / len(kern), kern[len(kern) // 2]


IDLE_WARMUP, IDLE_CALLS = 5, 20


def _idle_start_ms(torch, fn) -> float:
    """Wall ms per call of IDLE_CALLS calls after one second idle and
    IDLE_WARMUP warmup calls (what a caller sees at the start of a burst)."""
    torch.cuda.synchronize()
    time.sleep(1.0)
    for _ in range(IDLE_WARMUP):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(IDLE_CALLS):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / IDLE_CALLS


def _cold_ms(torch, fn, reps: int = 5) -> float:
    """Median of HIP-event pairs around single calls, each after a 1 GiB
    overwrite that evicts the 256 MB MALL (the measurement method of the
    baseline: event pairs, median, cache flushed between reps)."""
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    times = []
    for _ in range(reps):
        flush.fill_(1)
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    del flush
    times.sort()
    return times[len(times) // 2]


def _rand_int4_packed(torch, rows, cols, gen):
    """Uniform int4 codes in [-8, 7] packed two per byte along cols."""
    from amd_strix_halo_kernels import pack_int4_k_major

    q = torch.randint(-8, 8, (rows, cols), dtype=torch.int8, device="cuda", generator=gen)
    return pack_int4_k_major(q)


def _uniform_bf16(torch, shape, lo, hi, gen):
    return (torch.rand(shape, device="cuda", generator=gen) * (hi - lo) + lo).to(torch.bfloat16)


def _split_fp6_times(torch, shk, kernel, a, b, sa, sb, m, n, k, steps, warmup):
    """Per-kernel durations of a fp6 launch: the same three launches as
    ``mm`` (convert A, convert B, GEMM) made through the split C ABI with a HIP
    event between each, on torch's current stream.  Returns mean ms of
    (convert A, convert B, GEMM)."""
    from amd_strix_halo_kernels import native

    work = native.gemm_workspace(kernel, m, n, k, device=a.device)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=a.device)

    def run(ev=None):
        if ev is not None:
            ev[0].record()
        native.convert_operand(kernel, 0, a, m=m, n=n, k=k, workspace=work)
        if ev is not None:
            ev[1].record()
        native.convert_operand(kernel, 1, b, m=m, n=n, k=k, workspace=work)
        if ev is not None:
            ev[2].record()
        native.launch_converted(kernel, m=m, n=n, k=k, workspace=work, a_scale=sa, b_scale=sb, out=out)
        if ev is not None:
            ev[3].record()

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for ev in events:
        run(ev)
    torch.cuda.synchronize()
    sums = [0.0, 0.0, 0.0]
    for ev in events:
        for i in range(3):
            sums[i] += ev[i].elapsed_time(ev[i + 1])
    return tuple(x / steps for x in sums)


def bench_c2(torch, shk, steps, warmup):
    from amd_strix_halo_kernels import kernel_table as kt

    m = n = k = 8192
    gen = torch.Generator(device="cuda").manual_seed(2)
    a = _rand_int4_packed(torch, m, k, gen)                      # [M, K/2]
    b = _rand_int4_packed(torch, n, k, gen).t().contiguous()     # [K/2, N]
    sa = _uniform_bf16(torch, (m,), 0.005, 0.02, gen)
    sb = _uniform_bf16(torch, (n,), 0.005, 0.02, gen)
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL),
                                         epilogue=shk.Epilogue.NONE, m=m, n=n, k=k)

    def step():
        return shk.mm(a, b, a_scale=sa, b_scale=sb)

    # The auxiliary measurements run first.  The chip is power-limited, and
    # its controller overshoots after a load step: calls issued right after
    # an idle period run fast for ~2 ms, then ~20% slow for tens of ms, and
    # settle (0.33 ms/call for 20 calls after 5 warmup calls from idle,
    # 0.29 after 200 calls of continuous load).  The idle-start figure (one
    # second idle, 5 warmup calls, 20 timed) and the flushed event median
    # come first; the per-kernel split (>= 200 calls, an auxiliary figure)
    # comes right before the timed loop, which then sees the steady state a
    # serving loop runs in.  preload_calls counts every call before it.
    idle_ms = _idle_start_ms(torch, step)
    flushed = _cold_ms(torch, step, reps=max(steps, 5))
    preload = IDLE_WARMUP + IDLE_CALLS + max(steps, 5)
    fp6 = kt.TABLE[kernel.table_index].operand_format == kt.OPERANDS_FP6
    split = None
    if fp6:
        split_steps = max(steps, 200)
        split = _split_fp6_times(torch, shk, kernel, a, b, sa, sb, m, n, k, split_steps, warmup)
        preload += split_steps + warmup
    preload += warmup
    wall, kern_mean, kern_med = _time_steps(torch, step, steps, warmup)
    ops = 2 * m * n * k
    bytes_alg = m * k // 2 + k * n // 2 + 2 * m + 2 * n + 2 * m * n
    res = {
        "m": m, "n": n, "k": k, "kernel": kernel.kernel_id, "ops": ops, "bytes": bytes_alg,
        "wall_ms": wall, "kernel_ms": kern_mean, "kernel_ms_median": kern_med, "flushed_event_median_ms": flushed,
        "idle_start_ms": idle_ms, "preload_calls": preload, "host": (a, b, sa, sb), "fp6": fp6,
    }
    if fp6:
        res["convert_a_ms"], res["convert_b_ms"], res["gemm_ms"] = split
    return res


def bench_c3(torch, shk, steps, warmup):
    m, k, n, s = 4096, 4096, 16384, 256
    gen = torch.Generator(device="cuda").manual_seed(3)
    a = _rand_int4_packed(torch, m, k, gen)
    b = _rand_int4_packed(torch, n, k, gen).t().contiguous()
    sa = _uniform_bf16(torch, (m, k // s), 0.005, 0.02, gen)
    sb = _uniform_bf16(torch, (k // s, n), 0.005, 0.02, gen)
    spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, s)

    def step():
        return shk.mm(a, b, a_scale=sa, b_scale=sb, scale=spec, epilogue=shk.Epilogue.RELU2)

    wall, dev, kern, _ = _time_steps_device(torch, step, steps, warmup)
    ops = 2 * m * n * k

    def cpu():
        return _cpu_dense_torch(
            torch, shk, lambda a_, b_, sa_, sb_: shk.mm(a_, b_, a_scale=sa_, b_scale=sb_, scale=spec,
                                                        epilogue=shk.Epilogue.RELU2, use_reference=True),
            a, b, sa, sb, m=m, ops_per_row=2 * n * k, what="C3 int4 sc256 ReLU2")

    return {"tops": ops / (dev * 1e-3) / 1e12, "device_ms": dev, "wall_ms": wall, "event_ms_per_call": kern,
            "frac_int8_peak": ops / (dev * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS, "_cpu": cpu}


def bench_c4(torch, shk, steps, warmup):
    m, k, d = 4096, 4096, 11008
    gen = torch.Generator(device="cuda").manual_seed(4)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda", generator=gen)
    b = torch.randint(-127, 128, (k, 2 * d), dtype=torch.int8, device="cuda", generator=gen)
    sa = _uniform_bf16(torch, (m,), 1e-4, 1e-3, gen)
    sb = _uniform_bf16(torch, (2 * d,), 1e-4, 1e-3, gen)

    def step():
        return shk.fused_swiglu_up_gate(a, b, a_scale=sa, b_scale=sb, dtype=shk.OperandDType.INT8)

    wall, dev, kern, _ = _time_steps_device(torch, step, steps, warmup)
    ops = 2 * m * (2 * d) * k

    def cpu():
        return _cpu_dense_torch(
            torch, shk, lambda a_, b_, sa_, sb_: shk.fused_swiglu_up_gate(a_, b_, a_scale=sa_, b_scale=sb_,
                                                                          dtype=shk.OperandDType.INT8,
                                                                          use_reference=True),
            a, b, sa, sb, m=m, ops_per_row=2 * (2 * d) * k, what="C4 int8 fused SwiGLU")

    return {"tops": ops / (dev * 1e-3) / 1e12, "device_ms": dev, "wall_ms": wall, "event_ms_per_call": kern,
            "frac_int8_peak": ops / (dev * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS, "_cpu": cpu}


def bench_c2_persistent(torch, shk, steps, warmup):
    """C2 through mm(schedule=KernelSchedule.PERSISTENT): the same fp6 tile on
    one workgroup per CU, each taking every 256th tile (the whole call,
    conversions included, as `value`)."""
    m = n = k = 8192
    gen = torch.Generator(device="cuda").manual_seed(2)
    a = torch.randint(0, 256, (m, k // 2), dtype=torch.uint8, device="cuda", generator=gen)
    b = torch.randint(0, 256, (k // 2, n), dtype=torch.uint8, device="cuda", generator=gen)
    sa = _uniform_bf16(torch, (m,), 0.005, 0.02, gen)
    sb = _uniform_bf16(torch, (n,), 0.005, 0.02, gen)

    def step():
        return shk.mm(a, b, a_scale=sa, b_scale=sb, schedule=shk.KernelSchedule.PERSISTENT)

    wall, kern, _ = _time_steps(torch, step, steps, warmup)
    ops = 2 * m * n * k
    return {"tops": ops / (wall * 1e-3) / 1e12, "wall_ms": wall, "kernel_ms": kern,
            "frac_int8_peak": ops / (wall * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS}


def bench_quant(torch, shk, steps, warmup):
    """Device fake quantization + int4 packing of a C2-sized bf16 operand
    (8192 x 8192), along each axis, against the HBM roofline: algorithmic
    bytes = 2 per value read + 0.5 per value written.  The reference's torch
    formulas (fake_quant_int then pack_int4_k_major, several element-wise
    launches with int8/int16 intermediates) run on the same tensor beside it."""
    m = n = 8192
    gen = torch.Generator(device="cuda").manual_seed(11)
    x = (torch.randn((m, n), generator=gen, device="cuda") * 0.05).to(torch.bfloat16)
    nbytes = m * n * 2 + m * n // 2
    out = {}
    for axis in (-1, -2):
        _, kern, _ = _time_steps(torch, lambda: shk.quantize_pack_int4(x, scale=0.01, axis=axis), steps, warmup)
        gbs = nbytes / (kern * 1e-3) / 1e9
        out[f"axis{axis}"] = {"kernel_ms": kern, "gbs": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}

    def torch_formulas():
        q = torch.clamp(torch.round(x.float() / 0.01), -8, 7).to(torch.int8)
        return ((q[:, 1::2].to(torch.int16) & 0xF) << 4 | (q[:, 0::2].to(torch.int16) & 0xF)).to(torch.uint8)

    _, kern, _ = _time_steps(torch, torch_formulas, max(3, steps // 4), 2)
    out["torch_formulas_axis-1_ms"] = kern
    out["bytes"] = nbytes
    return out


SKINNY_COPIES = 16  # distinct 32 MiB weight matrices cycled by the HBM figure (512 MiB: beyond the MALL)
SKINNY_LAUNCHES = 64  # launches per captured graph


def bench_skinny(torch, shk, steps, warmup, subchannel=None):
    """Decode-sized int4 GEMM, M = 16, N = K = 8192, per-channel or with
    subchannel scale groups (GPTQ-style groups of 128), on the skinny tile
    (packed B streamed straight from HBM), against the HBM roofline.

    Device time per launch: HIP events around the replay of a HIP graph of
    SKINNY_LAUNCHES back-to-back C-ABI launches (no host work between them),
    median over replays.  hbm: the launches cycle SKINNY_COPIES distinct
    weight matrices and scales, 512 MiB of B (more than the 256 MB MALL), as
    a decode step streams one layer's weights after another; warm: the same B
    every launch (MALL-resident).  mm_wall_us is the public call's wall time
    per call (host-bound at this size)."""
    from amd_strix_halo_kernels import kernel_table as kt
    from amd_strix_halo_kernels import native

    m, n, k = 16, 8192, 8192
    s = subchannel or 0
    gen = torch.Generator(device="cuda").manual_seed(6)
    a = _rand_int4_packed(torch, m, k, gen)
    bs = [torch.randint(0, 256, (k // 2, n), dtype=torch.uint8, device="cuda", generator=gen)
          for _ in range(SKINNY_COPIES)]
    sa = _uniform_bf16(torch, (m, k // s) if s else (m,), 0.005, 0.02, gen)
    sbs = [_uniform_bf16(torch, (k // s, n) if s else (n,), 0.005, 0.02, gen) for _ in range(SKINNY_COPIES)]
    spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, s) if s else shk.ScaleSpec(shk.ScaleMode.PER_CHANNEL)
    kernel = shk.default_registry.select(dtype=shk.OperandDType.INT4, scale=spec, epilogue=shk.Epilogue.NONE,
                                         m=m, n=n, k=k)
    desc = kt.TABLE[kernel.table_index]
    lib = native.load_dispatch_library()
    ws = desc.workspace_bytes(m, n, k)
    work = torch.zeros(max(ws, 256), dtype=torch.uint8, device="cuda")  # split counters start at zero
    out = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    dev = torch.cuda.current_device()

    def launch(i, stream):
        rc = lib.amd_strix_halo_kernels_launch_gemm_ws(
            kernel.table_index, dev, stream, a.data_ptr(), bs[i].data_ptr(), sa.data_ptr(), sbs[i].data_ptr(),
            out.data_ptr(), m, n, k, s, kt.EPILOGUE_NONE, kt.OUT_BF16, work.data_ptr() if ws else None, ws)
        if rc:
            raise RuntimeError(lib.amd_strix_halo_kernels_last_error().decode())

    launch(0, torch.cuda.current_stream().cuda_stream)
    want = shk.mm(a, bs[0], a_scale=sa, b_scale=sbs[0], scale=spec)
    torch.cuda.synchronize()
    if not torch.equal(want, out):
        raise RuntimeError("skinny: the direct launch differs from mm()")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    nbytes = m * k // 2 + k * n // 2 + 2 * m * n + (2 * (m + n) * (k // s) if s else 2 * m + 2 * n)
    res = {"m": m, "n": n, "k": k, "subchannel": s or None, "kernel": kernel.kernel_id,
           "splits": kt.sk_split_count(desc, m, n, k),
           "bytes": nbytes, "launches_per_graph": SKINNY_LAUNCHES, "weight_copies": SKINNY_COPIES}
    for name, rotate in (("warm", False), ("hbm", True)):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for i in range(SKINNY_LAUNCHES):
                launch(i % SKINNY_COPIES if rotate else 0, side.cuda_stream)
        for _ in range(max(2, warmup // 2)):
            graph.replay()
        torch.cuda.synchronize()
        per = []
        for _ in range(max(5, steps // 4)):
            s_ev = torch.cuda.Event(enable_timing=True)
            e_ev = torch.cuda.Event(enable_timing=True)
            s_ev.record()
            graph.replay()
            e_ev.record()
            torch.cuda.synchronize()
            per.append(s_ev.elapsed_time(e_ev) / SKINNY_LAUNCHES)
        per.sort()
        us = per[len(per) // 2] * 1e3
        res[f"{name}_us"] = us
        res[f"{name}_gbs"] = nbytes / (us * 1e-6) / 1e9
        del graph
    # the last replay's last launch read weight copy (SKINNY_LAUNCHES - 1) % SKINNY_COPIES
    last = (SKINNY_LAUNCHES - 1) % SKINNY_COPIES
    if not torch.equal(shk.mm(a, bs[last], a_scale=sa, b_scale=sbs[last], scale=spec), out):
        raise RuntimeError("skinny: the graph replay's output differs from mm()")
    res["frac_hbm"] = res["hbm_gbs"] / HBM_PEAK_GBS
    res["warm_frac_hbm"] = res["warm_gbs"] / HBM_PEAK_GBS
    wall, _, _ = _time_steps(torch, lambda: shk.mm(a, bs[0], a_scale=sa, b_scale=sbs[0], scale=spec), steps, warmup)
    res["mm_wall_us"] = wall * 1e3
    return res


def _multinomial_sizes(torch, rows, groups, seed):
    g = torch.Generator().manual_seed(seed)
    # Dirichlet(1) = normalised exponentials; multinomial counts; then the
    # smallest group's rows move to the largest so one group is empty.
    e = -torch.log(torch.rand(groups, generator=g, dtype=torch.float64))
    probs = e / e.sum()
    idx = torch.multinomial(probs, rows, replacement=True, generator=g)
    sizes = torch.bincount(idx, minlength=groups).to(torch.int64)
    if not (sizes == 0).any():
        lo, hi = int(sizes.argmin()), int(sizes.argmax())
        sizes[hi] += sizes[lo]
        sizes[lo] = 0
    return sizes


def bench_c5(torch, shk, steps, warmup):
    groups, rows, k, n = 8, 8192, 2048, 1408
    gen = torch.Generator(device="cuda").manual_seed(5)
    sizes = _multinomial_sizes(torch, rows, groups, 5)
    lhs = _rand_int4_packed(torch, rows, k, gen)
    rhs = torch.stack([_rand_int4_packed(torch, n, k, gen).t().contiguous() for _ in range(groups)])
    sa = _uniform_bf16(torch, (rows,), 0.005, 0.02, gen)
    sb = _uniform_bf16(torch, (groups, n), 0.005, 0.02, gen)
    gs = sizes.to(device="cuda", dtype=torch.int32)

    from amd_strix_halo_kernels import kernel_table as kt
    from amd_strix_halo_kernels import native

    out_f = torch.empty((rows, n), device="cuda", dtype=torch.bfloat16)

    def fwd():
        # The device work of one ragged_dot_int4 call (task list + grouped
        # kernel); the API's host-side group-size validation is not timed.
        # (the fp6 entry, as ragged_dot_int4 picks for this shape: both
        # operand conversions are inside the timed call)
        return native.launch_ragged_fwd(lhs, rhs, gs, a_scale=sa, b_scale=sb, out=out_f,
                                        layout=shk.GemmLayout.NN, subchannel=None, block_m=kt.RAGGED_FP6_BLOCK_M,
                                        align_tile=kt.RAGGED_FP6_ALIGN, rows=rows, cols=n, k_packed=k // 2,
                                        out_mode=kt.OUT_BF16, fp6=True)

    ref_out = shk.ragged_dot_int4(lhs, rhs, gs, a_scale=sa, b_scale=sb)
    fwd()
    torch.cuda.synchronize()
    if not torch.equal(ref_out, out_f):
        raise RuntimeError("ragged forward: direct launch differs from the API call")

    wall_f, dev_f, kern_f, _ = _time_steps_device(torch, fwd, steps, warmup)
    ops = 2 * rows * n * k
    bytes_f = rows * k // 2 + groups * k * n // 2 + 2 * rows + 2 * groups * n + 2 * rows * n

    cap = int(sizes.max()) + int(sizes.max()) % 2
    x = _rand_int4_packed(torch, groups * 2048, cap, gen).view(groups, 2048, cap // 2)
    dy = torch.stack([_rand_int4_packed(torch, n, cap, gen).t().contiguous() for _ in range(groups)])
    sa_b = _uniform_bf16(torch, (groups, 2048), 0.005, 0.02, gen)
    sb_b = _uniform_bf16(torch, (groups, n), 0.005, 0.02, gen)
    out_b = torch.empty((groups, 2048, n), device="cuda", dtype=torch.float32)

    def bwd():
        return native.launch_ragged_bwd(x, dy, gs, a_scale=sa_b, b_scale=sb_b, out=out_b, layout=shk.GemmLayout.NN,
                                        subchannel=None, split_k=1, rows=2048, cols=n, k_packed=cap // 2, fp6=True)

    api_b = shk.ragged_dot_int4_bwd(x, dy, gs, a_scale=sa_b, b_scale=sb_b)
    bwd()
    torch.cuda.synchronize()
    if not torch.equal(api_b, out_b):
        raise RuntimeError("ragged backward: direct launch differs from the API call")

    wall_b, dev_b, kern_b, _ = _time_steps_device(torch, bwd, steps, warmup)

    # The public calls, as the reference's ragged benchmark times them
    # (autotune.py:746-777): host validation of group_sizes (one device-to-host
    # copy and sync per call) plus the same device work.
    def api_fwd():
        return shk.ragged_dot_int4(lhs, rhs, gs, a_scale=sa, b_scale=sb, out=out_f)

    def api_bwd():
        return shk.ragged_dot_int4_bwd(x, dy, gs, a_scale=sa_b, b_scale=sb_b, out=out_b)

    api_wall_f, api_kern_f, _ = _time_steps(torch, api_fwd, steps, warmup)
    api_wall_b, api_kern_b, _ = _time_steps(torch, api_bwd, steps, warmup)
    ops_b = 2 * 2048 * n * rows
    bytes_b = groups * 2048 * cap // 2 + groups * cap * n // 2 + 2 * groups * (2048 + n) + 4 * groups * 2048 * n

    def cpu():
        return _cpu_ragged_torch(torch, lhs, rhs, sizes, sa, sb, x, dy, sa_b, sb_b, n=n, k=k)

    return {
        "_cpu": cpu,
        "group_sizes": sizes.tolist(),
        "fwd": {"device_ms": dev_f, "wall_ms": wall_f, "event_ms_per_call": kern_f,
                "tops": ops / (dev_f * 1e-3) / 1e12,
                "api_wall_ms": api_wall_f, "api_event_ms": api_kern_f,
                "gbs": bytes_f / (dev_f * 1e-3) / 1e9,
                "frac_hbm": bytes_f / (dev_f * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "frac_int8_peak": ops / (dev_f * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS},
        "bwd": {"device_ms": dev_b, "wall_ms": wall_b, "event_ms_per_call": kern_b,
                "tops": ops_b / (dev_b * 1e-3) / 1e12,
                "api_wall_ms": api_wall_b, "api_event_ms": api_kern_b,
                "gbs": bytes_b / (dev_b * 1e-3) / 1e9,
                "frac_hbm": bytes_b / (dev_b * 1e-3) / 1e9 / HBM_PEAK_GBS},
    }


def bench_c5_subchannel(torch, shk, steps, warmup, subchannel=128):
    """C5's shape with scale groups of `subchannel`: the device work of the
    forward and backward calls on their fp6 subchannel entries (as the API
    picks them; the backward's K capacity is rounded up to 64, which keeps
    ceil(K/32) even, so that every group size qualifies), each checked
    against the API call first."""
    groups, rows, k, n = 8, 8192, 2048, 1408
    gen = torch.Generator(device="cuda").manual_seed(5)
    sizes = _multinomial_sizes(torch, rows, groups, 5)
    cols = k // subchannel
    lhs = _rand_int4_packed(torch, rows, k, gen)
    rhs = torch.stack([_rand_int4_packed(torch, n, k, gen).t().contiguous() for _ in range(groups)])
    sa = _uniform_bf16(torch, (rows, cols), 0.005, 0.02, gen)
    sb = _uniform_bf16(torch, (groups, cols, n), 0.005, 0.02, gen)
    gs = sizes.to(device="cuda", dtype=torch.int32)
    spec = shk.ScaleSpec(shk.ScaleMode.SUBCHANNEL, subchannel)

    from amd_strix_halo_kernels import kernel_table as kt
    from amd_strix_halo_kernels import native

    if not kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_FWD, subchannel=subchannel, m=rows, n=n, k_packed=k // 2):
        raise RuntimeError("C5 subchannel forward: the fp6 entry does not take this shape")
    out_f = torch.empty((rows, n), device="cuda", dtype=torch.bfloat16)

    def fwd():
        return native.launch_ragged_fwd(lhs, rhs, gs, a_scale=sa, b_scale=sb, out=out_f, layout=shk.GemmLayout.NN,
                                        subchannel=subchannel, block_m=kt.RAGGED_FP6_BLOCK_M,
                                        align_tile=kt.RAGGED_FP6_ALIGN, rows=rows, cols=n, k_packed=k // 2,
                                        out_mode=kt.OUT_BF16, fp6=True)

    ref_out = shk.ragged_dot_int4(lhs, rhs, gs, a_scale=sa, b_scale=sb, scale=spec)
    fwd()
    torch.cuda.synchronize()
    if not torch.equal(ref_out, out_f):
        raise RuntimeError("subchannel ragged forward: direct launch differs from the API call")
    wall_f, dev_f, kern_f, _ = _time_steps_device(torch, fwd, steps, warmup)
    ops = 2 * rows * n * k

    cap = -(-int(sizes.max()) // 64) * 64
    bcols = -(-cap // subchannel)
    x = _rand_int4_packed(torch, groups * 2048, cap, gen).view(groups, 2048, cap // 2)
    dy = torch.stack([_rand_int4_packed(torch, n, cap, gen).t().contiguous() for _ in range(groups)])
    sa_b = _uniform_bf16(torch, (groups, 2048, bcols), 0.005, 0.02, gen)
    sb_b = _uniform_bf16(torch, (groups, bcols, n), 0.005, 0.02, gen)
    if not kt.ragged_fp6_eligible(kt.FAMILY_RAGGED_BWD, subchannel=subchannel, m=2048, n=n, k_packed=cap // 2):
        raise RuntimeError("C5 subchannel backward: the fp6 entry does not take this shape")
    out_b = torch.empty((groups, 2048, n), device="cuda", dtype=torch.float32)

    def bwd():
        return native.launch_ragged_bwd(x, dy, gs, a_scale=sa_b, b_scale=sb_b, out=out_b, layout=shk.GemmLayout.NN,
                                        subchannel=subchannel, split_k=1, rows=2048, cols=n, k_packed=cap // 2,
                                        fp6=True)

    api_b = shk.ragged_dot_int4_bwd(x, dy, gs, a_scale=sa_b, b_scale=sb_b, scale=spec)
    bwd()
    torch.cuda.synchronize()
    if not torch.equal(api_b, out_b):
        raise RuntimeError("subchannel ragged backward: direct launch differs from the API call")
    wall_b, dev_b, kern_b, _ = _time_steps_device(torch, bwd, steps, warmup)
    ops_b = 2 * 2048 * n * rows
    return {
        "subchannel": subchannel, "group_sizes": sizes.tolist(), "bwd_k_capacity": cap,
        "fwd": {"device_ms": dev_f, "wall_ms": wall_f, "event_ms_per_call": kern_f,
                "tops": ops / (dev_f * 1e-3) / 1e12,
                "frac_int8_peak": ops / (dev_f * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS},
        "bwd": {"device_ms": dev_b, "wall_ms": wall_b, "event_ms_per_call": kern_b,
                "tops": ops_b / (dev_b * 1e-3) / 1e12,
                "frac_int8_peak": ops_b / (dev_b * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS},
    }


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


CPU_TARGET_S = 6.0  # seconds of CPU work per torch-path baseline sample


def _cpu_info(torch) -> dict:
    return {"cores": torch.get_num_threads(), "cpu_model": _cpu_model(), "torch": torch.__version__}


def _cpu_rows_sample(torch, run, m: int, ops_per_row: int, target_s: float):
    """Grows a row sample (multiples of 16) of run(rows) until one timed call
    lasts target_s or covers all m rows; returns (rows, seconds)."""
    rows = 16
    while True:
        t0 = time.perf_counter()
        run(rows)
        secs = time.perf_counter() - t0
        if secs >= target_s or rows >= m:
            return rows, secs
        grow = int(rows * target_s / max(secs, 1e-3) * 1.1)
        rows = min(m, max(rows * 2, (grow + 15) // 16 * 16))


def _cpu_dense_torch(torch, shk, call, a, b, sa, sb, *, m: int, ops_per_row: int, what: str):
    """The torch reference path (use_reference=True: unpack, int32 matmul,
    fp32 scaling in the kernel's order, epilogue, bf16; api.py:257-325 of the
    reference) on the host, over a row sample of the same operands."""
    b_c, sb_c = b.cpu(), sb.cpu()
    a_c, sa_c = a.cpu(), sa.cpu()

    def run(rows):
        call(a_c[:rows], b_c, sa_c[:rows], sb_c)

    rows, secs = _cpu_rows_sample(torch, run, m, ops_per_row, CPU_TARGET_S)
    return {"value": rows * ops_per_row / secs / 1e12, "unit": "TOPS", "kind": "port", **_cpu_info(torch),
            "path": "torch reference path (use_reference=True) on CPU tensors", "reps": 1,
            "sample": f"{what}: rows 0..{rows - 1} of {m}, one timed call of {secs:.1f} s (unpack of B included)"}


def _cpu_ragged_torch(torch, lhs, rhs, sizes, sa, sb, x, dy, sa_b, sb_b, *, n: int, k: int, reps: int = 3):
    """C5 on the host: the grouped references of the reference's tests
    (tests/test_ragged_dot.py:19-32 forward, :82-96 backward; fp32 matmul of
    the unpacked int4 values, exact at these K), 1 untimed warmup and `reps`
    timed calls each, median; unpack included."""
    from amd_strix_halo_kernels.quant import unpack_int4_k_major

    lhs_c, rhs_c, sa_c, sb_c = lhs.cpu(), rhs.cpu(), sa.cpu(), sb.cpu()
    x_c, dy_c, sa_bc, sb_bc = x.cpu(), dy.cpu(), sa_b.cpu(), sb_b.cpu()
    group_sizes = [int(g) for g in sizes.tolist()]

    def fwd():
        a_q = unpack_int4_k_major(lhs_c)
        b_q = unpack_int4_k_major(rhs_c.transpose(-2, -1)).transpose(-2, -1)
        out = torch.empty((a_q.shape[0], b_q.shape[2]), dtype=torch.float32)
        row = 0
        for g, size in enumerate(group_sizes):
            part = torch.matmul(a_q[row:row + size].to(torch.float32), b_q[g].to(torch.float32))
            part *= sa_c[row:row + size, None].to(torch.float32)
            part *= sb_c[g, None, :].to(torch.float32)
            out[row:row + size] = part
            row += size
        return out.to(torch.bfloat16)

    def bwd():
        a_q = unpack_int4_k_major(x_c)
        b_q = unpack_int4_k_major(dy_c.transpose(-2, -1)).transpose(-2, -1)
        out = torch.empty((a_q.shape[0], a_q.shape[1], b_q.shape[2]), dtype=torch.float32)
        for g, size in enumerate(group_sizes):
            part = torch.matmul(a_q[g, :, :size].to(torch.float32), b_q[g, :size, :].to(torch.float32))
            part *= sa_bc[g, :, None].to(torch.float32)
            part *= sb_bc[g, None, :].to(torch.float32)
            out[g] = part
        return out

    res = {}
    rows = sum(group_sizes)
    for name, fn, ops in (("fwd", fwd, 2 * rows * n * k), ("bwd", bwd, 2 * x.shape[1] * n * rows)):
        fn()
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        times.sort()
        med = times[len(times) // 2]
        res[name] = {"value": ops / med / 1e12, "unit": "TOPS", "ms": med * 1e3, "kind": "port", **_cpu_info(torch),
                     "path": "grouped torch references of the reference's tests, on CPU tensors", "reps": reps,
                     "sample": "the whole C5 call (all groups), median of the timed reps after one warmup"}
    return res


def cpu_baseline(torch, host, target_s: float = 12.0):
    """Times the C oracle's whole dense path on a row slice of the C2 operands."""
    import numpy as np

    from oracle import native as oracle_native

    if not oracle_native.available():
        from oracle import build as obuild

        obuild.build(verbose=False)
    a, b, sa, sb = host
    a_np = a.cpu().numpy()
    b_np = b.cpu().numpy()
    sa_np = sa.view(torch.int16).cpu().numpy().view(np.uint16)
    sb_np = sb.view(torch.int16).cpu().numpy().view(np.uint16)
    m, n, k = a_np.shape[0], b_np.shape[1], 2 * a_np.shape[1]
    threads = oracle_native.default_threads()
    # Grow the row sample until the timed call lasts at least target_s (or
    # covers every row); each call includes its own unpack of B.
    rows = 256
    while True:
        t0 = time.perf_counter()
        oracle_native.dense_int4_nn(a_np, b_np, sa_np, sb_np, m=m, n=n, k=k, row0=0, rows=rows, threads=threads)
        secs = time.perf_counter() - t0
        if secs >= target_s or rows >= m:
            break
        rows = min(m, max(rows * 2, int(rows * target_s / max(secs, 1e-3) * 1.1)))
    ops = 2 * rows * n * k
    return {"value": ops / secs / 1e12, "unit": "TOPS", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(), "torch": torch.__version__,
            "sample": f"C2 rows 0..{rows - 1} of 8192 (N=K=8192, full unpack->int32 matmul->scale->bf16), "
                      f"{secs:.1f} s"}


# single configurations of --only: (name, runner)
_ONLY = {
    "c3": ("c3_int4_sc256_relu2_4096x16384x4096", bench_c3),
    "c4": ("c4_int8_swiglu_4096x11008x4096", bench_c4),
    "c5": ("c5_ragged_g8_m8192_k2048_n1408", bench_c5),
    "c5_sc": ("c5_ragged_sc128_g8_m8192_k2048_n1408", bench_c5_subchannel),
    "c2p": ("c2_persistent_schedule_8192_cubed", bench_c2_persistent),
    "quant": ("quantize_pack_int4_8192x8192_bf16", bench_quant),
    "skinny": ("skinny_int4_pc_16x8192x8192", bench_skinny),
    "skinny_sc": ("skinny_int4_sc128_16x8192x8192", lambda torch, shk, steps, warmup: bench_skinny(
        torch, shk, steps, warmup, subchannel=128)),
}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=sorted(_ONLY) + ["c2"],
                   help="run one configuration and print its figures (for profiler runs)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a 256 MiB device-to-device copy 5 times (HBM counter calibration)")
    args = p.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build runs the hot path on a single MI355X "
              "(multi-GPU sharding is a design note, not built); use --gpus 1", file=sys.stderr)
        return 2

    import torch

    import amd_strix_halo_kernels as shk

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": COPY_BYTES, "launches": 5}), flush=True)
        return 0
    if args.only and args.only != "c2":
        name, fn = _ONLY[args.only]
        _log(f"bench: {name} only")
        res = fn(torch, shk, args.steps, args.warmup)
        res.pop("_cpu", None)
        print(json.dumps({"only": name, "steps": args.steps, "warmup": args.warmup, "result": res}), flush=True)
        return 0
    if args.only == "c2":
        args.no_secondary = args.no_cpu_baseline = True
    _log("bench: C2 int4 per-channel 8192^3")
    c2 = bench_c2(torch, shk, args.steps, args.warmup)
    tops_kernel = c2["ops"] / (c2["kernel_ms"] * 1e-3) / 1e12
    tops_wall = c2["ops"] / (c2["wall_ms"] * 1e-3) / 1e12
    secondary = {}
    if not args.no_secondary:
        _log("bench: C3 int4 sc256 relu2")
        secondary["c3_int4_sc256_relu2_4096x16384x4096"] = bench_c3(torch, shk, max(10, args.steps // 2),
                                                                    args.warmup)
        _log("bench: C4 int8 swiglu")
        secondary["c4_int8_swiglu_4096x11008x4096"] = bench_c4(torch, shk, max(10, args.steps // 2), args.warmup)
        _log("bench: C5 ragged fwd/bwd")
        secondary["c5_ragged_g8_m8192_k2048_n1408"] = bench_c5(torch, shk, max(10, args.steps // 2), args.warmup)
        _log("bench: C5 ragged fwd/bwd, scale groups of 128")
        secondary["c5_ragged_sc128_g8_m8192_k2048_n1408"] = bench_c5_subchannel(torch, shk, max(10, args.steps // 2),
                                                                               args.warmup)
        _log("bench: C2 on the persistent schedule")
        secondary["c2_persistent_schedule_8192_cubed"] = bench_c2_persistent(torch, shk, max(10, args.steps // 2),
                                                                            args.warmup)
        _log("bench: device quantize + int4 pack, 8192x8192 bf16")
        secondary["quantize_pack_int4_8192x8192_bf16"] = bench_quant(torch, shk, max(10, args.steps // 2),
                                                                     args.warmup)
        _log("bench: skinny int4 per-channel 16x8192x8192")
        secondary["skinny_int4_pc_16x8192x8192"] = bench_skinny(torch, shk, max(10, args.steps // 2), args.warmup)
        _log("bench: skinny int4 subchannel-128 16x8192x8192")
        secondary["skinny_int4_sc128_16x8192x8192"] = bench_skinny(torch, shk, max(10, args.steps // 2),
                                                                   args.warmup, subchannel=128)
    for key, res in secondary.items():
        cpu_fn = res.pop("_cpu", None)
        if cpu_fn is not None and not args.no_cpu_baseline:
            _log(f"bench: CPU baseline of {key} (torch path)")
            res["cpu_baseline"] = cpu_fn()
    cpu = None
    if not args.no_cpu_baseline:
        _log("bench: CPU baseline (C oracle)")
        cpu = cpu_baseline(torch, c2["host"])
    if c2["fp6"]:
        # the dominant kernel is the fp6 GEMM (f6_gemm_kernel); the two
        # operand conversions are reported beside it
        achieved = c2["ops"] / (c2["gemm_ms"] * 1e-3) / 1e12
        peak = FP6_MFMA_PEAK_TFLOPS
        dtype = "fp6"
        operands = ("packed int4 converted to fp6 blocks in a workspace (e2m3 holding v/8, exact for -8..7), "
                    "fp6 MFMA (v_mfma_f32_32x32x64_f8f6f4), fp32 accumulation exact for K <= 262144")
        note = ("fp6 MFMA tera-ops/s of the GEMM kernel: algorithmic 2*M*N*K over its HIP-event launch duration; "
                "value (the headline) counts the whole mm() call including both operand conversions, as the wall "
                "time of K back-to-back calls in the steady state a serving loop runs in, after preload_calls "
                "untimed calls; flushed_event_median_ms is the baseline's method (event median over K reps with "
                "the MALL flushed before each) and idle_start_ms the wall time per call right after an idle "
                "second")
    else:
        achieved = tops_kernel
        peak = INT8_MFMA_PEAK_TOPS
        dtype = "int8"
        operands = "packed int4 (two nibbles per byte along K), int8 MFMA, int32 accumulation"
        note = ("int8 MFMA tera-ops/s; algorithmic 2*M*N*K per launch over the HIP-event launch duration; value "
                "(the headline) is the steady-state wall time of K back-to-back calls after preload_calls untimed "
                "calls; flushed_event_median_ms is the baseline's method")
    line = {
        "metric": METRIC,
        "value": tops_wall,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c2["wall_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": {
            "workload": "C2: int4 x int4 per-channel GEMM, epilogue none, M=N=K=8192, bf16 out",
            "operands": operands,
            "kernel": c2["kernel"],
            "parallelism": "single GPU",
        },
        "frac_int8_mfma_peak": tops_wall / INT8_MFMA_PEAK_TOPS,
        "kernel_ms": c2["kernel_ms"],
        "kernel_ms_median": c2["kernel_ms_median"],
        # the baseline's method (event pairs, median over K reps, MALL flushed
        # before each) beside the steady-state headline
        "flushed_event_median_ms": c2["flushed_event_median_ms"],
        "flushed_tops": c2["ops"] / (c2["flushed_event_median_ms"] * 1e-3) / 1e12,
        "idle_start_ms": c2["idle_start_ms"],
        "idle_start_tops": c2["ops"] / (c2["idle_start_ms"] * 1e-3) / 1e12,
        "preload_calls": c2["preload_calls"],
        "roofline": {
            "bound": "mfma",
            "achieved": achieved,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": achieved / peak,
            "traffic": _measured_traffic() if c2["fp6"] else None,
            "note": note,
        },
        "fp6_launch_ms": ({"convert_a": c2["convert_a_ms"], "convert_b": c2["convert_b_ms"], "gemm": c2["gemm_ms"]}
                          if c2["fp6"] else None),
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
