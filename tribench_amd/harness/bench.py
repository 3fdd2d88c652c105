"""Timing harness (counterpart of tribench/bench.py) with HIP timers.

run_benchmark() keeps the reference's two-stage flow (bench.py:108-210):
first call (build/launch cost, excluded), correctness gate, timed loop, then
percentiles and derived metrics.  Timers:

  hip_event  HIP events recorded on torch's current stream around each call,
             with a synchronize per call (the reference's cuda_event timer,
             bench.py:69-94) — the default
  hip_graph  the call captured once into a HIP graph and replayed; each
             sample is one replay (launch overhead removed)
  cpu_wall   time.perf_counter around each call (for CPU devices)

On top of the reference's fields, a result carries the effective TOPS, the
roofline fraction against the MI355X peak of the path's bounding unit, and,
when the pack declares a ``prepass`` stage, that stage's own p50 and its HBM
rate against 8 TB/s.
"""
from __future__ import annotations

import os
import time
from typing import Callable

import torch

from . import stats
from .cases import Case, seeded_inputs
from .correctness import check_correctness
from .metrics import PEAKS_MI355X, compute_gbps, compute_tflops, get_estimate_dict
from .types import BenchResult, CorrectnessResult, KernelMeta


def _sync(device: str) -> None:
    if device.startswith("cuda") and torch.cuda.is_available():
        torch.cuda.synchronize()


def _bench_hip_event(fn: Callable, warmup_ms: float, rep_ms: float) -> list[float]:
    """Per-call HIP event pairs on the current stream."""
    fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    fn()
    e.record()
    torch.cuda.synchronize()
    est = max(s.elapsed_time(e), 1e-3)
    for _ in range(max(1, int(warmup_ms / est))):
        fn()
    torch.cuda.synchronize()
    times: list[float] = []
    for _ in range(max(3, int(rep_ms / est))):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    return times


def _bench_hip_graph(fn: Callable, warmup_ms: float, rep_ms: float) -> list[float]:
    """Capture fn into one HIP graph (on a side stream) and time replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return _bench_hip_event(graph.replay, warmup_ms, rep_ms)


def _bench_cpu_wall(fn: Callable, warmup_ms: float, rep_ms: float) -> list[float]:
    t0 = time.perf_counter()
    fn()
    est = max((time.perf_counter() - t0) * 1e3, 1e-3)
    for _ in range(int(warmup_ms / est)):
        fn()
    times = []
    for _ in range(max(1, int(rep_ms / est))):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return times


TIMER_BACKENDS: dict[str, Callable] = {
    "hip_event": _bench_hip_event,
    "hip_graph": _bench_hip_graph,
    "cpu_wall": _bench_cpu_wall,
}


def cpu_info() -> tuple[int, str]:
    """(threads available to this process, CPU model name)."""
    try:
        threads = len(os.sched_getaffinity(0))
    except AttributeError:
        threads = os.cpu_count() or 1
    from .env import cpu_model

    return threads, cpu_model()


def run_benchmark(
    *,
    kernel_name: str,
    meta: KernelMeta,
    make_inputs_fn: Callable,
    reference_fn: Callable,
    triton_fn: Callable,
    estimate_fn: Callable | None,
    case: Case,
    device: str,
    seed: int,
    warmup_ms: float = 200.0,
    rep_ms: float = 2000.0,
    quantiles: list[float] | None = None,
    timer_backend: str = "hip_event",
    run_correctness: bool = True,
    pass_type: str = "forward",
    stage_fns: dict[str, Callable] | None = None,
    roofline_unit: str = "int8",
) -> BenchResult:
    """Build/warm up, check, then time ``triton_fn(**inputs)`` for one case.

    ``triton_fn`` keeps the reference's parameter name; it is whichever
    implementation is being measured.  ``stage_fns`` maps a stage name to a
    callable with the same inputs; the ``prepass`` stage is timed on its own.
    """
    if timer_backend not in TIMER_BACKENDS:
        raise ValueError(f"Unknown timer backend '{timer_backend}'. Available: {list(TIMER_BACKENDS)}")
    if timer_backend != "cpu_wall" and not device.startswith("cuda"):
        timer_backend = "cpu_wall"
    timer = TIMER_BACKENDS[timer_backend]
    with stats.PeakMemory(device) as mem:
        inputs = seeded_inputs(make_inputs_fn, case, device, seed)

        t0 = time.perf_counter()
        _ = triton_fn(**inputs)
        _sync(device)
        compile_time_ms = (time.perf_counter() - t0) * 1e3

        corr: CorrectnessResult | None = None
        if run_correctness:
            ref_out = reference_fn(**inputs)
            out = triton_fn(**inputs)
            _sync(device)
            corr = check_correctness(ref_out, out, case.dtype, meta.correctness.for_case(case.name))
            del ref_out, out

        st = stats.summarize(timer(lambda: triton_fn(**inputs), warmup_ms, rep_ms))
    p50 = st.p50
    per_s = stats.rates(stats.workload(case.params), p50)

    est = get_estimate_dict(estimate_fn, case.params)
    flops, bytes_ = est.get("flops"), est.get("bytes")
    tflops = compute_tflops(flops, p50) if flops else None
    gbps = compute_gbps(bytes_, p50) if bytes_ else None
    algo = est.get("algo_flops")
    peak = PEAKS_MI355X.get(roofline_unit)

    res = BenchResult(
        kernel=kernel_name, case_name=case.name, dtype=case.dtype, layout=case.layout,
        latency_ms_p50=p50, latency_ms_p90=st.p90, latency_ms_p95=st.p95, latency_ms_p99=st.p99,
        latency_ms_min=st.min, latency_ms_max=st.max, latency_ms_mean=st.mean,
        latency_ms_std=st.std, pass_type=pass_type, tflops=tflops, gbps=gbps,
        tail_ratio_p99_p50=st.tail, jitter_cv=st.jitter, **per_s,
        peak_mem_alloc_mb=mem.allocated_mib, peak_mem_reserved_mb=mem.reserved_mib,
        timer_backend=timer_backend, warmup_ms=warmup_ms, rep_ms=rep_ms, correctness=corr,
        compile_time_ms=compile_time_ms,
        effective_tops=tflops,
        algo_tops=compute_tflops(algo, p50) if algo else None,
        roofline_peak=peak, roofline_unit=roofline_unit,
    )
    # the roofline counts the work done (unmasked pairs for causal cases),
    # not the metric's 4*B*H*N^2*D
    rate = res.algo_tops if res.algo_tops else tflops
    res.roofline_fraction = (rate / peak) if (rate and peak) else None
    pre_fn = (stage_fns or {}).get("prepass")
    if pre_fn is not None and device.startswith("cuda"):
        pre_p50 = stats.summarize(timer(lambda: pre_fn(**inputs), warmup_ms / 4, rep_ms / 4)).p50
        res.prepass_ms_p50 = pre_p50
        pb = est.get("prepass_bytes")
        if pb and est.get("vtile_bytes"):
            pb += est["vtile_bytes"]  # the stage also converts V (v.to(float16))
        if pb:
            res.prepass_gbps = compute_gbps(pb, pre_p50)
            res.prepass_hbm_fraction = res.prepass_gbps / PEAKS_MI355X["hbm_gbps"]
    return res


def run_cpu_reference(
    *,
    kernel_name: str,
    make_inputs_fn: Callable,
    reference_fn: Callable,
    estimate_fn: Callable | None,
    case: Case,
    seed: int,
    reps: int = 3,
    max_rep_s: float = 30.0,
) -> BenchResult:
    """Time the pack's reference on this host's CPU cores (p50 of ``reps``;
    a single rep when one rep exceeds ``max_rep_s``)."""
    threads, model = cpu_info()
    torch.set_num_threads(threads)
    inputs = seeded_inputs(make_inputs_fn, case, "cpu", seed)
    times: list[float] = []
    for i in range(reps):
        t0 = time.perf_counter()
        reference_fn(**inputs)
        dt = time.perf_counter() - t0
        times.append(dt * 1e3)
        if dt > max_rep_s:
            break
    st = stats.summarize(times)
    est = get_estimate_dict(estimate_fn, case.params)
    flops = est.get("flops")
    tflops = compute_tflops(flops, st.p50) if flops else None
    return BenchResult(
        kernel=kernel_name, case_name=case.name, dtype=case.dtype, layout=case.layout,
        latency_ms_p50=st.p50, latency_ms_p90=st.p90, latency_ms_p95=st.p95, latency_ms_p99=st.p99,
        latency_ms_min=st.min, latency_ms_max=st.max, latency_ms_mean=st.mean,
        latency_ms_std=st.std, variant="cpu_ref", tflops=tflops, effective_tops=tflops,
        timer_backend="cpu_wall", warmup_ms=0.0, rep_ms=0.0, cpu_threads=threads, cpu_model=model,
    )
