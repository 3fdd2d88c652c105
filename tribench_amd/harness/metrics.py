"""Derived metrics (counterpart of tribench/metrics.py) and MI355X rooflines.

compute_tflops / compute_gbps / get_estimates keep the reference's meaning
(metrics.py:6-33).  Added: the MI355X peak table and the roofline fraction of
a measured rate.  Peaks are AMD's published dense (non-sparse) figures for
the MI355X (gfx950, 256 CUs at 2.4 GHz): INT8 5.0 POPS, FP8 5.0 PFLOPS,
FP16/BF16 2.5 PFLOPS, FP32 157.3 TFLOPS (vector), FP64 78.6 TFLOPS, HBM3E
8.0 TB/s.
"""
from __future__ import annotations

from typing import Any, Callable

# peak rates in T(FL)OPS, and HBM bandwidth in GB/s
PEAKS_MI355X: dict[str, float] = {
    # the published dense figures (256 CU x 4 SIMD x 2048 or 1024 ops/clk x
    # 2.4 GHz = 5033 / 2516, rounded as AMD quotes them; bench.py uses the same)
    "int8": 5000.0,
    "fp8": 5000.0,
    "fp16": 2500.0,
    "bf16": 2500.0,
    "fp32": 157.3,
    "fp64": 78.6,
    "hbm_gbps": 8000.0,
}


def compute_tflops(flops: float, latency_ms: float) -> float:
    """TFLOPS from a FLOP count and a latency in milliseconds."""
    if latency_ms <= 0:
        return 0.0
    return flops / (latency_ms * 1e-3) / 1e12


def compute_gbps(bytes_: float, latency_ms: float) -> float:
    """GB/s from a byte count and a latency in milliseconds."""
    if latency_ms <= 0:
        return 0.0
    return bytes_ / (latency_ms * 1e-3) / 1e9


def get_estimates(estimate_fn: Callable | None, case_params: dict[str, Any]) -> tuple[float | None, float | None]:
    """(flops, bytes) of the pack's estimate(), or (None, None)."""
    if estimate_fn is None:
        return None, None
    res = estimate_fn(case_params)
    return res.get("flops"), res.get("bytes")


def get_estimate_dict(estimate_fn: Callable | None, case_params: dict[str, Any]) -> dict[str, Any]:
    return {} if estimate_fn is None else dict(estimate_fn(case_params))


def roofline_fraction(rate: float | None, unit: str = "int8") -> float | None:
    """rate (in T(FL)OPS, or GB/s for unit 'hbm_gbps') over the MI355X peak."""
    if rate is None:
        return None
    return rate / PEAKS_MI355X[unit]
