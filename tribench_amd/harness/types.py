"""Schema and result types of the harness (counterpart of tribench/types.py).

Same dataclasses and fields as the reference (types.py:24-147); BenchResult
gains the MI355X report fields: effective TOPS, roofline peak and fraction,
pre-pass time and HBM fraction, cosine similarity, and CPU-baseline details.
"""
from __future__ import annotations

import dataclasses as dc
from typing import Any, Protocol, runtime_checkable

import torch


@dc.dataclass
class CaseDef:
    name: str
    params: dict[str, Any]


@dc.dataclass
class SupportedSpec:
    dtypes: list[str]
    layouts: list[str] = dc.field(default_factory=lambda: ["contiguous"])
    backends: list[str] = dc.field(default_factory=lambda: ["hip"])


@dc.dataclass
class EntrypointsSpec:
    make_inputs: str
    reference: str
    triton: str | None = None
    backward: str | None = None
    estimate: str | None = None
    variants: dict[str, str] = dc.field(default_factory=dict)


@dc.dataclass
class CorrectnessSpec:
    """Correctness thresholds: allclose(atol, rtol) as the reference, plus the
    optional north-star bounds ``max_abs`` and ``min_cos`` against the fp32
    reference output."""
    atol: float = 1e-2
    rtol: float = 1e-2
    per_dtype: dict[str, dict[str, float]] = dc.field(default_factory=dict)
    max_abs: float | None = None
    min_cos: float | None = None
    # case name -> overrides of atol / rtol / max_abs / min_cos for that case
    per_case: dict[str, dict[str, float]] = dc.field(default_factory=dict)

    def for_case(self, case_name: str | None) -> "CorrectnessSpec":
        """This spec with the case's overrides applied (itself if it has none)."""
        o = self.per_case.get(case_name or "", {})
        if not o:
            return self
        return dc.replace(self, atol=o.get("atol", self.atol), rtol=o.get("rtol", self.rtol),
                          per_dtype={} if ("atol" in o or "rtol" in o) else self.per_dtype,
                          max_abs=o.get("max_abs", self.max_abs), min_cos=o.get("min_cos", self.min_cos))


@dc.dataclass
class KernelMeta:
    schema_version: str
    name: str
    family: str
    description: str
    tags: list[str]
    entrypoints: EntrypointsSpec
    supported: SupportedSpec
    cases: list[CaseDef]
    correctness: CorrectnessSpec
    metrics: str
    notes: str = ""
    kernel_dir: str = ""


@runtime_checkable
class KernelEntrypoints(Protocol):
    def make_inputs(self, case: dict, device: str, seed: int, dtype: Any) -> dict: ...
    def reference(self, **inputs: Any) -> Any: ...


@dc.dataclass
class CorrectnessResult:
    passed: bool
    atol: float
    rtol: float
    max_abs_err: float = 0.0
    max_rel_err: float = 0.0
    cosine: float | None = None
    error_msg: str = ""


@dc.dataclass
class BenchResult:
    kernel: str
    case_name: str
    dtype: str
    layout: str
    latency_ms_p50: float
    latency_ms_p90: float
    latency_ms_p95: float
    latency_ms_p99: float
    latency_ms_min: float
    latency_ms_max: float
    latency_ms_mean: float
    latency_ms_std: float
    pass_type: str = "forward"
    variant: str | None = None
    tflops: float | None = None
    gbps: float | None = None
    triton_vs_variant_p50_ratio: float | None = None
    tail_ratio_p99_p50: float | None = None
    jitter_cv: float | None = None
    tokens_per_s: float | None = None
    elements_per_s: float | None = None
    sequences_per_s: float | None = None
    peak_mem_alloc_mb: float | None = None
    peak_mem_reserved_mb: float | None = None
    timer_backend: str = "hip_event"
    warmup_ms: float = 200.0
    rep_ms: float = 2000.0
    correctness: CorrectnessResult | None = None
    compile_time_ms: float | None = None
    # MI355X report fields
    effective_tops: float | None = None      # metric ops (estimate "flops") / p50
    algo_tops: float | None = None           # algorithmic ops / p50
    roofline_peak: float | None = None       # TOPS of the bounding unit
    roofline_unit: str | None = None
    roofline_fraction: float | None = None   # effective_tops / roofline_peak
    prepass_ms_p50: float | None = None
    prepass_gbps: float | None = None
    prepass_hbm_fraction: float | None = None
    cpu_threads: int | None = None
    cpu_model: str | None = None


@dc.dataclass
class EnvInfo:
    torch_version: str = ""
    hip_version: str = ""
    rocm_arch: str = ""
    gpu_name: str = ""
    gpu_count: int = 0
    cpu_model: str = ""
    cpu_threads: int = 0
    git_commit: str = ""
    git_dirty: bool = False
    cmdline: str = ""
    timestamp_utc: str = ""


@dc.dataclass
class RunRecord:
    schema_version: str = "1.0"
    run_id: str = ""
    env: EnvInfo = dc.field(default_factory=EnvInfo)
    seed: int = 0
    timer_backend: str = "hip_event"
    warmup_ms: float = 200.0
    rep_ms: float = 2000.0
    quantiles: list[float] = dc.field(default_factory=lambda: [0.5, 0.9, 0.95, 0.99])
    results: list[BenchResult] = dc.field(default_factory=list)


DTYPE_MAP: dict[str, torch.dtype] = {
    "fp16": torch.float16,
    "fp32": torch.float32,
    "bf16": torch.bfloat16,
    "fp64": torch.float64,
}
DTYPE_STR_MAP: dict[torch.dtype, str] = {v: k for k, v in DTYPE_MAP.items()}


def resolve_dtype(s: str) -> torch.dtype:
    if s not in DTYPE_MAP:
        raise ValueError(f"Unknown dtype '{s}'. Supported: {list(DTYPE_MAP.keys())}")
    return DTYPE_MAP[s]
