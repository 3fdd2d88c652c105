"""Tail/jitter/domain throughputs and peak memory (counterpart of tribench/eval_metrics.py)."""
from __future__ import annotations

import dataclasses as dc
from typing import Any

import torch


@dc.dataclass
class DomainThroughput:
    tokens_per_s: float | None = None
    elements_per_s: float | None = None
    sequences_per_s: float | None = None


def compute_tail_ratio(p99_ms: float, p50_ms: float) -> float | None:
    return None if p50_ms <= 0 else p99_ms / p50_ms


def compute_jitter_cv(std_ms: float, mean_ms: float) -> float | None:
    return None if mean_ms <= 0 else std_ms / mean_ms


def _positive_int(v: Any) -> int | None:
    if isinstance(v, bool) or not isinstance(v, int) or v <= 0:
        return None
    return v


def _infer_domain_counts(p: dict[str, Any]) -> tuple[int | None, int | None, int | None]:
    """Token / element / sequence counts from common case keys (eval_metrics.py:34-77)."""
    b = _positive_int(p.get("B")) or _positive_int(p.get("batch_size"))
    t = _positive_int(p.get("T")) or _positive_int(p.get("seq_len"))
    tokens = b * t if (b is not None and t is not None) else t
    sequences = b
    n, m = _positive_int(p.get("N")), _positive_int(p.get("M"))
    h, s = _positive_int(p.get("H")), _positive_int(p.get("S"))
    heads, hd = _positive_int(p.get("num_heads")), _positive_int(p.get("head_dim"))
    elements = None
    if b is not None and m is not None and n is not None:
        elements = b * m * n
    elif m is not None and n is not None:
        elements = m * n
    elif b is not None and t is not None and h is not None:
        elements = b * t * h
    elif b is not None and s is not None and h is not None:
        elements = b * s * h
    elif b is not None and heads is not None and t is not None and hd is not None:
        elements = b * heads * t * hd
    elif n is not None and b is not None:
        elements = b * n
    elif n is not None:
        elements = n
    return tokens, elements, sequences


def compute_domain_throughputs(case_params: dict[str, Any], latency_ms: float) -> DomainThroughput:
    if latency_ms <= 0:
        return DomainThroughput()
    sec = latency_ms * 1e-3
    tokens, elements, sequences = _infer_domain_counts(case_params)
    return DomainThroughput(
        tokens_per_s=None if tokens is None else tokens / sec,
        elements_per_s=None if elements is None else elements / sec,
        sequences_per_s=None if sequences is None else sequences / sec,
    )


def reset_peak_memory_stats(device: str) -> None:
    if device.startswith("cuda") and torch.cuda.is_available():
        try:
            torch.cuda.reset_peak_memory_stats(device=device)
        except Exception:
            pass


def read_peak_memory_mb(device: str) -> tuple[float | None, float | None]:
    if not device.startswith("cuda") or not torch.cuda.is_available():
        return None, None
    try:
        mib = 1024.0 * 1024.0
        return (torch.cuda.max_memory_allocated(device=device) / mib,
                torch.cuda.max_memory_reserved(device=device) / mib)
    except Exception:
        return None, None
