"""Latency summaries and the quantities derived from them for a result row.

* :func:`summarize` — percentiles, mean and spread of per-call latencies, with
  the tail ratio p99/p50 and the jitter std/mean that run.json reports;
* :func:`workload` / :func:`rates` — tokens, elements and sequences of one
  call, read from a case's shape parameters, and their per-second rates;
* :class:`PeakMemory` — the device allocator's high-water marks over a block.
"""
from __future__ import annotations

import dataclasses as dc
from typing import Any, Iterable

import numpy as np
import torch


@dc.dataclass(frozen=True)
class LatencySummary:
    p50: float
    p90: float
    p95: float
    p99: float
    min: float
    max: float
    mean: float
    std: float

    @property
    def tail(self) -> float | None:
        """p99 / p50: how far the slow calls stray from the typical one."""
        return self.p99 / self.p50 if self.p50 > 0 else None

    @property
    def jitter(self) -> float | None:
        """Coefficient of variation std / mean."""
        return self.std / self.mean if self.mean > 0 else None


def summarize(latencies_ms: Iterable[float]) -> LatencySummary:
    a = np.asarray(list(latencies_ms), dtype=np.float64)
    if a.size == 0:
        raise ValueError("no latency samples")
    p50, p90, p95, p99 = (float(x) for x in np.percentile(a, [50, 90, 95, 99]))
    return LatencySummary(p50=p50, p90=p90, p95=p95, p99=p99, min=float(a.min()), max=float(a.max()),
                          mean=float(a.mean()), std=float(a.std()))


# The names under which a case may give each dimension (first match wins).
_DIMENSIONS = {
    "batch": ("batch_size", "B"),
    "seq": ("seq_len", "T"),
    "heads": ("num_heads", "H"),
    "head_dim": ("head_dim", "D"),
    "rows": ("M",),
    "cols": ("N", "K"),
}


@dc.dataclass(frozen=True)
class Workload:
    tokens: int | None = None
    elements: int | None = None
    sequences: int | None = None


def _dims(params: dict[str, Any]) -> dict[str, int]:
    found: dict[str, int] = {}
    for dim, keys in _DIMENSIONS.items():
        for key in keys:
            v = params.get(key)
            if isinstance(v, int) and not isinstance(v, bool) and v > 0:
                found[dim] = v
                break
    return found


def workload(params: dict[str, Any]) -> Workload:
    """Tokens (batch x sequence length), elements (of the main activation:
    batch x heads x tokens x head_dim for attention shapes, batch x rows x
    cols for matrix shapes, else the product of the dimensions given) and
    sequences (the batch) of one call; None where the case does not say."""
    d = _dims(params)
    batch, seq = d.get("batch"), d.get("seq")
    tokens = batch * seq if batch and seq else seq
    if {"heads", "seq", "head_dim"} <= d.keys():
        elements = (batch or 1) * d["heads"] * seq * d["head_dim"]
    elif {"rows", "cols"} <= d.keys():
        elements = (batch or 1) * d["rows"] * d["cols"]
    elif d:
        elements = int(np.prod(list(d.values())))
    else:
        elements = None
    return Workload(tokens=tokens, elements=elements, sequences=batch)


def rates(work: Workload, latency_ms: float) -> dict[str, float | None]:
    """Per-second rates of a workload done in ``latency_ms``."""
    if latency_ms <= 0:
        return {"tokens_per_s": None, "elements_per_s": None, "sequences_per_s": None}
    per_s = 1e3 / latency_ms
    return {f"{k}_per_s": (None if v is None else v * per_s) for k, v in dc.asdict(work).items()}


class PeakMemory:
    """High-water marks of torch's caching allocator (MiB) over a ``with``
    block on a GPU device; both stay None on the CPU."""

    def __init__(self, device: str) -> None:
        self.device = device
        self.allocated_mib: float | None = None
        self.reserved_mib: float | None = None

    def _active(self) -> bool:
        return self.device.startswith("cuda") and torch.cuda.is_available()

    def __enter__(self) -> "PeakMemory":
        if self._active():
            torch.cuda.reset_peak_memory_stats(self.device)
        return self

    def __exit__(self, *exc) -> None:
        if self._active():
            mib = float(1 << 20)
            self.allocated_mib = torch.cuda.max_memory_allocated(self.device) / mib
            self.reserved_mib = torch.cuda.max_memory_reserved(self.device) / mib
