"""run.json / summary.md writers (counterpart of tribench/io.py)."""
from __future__ import annotations

import dataclasses as dc
import datetime as _dt
import json
from pathlib import Path
from typing import Any

from .types import RunRecord


def _to_dict(obj: Any) -> Any:
    if dc.is_dataclass(obj):
        return {k: _to_dict(v) for k, v in dc.asdict(obj).items()}
    if isinstance(obj, (list, tuple)):
        return [_to_dict(x) for x in obj]
    return obj


def make_run_id(kernel: str, device: str) -> str:
    ts = _dt.datetime.now().strftime("%Y%m%d-%H%M%S")
    return f"{ts}_{kernel.replace(',', '+')}_{device.replace(':', '')}"


def write_json(record: RunRecord, output_dir: str | Path) -> Path:
    d = Path(output_dir) / record.run_id
    d.mkdir(parents=True, exist_ok=True)
    p = d / "run.json"
    p.write_text(json.dumps(_to_dict(record), indent=2))
    return p


def _fmt(v, spec: str) -> str:
    return "-" if v is None else format(v, spec)


def write_summary_md(record: RunRecord, output_dir: str | Path) -> Path:
    d = Path(output_dir) / record.run_id
    d.mkdir(parents=True, exist_ok=True)
    e = record.env
    lines = [f"# Run {record.run_id}", "",
             f"- GPU: {e.gpu_name} ({e.rocm_arch}), torch {e.torch_version}, HIP {e.hip_version}",
             f"- CPU: {e.cpu_model} ({e.cpu_threads} threads)",
             f"- git: {e.git_commit[:12]}{' (dirty)' if e.git_dirty else ''}; timer {record.timer_backend}", "",
             "| kernel | case | impl | dtype | p50 ms | p95 ms | eff. TOPS | roofline | prepass GB/s | correct |",
             "|---|---|---|---|---|---|---|---|---|---|"]
    for r in record.results:
        ok = "-" if r.correctness is None else ("PASS" if r.correctness.passed else "FAIL")
        roof = "-" if r.roofline_fraction is None else f"{100 * r.roofline_fraction:.1f}% {r.roofline_unit}"
        lines.append(f"| {r.kernel} | {r.case_name} | {r.variant or 'triton'} | {r.dtype} | "
                     f"{r.latency_ms_p50:.4f} | {r.latency_ms_p95:.4f} | {_fmt(r.effective_tops, '.1f')} | "
                     f"{roof} | {_fmt(r.prepass_gbps, '.0f')} | {ok} |")
    p = d / "summary.md"
    p.write_text("\n".join(lines) + "\n")
    return p
