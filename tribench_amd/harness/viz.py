"""Self-contained HTML report of a run (counterpart of tribench/viz.py).

The reference draws its charts with Chart.js fetched from a CDN
(viz.py:227) and lists CUDA/Triton fields (viz.py:515-518).  This report needs
no network: environment cards with the ROCm fields (HIP version, gcnArchName),
the result table with the MI355X columns (effective and algorithmic TOPS,
roofline fraction of the bounding unit, pre-pass time and HBM fraction,
correctness with cosine) and bar charts drawn as inline SVG.  Like the
reference, ``generate_run_plots(record, run_dir)`` writes ``report.html`` into
the run directory and returns its path (viz.py:495-533).
"""
from __future__ import annotations

import html
from pathlib import Path

from .types import BenchResult, RunRecord

_COLORS = ["#5470c6", "#ee6666", "#91cc75", "#8675a9", "#fac858", "#73c0de", "#3ba272", "#fc8452"]


def _esc(s) -> str:
    return html.escape("" if s is None else str(s), quote=True)


def _fmt(v, spec: str) -> str:
    return "-" if v is None else format(v, spec)


def _impl(r: BenchResult) -> str:
    return r.variant or "triton"


def _passed(r: BenchResult) -> bool:
    return r.correctness is None or r.correctness.passed


def _bars_svg(title: str, rows: list[tuple[str, float, str]], unit: str, vmax: float | None = None) -> str:
    """Horizontal bars: (label, value, colour) each; vmax fixes the scale (e.g. 1.0 for fractions)."""
    if not rows:
        return ""
    top = vmax if vmax is not None else max(v for _, v, _ in rows) or 1.0
    lw, bw, h = 330, 420, 22
    out = [f'<h2>{_esc(title)}</h2>',
           f'<svg class="chart" width="{lw + bw + 110}" height="{h * len(rows) + 10}" '
           f'xmlns="http://www.w3.org/2000/svg" role="img">']
    for i, (label, v, col) in enumerate(rows):
        y = 5 + i * h
        w = max(1.0, bw * min(v / top, 1.0)) if top > 0 else 1.0
        out.append(f'<text x="{lw - 8}" y="{y + 15}" text-anchor="end">{_esc(label)}</text>'
                   f'<rect x="{lw}" y="{y + 3}" width="{w:.1f}" height="{h - 6}" fill="{col}"/>'
                   f'<text x="{lw + w + 6:.1f}" y="{y + 15}">{_esc(format(v, ".4g"))} {_esc(unit)}</text>')
    out.append("</svg>")
    return "\n".join(out)


_COLUMNS = ["kernel", "case", "pass", "dtype", "impl", "min ms", "p50 ms", "p90 ms", "p95 ms", "p99 ms",
            "CV", "p99/p50", "eff. TOPS", "algo TOPS", "roofline", "pre-pass ms", "pre-pass GB/s",
            "pre-pass HBM", "max abs err", "cosine", "correct"]


def _row_html(r: BenchResult) -> str:
    c = r.correctness
    roof = "-" if r.roofline_fraction is None else f"{100 * r.roofline_fraction:.1f}% of {r.roofline_peak:g} {r.roofline_unit or ''}"
    impl = _impl(r)
    if r.cpu_threads:
        impl = f"{impl} ({r.cpu_threads} threads)"
    cells = [r.kernel, r.case_name, r.pass_type, r.dtype, impl, f"{r.latency_ms_min:.4f}",
             f"{r.latency_ms_p50:.4f}", f"{r.latency_ms_p90:.4f}", f"{r.latency_ms_p95:.4f}",
             f"{r.latency_ms_p99:.4f}", _fmt(r.jitter_cv, ".3f"), _fmt(r.tail_ratio_p99_p50, ".3f"),
             _fmt(r.effective_tops, ".1f"), _fmt(r.algo_tops, ".1f"), roof, _fmt(r.prepass_ms_p50, ".4f"),
             _fmt(r.prepass_gbps, ".0f"),
             "-" if r.prepass_hbm_fraction is None else f"{100 * r.prepass_hbm_fraction:.1f}%",
             "-" if c is None else f"{c.max_abs_err:.3e}", "-" if c is None or c.cosine is None else f"{c.cosine:.6f}",
             "-" if c is None else ("PASS" if c.passed else "FAIL")]
    cls = "" if _passed(r) else ' class="fail"'
    return f"<tr{cls}>" + "".join(f"<td>{_esc(x)}</td>" for x in cells) + "</tr>"


_STYLE = """
body{background:#0d1117;color:#c9d1d9;font-family:-apple-system,"Segoe UI",Roboto,sans-serif;padding:2rem}
h1{color:#f0f6fc;font-size:1.7rem;margin:0 0 .3rem}
h2{color:#f0f6fc;font-size:1.1rem;margin:1.8rem 0 .6rem}
.run-id{color:#8b949e;font-size:.85rem;margin-bottom:1.4rem}
.cards{display:grid;grid-template-columns:repeat(auto-fill,minmax(190px,1fr));gap:.6rem}
.card{background:#161b22;border:1px solid #30363d;border-radius:6px;padding:.6rem .9rem}
.label{font-size:.65rem;text-transform:uppercase;letter-spacing:.06em;color:#8b949e}
.value{font-size:.92rem;font-weight:600;color:#f0f6fc;word-break:break-all}
table{border-collapse:collapse;font-size:.78rem}
th,td{border:1px solid #30363d;padding:.3rem .5rem;text-align:right;white-space:nowrap}
th{background:#161b22;color:#f0f6fc}
td:nth-child(-n+5){text-align:left}
tr.fail td{color:#ff7b72}
svg.chart text{fill:#c9d1d9;font-size:12px}
"""


def render_html(record: RunRecord) -> str:
    """The report as one HTML string (no scripts, no external resources)."""
    e = record.env
    git = (e.git_commit[:12] if e.git_commit else "N/A") + (" (dirty)" if e.git_dirty else "")
    cards = [("GPU", f"{e.gpu_name or 'N/A'} ({e.rocm_arch or '?'})"), ("GPUs visible", e.gpu_count),
             ("HIP", e.hip_version or "N/A"), ("PyTorch", e.torch_version or "N/A"),
             ("CPU", f"{e.cpu_model or 'N/A'} ({e.cpu_threads} threads)"), ("git", git),
             ("timer", record.timer_backend), ("warmup / rep", f"{record.warmup_ms} ms / {record.rep_ms} ms"),
             ("seed", record.seed), ("timestamp (UTC)", e.timestamp_utc or "N/A")]
    kernels = list(dict.fromkeys(f"{r.kernel} [{_impl(r)}]" for r in record.results))
    color = {k: _COLORS[i % len(_COLORS)] for i, k in enumerate(kernels)}
    ok = [r for r in record.results if _passed(r)]
    lab = lambda r: f"{r.case_name} {r.dtype} [{_impl(r)}]"
    col = lambda r: color[f"{r.kernel} [{_impl(r)}]"]
    gpu = [r for r in ok if not r.cpu_threads]
    parts = ["<!DOCTYPE html>", '<html lang="en"><head><meta charset="UTF-8">',
             f"<title>TriBench report - {_esc(record.run_id)}</title><style>{_STYLE}</style></head><body>",
             "<h1>TriBench report</h1>", f'<div class="run-id">{_esc(record.run_id)}</div>',
             '<div class="cards">']
    parts += [f'<div class="card"><div class="label">{_esc(k)}</div><div class="value">{_esc(v)}</div></div>'
              for k, v in cards]
    parts.append("</div>")
    parts.append(_bars_svg("p50 latency", [(lab(r), r.latency_ms_p50, col(r)) for r in gpu], "ms"))
    parts.append(_bars_svg("Effective TOPS (metric ops / p50)",
                           [(lab(r), r.effective_tops, col(r)) for r in gpu if r.effective_tops], "TOPS"))
    parts.append(_bars_svg("Roofline fraction (algorithmic rate / peak of the bounding unit)",
                           [(lab(r), r.roofline_fraction, col(r)) for r in gpu if r.roofline_fraction is not None],
                           "", vmax=1.0))
    parts.append("<h2>Results</h2><table><tr>" + "".join(f"<th>{_esc(c)}</th>" for c in _COLUMNS) + "</tr>")
    parts += [_row_html(r) for r in record.results]
    parts.append("</table></body></html>")
    return "\n".join(p for p in parts if p)


def generate_run_plots(record: RunRecord, run_dir: str | Path) -> list[Path]:
    """Write ``report.html`` into run_dir; returns [its path], or [] with no results."""
    if not record.results:
        return []
    run_dir = Path(run_dir)
    run_dir.mkdir(parents=True, exist_ok=True)
    out = run_dir / "report.html"
    out.write_text(render_html(record), encoding="utf-8")
    return [out]
