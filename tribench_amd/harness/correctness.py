"""Correctness gate (counterpart of tribench/correctness.py).

Same tolerance precedence and allclose test as correctness.py:14-106 of the
reference; the result also carries the cosine similarity, and the pack may
state north-star bounds (``max_abs``, ``min_cos`` in meta.json's
``correctness``) that must hold as well.  ``correctness.per_case`` may
override any of the four for a named case (callers pass
``spec.for_case(name)``).
"""
from __future__ import annotations

from typing import Any

import torch

from .types import CorrectnessResult, CorrectnessSpec

DEFAULT_TOLERANCES: dict[str, dict[str, float]] = {
    "fp32": {"atol": 1e-5, "rtol": 1e-4},
    "fp64": {"atol": 1e-7, "rtol": 1e-5},
    "fp16": {"atol": 1e-2, "rtol": 1e-2},
    "bf16": {"atol": 1e-2, "rtol": 1e-2},
}


def _get_tolerance(dtype_str: str, spec: CorrectnessSpec) -> tuple[float, float]:
    """Per-dtype override, then a non-default pack tolerance, then the defaults."""
    if dtype_str in spec.per_dtype:
        d = spec.per_dtype[dtype_str]
        return d.get("atol", spec.atol), d.get("rtol", spec.rtol)
    if spec.atol != 1e-2 or spec.rtol != 1e-2:
        return spec.atol, spec.rtol
    if dtype_str in DEFAULT_TOLERANCES:
        d = DEFAULT_TOLERANCES[dtype_str]
        return d["atol"], d["rtol"]
    return spec.atol, spec.rtol


def cosine_similarity(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().flatten()
    b = b.detach().double().flatten()
    den = float(a.norm() * b.norm())
    if den == 0.0:
        return 1.0 if float((a - b).abs().max()) == 0.0 else 0.0
    return float(a @ b) / den


def check_correctness(ref_output: Any, tri_output: Any, dtype_str: str, spec: CorrectnessSpec) -> CorrectnessResult:
    """Compare a reference and an implementation output (tensors or sequences)."""
    atol, rtol = _get_tolerance(dtype_str, spec)

    def _compare(ref: Any, out: Any):
        if isinstance(ref, (list, tuple)) and isinstance(out, (list, tuple)):
            if len(ref) != len(out):
                return False, 0.0, 0.0, None, f"Length mismatch: ref={len(ref)}, out={len(out)}"
            ok, ma, mr, cmin, msgs = True, 0.0, 0.0, None, []
            for i, (r, t) in enumerate(zip(ref, out)):
                p, a, rel, c, msg = _compare(r, t)
                ok = ok and p
                ma, mr = max(ma, a), max(mr, rel)
                if c is not None:
                    cmin = c if cmin is None else min(cmin, c)
                if not p:
                    msgs.append(f"item[{i}]: {msg}")
            return ok, ma, mr, cmin, "; ".join(msgs)
        if not isinstance(ref, torch.Tensor):
            return True, 0.0, 0.0, None, ""
        if not isinstance(out, torch.Tensor):
            return False, 0.0, 0.0, None, f"Expected tensor, got {type(out)}"
        if ref.shape != out.shape:
            return False, 0.0, 0.0, None, f"Shape mismatch: ref={tuple(ref.shape)}, out={tuple(out.shape)}"
        r = ref.float()
        o = out.float().to(r.device)
        diff = (r - o).abs()
        max_abs = float(diff.max()) if diff.numel() else 0.0
        max_rel = float((diff / r.abs().clamp(min=1e-20)).max()) if diff.numel() else 0.0
        cos = cosine_similarity(r, o) if diff.numel() else 1.0
        passed = bool(torch.allclose(r, o, atol=atol, rtol=rtol))
        notes = []
        if spec.max_abs is not None and max_abs > spec.max_abs:
            passed = False
            notes.append(f"max_abs {max_abs:.3e} > {spec.max_abs}")
        if spec.min_cos is not None and cos < spec.min_cos:
            passed = False
            notes.append(f"cosine {cos:.6f} < {spec.min_cos}")
        msg = "" if passed else (f"max_abs_err={max_abs:.6e}, max_rel_err={max_rel:.6e}, cos={cos:.6f}"
                                 + (f" [{'; '.join(notes)}]" if notes else ""))
        return passed, max_abs, max_rel, cos, msg

    try:
        passed, max_abs, max_rel, cos, msg = _compare(ref_output, tri_output)
        if not passed:
            msg = (msg or "Comparison failed") + f" (atol={atol}, rtol={rtol})"
    except Exception as exc:  # the gate reports, it never raises
        return CorrectnessResult(passed=False, atol=atol, rtol=rtol, error_msg=str(exc))
    return CorrectnessResult(passed=passed, atol=atol, rtol=rtol, max_abs_err=max_abs, max_rel_err=max_rel,
                             cosine=cos, error_msg=msg)
