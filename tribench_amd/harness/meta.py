"""meta.json parsing and validation (counterpart of tribench/meta.py).

Same required fields, value sets and messages as meta.py:20-182 of the
reference, with one difference: the ``triton`` entrypoint is optional because
this stack has no Triton.  A pack must then name at least one implementation
(``triton`` or a ``variants`` entry).
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Any

from .types import CaseDef, CorrectnessSpec, EntrypointsSpec, KernelMeta, SupportedSpec

VALID_DTYPES = {"fp16", "bf16", "fp32", "fp64"}
VALID_LAYOUTS = {"contiguous", "lastdim_contig"}
VALID_BACKENDS = {"cuda", "hip"}

REQUIRED_TOP_FIELDS = {
    "schema_version", "name", "family", "description",
    "entrypoints", "supported", "cases",
}
REQUIRED_ENTRYPOINT_FIELDS = {"make_inputs", "reference"}
IMPL_ENTRYPOINT_FIELDS = ("triton",)


def load_meta(path: str | Path) -> KernelMeta:
    path = Path(path)
    with open(path, "r", encoding="utf-8") as f:
        raw: dict[str, Any] = json.load(f)
    ep = raw.get("entrypoints", {})
    entrypoints = EntrypointsSpec(
        make_inputs=ep.get("make_inputs"),
        reference=ep.get("reference"),
        triton=ep.get("triton"),
        backward=ep.get("backward"),
        estimate=ep.get("estimate"),
        variants=ep.get("variants", {}),
    )
    sup = raw.get("supported", {})
    supported = SupportedSpec(
        dtypes=sup.get("dtypes", ["fp32"]),
        layouts=sup.get("layouts", ["contiguous"]),
        backends=sup.get("backends", ["hip"]),
    )
    cases: list[CaseDef] = []
    for c in raw.get("cases", []):
        params = {k: v for k, v in c.items() if k != "name"}
        cases.append(CaseDef(name=c["name"], params=params))
    corr = raw.get("correctness", {})
    correctness = CorrectnessSpec(
        atol=corr.get("atol", 1e-2),
        rtol=corr.get("rtol", 1e-2),
        per_dtype=corr.get("per_dtype", {}),
        max_abs=corr.get("max_abs"),
        min_cos=corr.get("min_cos"),
        per_case=corr.get("per_case", {}),
    )
    return KernelMeta(
        schema_version=raw["schema_version"],
        name=raw["name"],
        family=raw.get("family", ""),
        description=raw.get("description", ""),
        tags=raw.get("tags", []),
        entrypoints=entrypoints,
        supported=supported,
        cases=cases,
        correctness=correctness,
        metrics=raw.get("metrics", ""),
        notes=raw.get("notes", ""),
        kernel_dir=str(path.parent),
    )


def validate_meta(raw: dict[str, Any]) -> list[str]:
    """Validate a raw meta.json dict; returns error strings (empty = valid)."""
    errors: list[str] = []
    for field in sorted(REQUIRED_TOP_FIELDS):
        if field not in raw:
            errors.append(f"Missing required field: '{field}'")
    sv = raw.get("schema_version")
    if sv is not None and not isinstance(sv, str):
        errors.append(f"'schema_version' must be a string, got {type(sv).__name__}")
    ep = raw.get("entrypoints")
    if isinstance(ep, dict):
        for field in sorted(REQUIRED_ENTRYPOINT_FIELDS):
            if field not in ep:
                errors.append(f"Missing entrypoint: '{field}'")
        variants = ep.get("variants")
        if variants is not None:
            if not isinstance(variants, dict):
                errors.append("'entrypoints.variants' must be a dict")
            else:
                for k, v in variants.items():
                    if not isinstance(k, str) or not isinstance(v, str):
                        errors.append("'entrypoints.variants' must be a dict of string keys/values")
        has_impl = any(f in ep for f in IMPL_ENTRYPOINT_FIELDS) or bool(isinstance(variants, dict) and variants)
        if not has_impl:
            errors.append("No implementation: give 'triton' or at least one 'variants' entry")
    elif ep is not None:
        errors.append("'entrypoints' must be a dict")
    sup = raw.get("supported")
    if isinstance(sup, dict):
        for dt in sup.get("dtypes", []):
            if dt not in VALID_DTYPES:
                errors.append(f"Invalid dtype '{dt}'. Valid: {VALID_DTYPES}")
        for ly in sup.get("layouts", []):
            if ly not in VALID_LAYOUTS:
                errors.append(f"Invalid layout '{ly}'. Valid: {VALID_LAYOUTS}")
        for be in sup.get("backends", []):
            if be not in VALID_BACKENDS:
                errors.append(f"Invalid backend '{be}'. Valid: {VALID_BACKENDS}")
    elif sup is not None:
        errors.append("'supported' must be a dict")
    cases = raw.get("cases")
    if isinstance(cases, list):
        for i, c in enumerate(cases):
            if not isinstance(c, dict):
                errors.append(f"cases[{i}] must be a dict")
            elif "name" not in c:
                errors.append(f"cases[{i}] missing 'name' field")
    elif cases is not None:
        errors.append("'cases' must be a list")
    per_case = (raw.get("correctness") or {}).get("per_case", {})
    if not isinstance(per_case, dict):
        errors.append("'correctness.per_case' must be a dict")
    else:
        names = {c.get("name") for c in cases if isinstance(c, dict)} if isinstance(cases, list) else set()
        for name, o in per_case.items():
            if name not in names:
                errors.append(f"correctness.per_case names unknown case '{name}'")
            elif not isinstance(o, dict) or set(o) - {"atol", "rtol", "max_abs", "min_cos"}:
                errors.append(f"correctness.per_case['{name}'] takes atol, rtol, max_abs, min_cos")
    return errors


def validate_entrypoints(meta: KernelMeta) -> list[str]:
    """Check that entrypoint files exist (symbols resolve lazily at load)."""
    errors: list[str] = []
    kernel_dir = Path(meta.kernel_dir)
    for ep_name in ("make_inputs", "reference", "triton", "backward", "estimate"):
        spec = getattr(meta.entrypoints, ep_name)
        if spec is None:
            continue
        if ":" not in spec:
            errors.append(f"Entrypoint '{ep_name}' must be 'file.py:symbol', got '{spec}'")
            continue
        file_part, _ = spec.rsplit(":", 1)
        if not (kernel_dir / file_part).exists():
            errors.append(f"Entrypoint file not found: {kernel_dir / file_part}")
    for var_name, spec in meta.entrypoints.variants.items():
        if ":" not in spec:
            errors.append(f"Variant '{var_name}' must be 'file.py:symbol', got '{spec}'")
            continue
        file_part, _ = spec.rsplit(":", 1)
        if not (kernel_dir / file_part).exists():
            errors.append(f"Variant '{var_name}' file not found: {kernel_dir / file_part}")
    return errors
