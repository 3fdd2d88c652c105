"""meta.json of a kernel pack: its schema, written down as data, and a checker.

The schema is TriBench's (tribench/meta.py:20-29 lists the accepted dtype,
layout and backend names and the required fields; tribench/types.py the
parsed form, mirrored in ``types.py``).  A pack that this harness accepts is
also accepted by TriBench's ``validate-meta``: the ``triton`` entrypoint is
required here too.  On this ROCm stack there is no Triton, so the packs of
this repository point ``triton`` at their HIP implementation, which is also
their ``hip`` variant; :class:`~tribench_amd.harness.packs.Pack` lists such a
shared implementation once.

Two extensions, both optional: ``correctness.max_abs`` / ``min_cos`` (bounds
against the fp32 reference next to allclose) and ``correctness.per_case``
(per-case overrides of the four tolerance keys).
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Any

from .types import CaseDef, CorrectnessSpec, EntrypointsSpec, KernelMeta, SupportedSpec

# Accepted names (interface: the same sets as TriBench's harness).
DTYPES = ("fp16", "bf16", "fp32", "fp64")
LAYOUTS = ("contiguous", "lastdim_contig")
BACKENDS = ("cuda", "hip")

# field -> expected JSON type; every one of them must be present
TOP_LEVEL = {
    "schema_version": str,
    "name": str,
    "family": str,
    "description": str,
    "entrypoints": dict,
    "supported": dict,
    "cases": list,
}
ENTRYPOINT_ROLES_REQUIRED = ("make_inputs", "reference", "triton")
ENTRYPOINT_ROLES_OPTIONAL = ("backward", "estimate")
SUPPORTED_LISTS = {"dtypes": DTYPES, "layouts": LAYOUTS, "backends": BACKENDS}
TOLERANCE_KEYS = ("atol", "rtol", "max_abs", "min_cos")


class SchemaError(ValueError):
    """A meta.json that cannot be parsed into a KernelMeta."""


def split_spec(spec: Any) -> tuple[str, str]:
    """``"file.py:symbol"`` -> (``"file.py"``, ``"symbol"``)."""
    if not isinstance(spec, str) or spec.count(":") < 1:
        raise SchemaError(f"entrypoint {spec!r} is not of the form 'file.py:symbol'")
    file_part, _, symbol = spec.rpartition(":")
    if not file_part.endswith(".py") or not symbol.isidentifier():
        raise SchemaError(f"entrypoint {spec!r} is not of the form 'file.py:symbol'")
    return file_part, symbol


def _entrypoint_problems(ep: dict, pack_dir: Path | None) -> list[str]:
    out: list[str] = []
    specs: list[tuple[str, Any]] = []
    for role in ENTRYPOINT_ROLES_REQUIRED:
        if role not in ep:
            out.append(f"entrypoints: '{role}' is required")
        else:
            specs.append((role, ep[role]))
    specs += [(role, ep[role]) for role in ENTRYPOINT_ROLES_OPTIONAL if role in ep]
    variants = ep.get("variants", {})
    if not isinstance(variants, dict):
        out.append("entrypoints.variants must map variant names to 'file.py:symbol'")
    else:
        specs += [(f"variants.{name}", spec) for name, spec in variants.items()]
    for role, spec in specs:
        try:
            file_part, _ = split_spec(spec)
        except SchemaError as exc:
            out.append(f"entrypoints.{role}: {exc}")
            continue
        if pack_dir is not None and not (pack_dir / file_part).is_file():
            out.append(f"entrypoints.{role}: {file_part} does not exist in {pack_dir}")
    return out


def _tolerance_problems(corr: Any, case_names: set[str]) -> list[str]:
    if corr is None:
        return []
    if not isinstance(corr, dict):
        return ["correctness must be an object"]
    out = [f"correctness.{k} must be a number" for k in TOLERANCE_KEYS
           if k in corr and not isinstance(corr[k], (int, float))]
    per_case = corr.get("per_case", {})
    if not isinstance(per_case, dict):
        return out + ["correctness.per_case must map case names to tolerance overrides"]
    for name, over in per_case.items():
        if name not in case_names:
            out.append(f"correctness.per_case: no case named '{name}'")
        elif not isinstance(over, dict) or not set(over) <= set(TOLERANCE_KEYS):
            out.append(f"correctness.per_case['{name}']: allowed keys are {', '.join(TOLERANCE_KEYS)}")
    return out


def check(raw: Any, pack_dir: str | Path | None = None) -> list[str]:
    """Every problem of a meta.json object (empty when it is valid).  With
    ``pack_dir`` the entrypoint files must exist there too."""
    if not isinstance(raw, dict):
        return ["meta.json must hold a JSON object"]
    pack_dir = Path(pack_dir) if pack_dir is not None else None
    out: list[str] = []
    for field, kind in TOP_LEVEL.items():
        if field not in raw:
            out.append(f"'{field}' is required")
        elif not isinstance(raw[field], kind):
            out.append(f"'{field}' must be a {kind.__name__}, not {type(raw[field]).__name__}")
    if isinstance(raw.get("entrypoints"), dict):
        out += _entrypoint_problems(raw["entrypoints"], pack_dir)
    if isinstance(raw.get("supported"), dict):
        for key, allowed in SUPPORTED_LISTS.items():
            for value in raw["supported"].get(key, []):
                if value not in allowed:
                    out.append(f"supported.{key}: '{value}' is not one of {', '.join(allowed)}")
    names: set[str] = set()
    if isinstance(raw.get("cases"), list):
        for i, case in enumerate(raw["cases"]):
            name = case.get("name") if isinstance(case, dict) else None
            if not isinstance(name, str):
                out.append(f"cases[{i}] needs a 'name'")
            elif name in names:
                out.append(f"cases[{i}]: the name '{name}' is used twice")
            else:
                names.add(name)
    out += _tolerance_problems(raw.get("correctness"), names)
    return out


def read(path: str | Path) -> KernelMeta:
    """Parse a pack's meta.json; raises SchemaError listing every problem
    :func:`check` finds (a pack with any of them is not loaded)."""
    path = Path(path)
    try:
        raw = json.loads(path.read_text(encoding="utf-8"))
    except (OSError, ValueError) as exc:
        raise SchemaError(f"{path}: {exc}") from exc
    problems = check(raw, path.parent)
    if problems:
        raise SchemaError(f"{path}: " + "; ".join(problems))
    ep = raw["entrypoints"]
    sup = raw["supported"]
    corr = raw.get("correctness", {})
    return KernelMeta(
        schema_version=raw["schema_version"],
        name=raw["name"],
        family=raw["family"],
        description=raw["description"],
        tags=list(raw.get("tags", [])),
        entrypoints=EntrypointsSpec(
            make_inputs=ep["make_inputs"], reference=ep["reference"], triton=ep["triton"],
            backward=ep.get("backward"), estimate=ep.get("estimate"), variants=dict(ep.get("variants", {}))),
        supported=SupportedSpec(
            dtypes=list(sup.get("dtypes", ["fp32"])), layouts=list(sup.get("layouts", ["contiguous"])),
            backends=list(sup.get("backends", ["hip"]))),
        cases=[CaseDef(name=c["name"], params={k: v for k, v in c.items() if k != "name"})
               for c in raw["cases"]],
        correctness=CorrectnessSpec(
            atol=corr.get("atol", 1e-2), rtol=corr.get("rtol", 1e-2), per_dtype=dict(corr.get("per_dtype", {})),
            max_abs=corr.get("max_abs"), min_cos=corr.get("min_cos"), per_case=dict(corr.get("per_case", {}))),
        metrics=raw.get("metrics", ""),
        notes=raw.get("notes", ""),
        kernel_dir=str(path.parent),
    )
