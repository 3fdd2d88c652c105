"""The benchmark grid of a kernel pack and the seeded inputs of each point.

A grid point is one named case of meta.json (its shape parameters) in one
dtype and one layout; the grid is every case x supported dtype x supported
layout, or the subsets the command line asks for.  Inputs come from the
pack's ``make_inputs(params, device, seed, dtype)``.  Before calling it the
harness seeds torch's global generators (CPU, then every GPU) with the run
seed, in the order TriBench's harness does (tribench/gen.py:57-69), so a pack
that draws from them gets the same numbers under either harness.
"""
from __future__ import annotations

import dataclasses as dc
import itertools
from typing import Any, Callable, Sequence

import torch

from .types import KernelMeta, resolve_dtype


@dc.dataclass(frozen=True)
class Case:
    """One point of the grid."""

    name: str
    params: dict[str, Any]
    dtype: str
    layout: str

    def label(self) -> str:
        return f"{self.name} dtype={self.dtype}"


def _subset(what: str, pack: str, wanted: Sequence[str] | None, offered: Sequence[str]) -> list[str]:
    """``wanted`` (in its order, repeats dropped) if every entry is offered,
    else ValueError naming the ones that are not; all of ``offered`` when
    nothing is asked for."""
    if not wanted:
        return list(offered)
    missing = [w for w in wanted if w not in offered]
    if missing:
        raise ValueError(f"kernel '{pack}' has no {what} {', '.join(repr(m) for m in missing)} "
                         f"(it offers: {', '.join(offered)})")
    return list(dict.fromkeys(wanted))


def case_grid(meta: KernelMeta, *, cases: Sequence[str] | None = None, dtypes: Sequence[str] | None = None,
              layouts: Sequence[str] | None = None) -> list[Case]:
    """The grid of ``meta``'s cases, dtypes and layouts, narrowed to the
    requested names.  Case names the pack does not offer are passed over
    (one command line may name cases of several packs, as
    tribench/gen.py:19-20 allows); a requested dtype or layout the pack does
    not support is a ValueError."""
    defs = {c.name: c for c in meta.cases}
    names = [n for n in defs if n in set(cases)] if cases else list(defs)
    dts = _subset("dtype", meta.name, dtypes, meta.supported.dtypes)
    lays = _subset("layout", meta.name, layouts, meta.supported.layouts)
    return [Case(name=n, params=dict(defs[n].params), dtype=d, layout=lay)
            for n, d, lay in itertools.product(names, dts, lays)]


def seeded_inputs(make_inputs: Callable, case: Case, device: str, seed: int) -> dict[str, Any]:
    """Seed torch's global generators with ``seed``, then build the case's
    inputs with the pack's ``make_inputs``."""
    torch.manual_seed(seed)
    if device.startswith("cuda") and torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)
    return make_inputs(dict(case.params), device, seed, resolve_dtype(case.dtype))
