"""Kernel packs: discovery under ``kernels/`` and by-path loading of their code.

A pack is a directory with a meta.json (see ``schema.py``) and the Python
files its entrypoints name as ``file.py:symbol``.  Each file is imported from
its path as the module ``tribench.kernels.<pack>.<file stem>`` with no parent
package in ``sys.modules`` — the way TriBench's registry imports pack files
(tribench/registry.py:62-75, 125-134) — so a pack file locates its own
resources (the HIP library) from ``__file__`` and a pack written for one
harness loads in the other.  A file is imported once per index and shared by
every entrypoint it defines.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path
from types import ModuleType
from typing import Callable

from . import schema
from .types import KernelMeta

KERNELS_DIR = Path(__file__).resolve().parent.parent / "kernels"


def import_by_path(path: Path, module_name: str) -> ModuleType:
    """Execute ``path`` as module ``module_name`` (registered in sys.modules
    under that name while and after it runs, so its own dataclasses and
    pickling resolve)."""
    spec = importlib.util.spec_from_file_location(module_name, str(path))
    if spec is None or spec.loader is None:
        raise ImportError(f"cannot import {path}")
    module = importlib.util.module_from_spec(spec)
    sys.modules[module_name] = module
    try:
        spec.loader.exec_module(module)
    except BaseException:
        sys.modules.pop(module_name, None)
        raise
    return module


class Pack:
    """One kernel pack: its parsed meta.json and its lazily imported files."""

    def __init__(self, meta: KernelMeta) -> None:
        self.meta = meta
        self.dir = Path(meta.kernel_dir)
        self._files: dict[str, ModuleType] = {}

    @property
    def name(self) -> str:
        return self.meta.name

    def resolve(self, spec: str) -> Callable:
        """The callable an entrypoint spec ``file.py:symbol`` names."""
        file_part, symbol = schema.split_spec(spec)
        module = self._files.get(file_part)
        if module is None:
            path = self.dir / file_part
            module = import_by_path(path, f"tribench.kernels.{self.name}.{path.stem}")
            self._files[file_part] = module
        try:
            return getattr(module, symbol)
        except AttributeError:
            raise AttributeError(f"{self.name}: {file_part} defines no '{symbol}'") from None

    def entry(self, role: str) -> Callable | None:
        """make_inputs / reference / triton / backward / estimate (None if absent)."""
        spec = getattr(self.meta.entrypoints, role)
        return None if spec is None else self.resolve(spec)

    def variant(self, name: str) -> Callable:
        spec = self.meta.entrypoints.variants.get(name)
        if spec is None:
            have = ", ".join(self.meta.entrypoints.variants) or "none"
            raise KeyError(f"{self.name}: no variant '{name}' (variants: {have})")
        return self.resolve(spec)

    def implementations(self) -> list[tuple[str, Callable]]:
        """(label, callable) of every implementation to test and time: the
        ``triton`` entrypoint, then the variants; an entrypoint spec that an
        earlier one already named is listed once, under the variant's name
        (this stack's packs put their HIP implementation in both slots)."""
        ep = self.meta.entrypoints
        labelled = [("triton", ep.triton)] + list(ep.variants.items())
        chosen: dict[str, str] = {}  # spec -> label
        for label, spec in labelled:
            if spec is None:
                continue
            if spec in chosen and label != "triton":
                chosen[spec] = label
            chosen.setdefault(spec, label)
        return [(label, self.resolve(spec)) for spec, label in chosen.items()]


class PackIndex:
    """Every pack under a kernels directory, by name.  A pack whose meta.json
    does not parse is left out and reported in ``broken``."""

    def __init__(self, kernels_dir: str | Path | None = None) -> None:
        self.root = Path(kernels_dir) if kernels_dir is not None else KERNELS_DIR
        self._packs: dict[str, Pack] = {}
        self.broken: dict[str, str] = {}
        for meta_path in sorted(self.root.glob("*/meta.json")):
            try:
                meta = schema.read(meta_path)
            except schema.SchemaError as exc:
                self.broken[str(meta_path)] = str(exc)
                continue
            if meta.name in self._packs:
                self.broken[str(meta_path)] = f"pack name '{meta.name}' is used by another pack"
                continue
            self._packs[meta.name] = Pack(meta)

    def names(self) -> list[str]:
        return sorted(self._packs)

    def metas(self) -> list[KernelMeta]:
        return [self._packs[n].meta for n in self.names()]

    def pack(self, name: str) -> Pack:
        try:
            return self._packs[name]
        except KeyError:
            raise KeyError(f"no kernel pack '{name}' (packs: {', '.join(self.names()) or 'none'})") from None

    def problems(self) -> dict[str, list[str]]:
        """Schema problems per meta.json path (empty when every pack is valid)."""
        return {path: [msg] for path, msg in self.broken.items()}
