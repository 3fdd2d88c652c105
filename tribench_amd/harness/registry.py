"""Kernel-pack discovery and lazy loading (counterpart of tribench/registry.py).

Packs are ``kernels/<name>/meta.json`` directories; entrypoints are
``file.py:symbol`` and are imported by file path under the module name
``tribench.kernels.<name>.<stem>`` with no parent package, exactly as the
reference does (registry.py:62-75, 125-134), so a pack written for one
harness loads in the other.
"""
from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path
from types import ModuleType
from typing import Any, Callable

from .meta import load_meta, validate_entrypoints, validate_meta
from .types import KernelMeta

_DEFAULT_KERNELS_DIR = Path(__file__).resolve().parent.parent / "kernels"


class KernelRegistry:
    """Discover and lazily load kernel packs from ``kernels/*/meta.json``."""

    def __init__(self, kernels_dir: str | Path | None = None) -> None:
        self._kernels_dir = Path(kernels_dir) if kernels_dir else _DEFAULT_KERNELS_DIR
        self._metas: dict[str, KernelMeta] = {}
        self._modules: dict[str, Any] = {}
        self.scan_errors: dict[str, str] = {}
        self._scan()

    def _scan(self) -> None:
        if not self._kernels_dir.is_dir():
            return
        for meta_path in sorted(self._kernels_dir.glob("*/meta.json")):
            try:
                meta = load_meta(meta_path)
                self._metas[meta.name] = meta
            except Exception as exc:  # a broken pack must not hide the others
                self.scan_errors[str(meta_path)] = f"{exc.__class__.__name__}: {exc}"

    def list_kernels(self) -> list[KernelMeta]:
        return list(self._metas.values())

    def get_meta(self, name: str) -> KernelMeta:
        if name not in self._metas:
            available = ", ".join(sorted(self._metas)) or "(none)"
            raise KeyError(f"Kernel '{name}' not found. Available: {available}")
        return self._metas[name]

    def kernel_names(self) -> list[str]:
        return sorted(self._metas)

    def load_symbol(self, name: str, ep_spec: str) -> Callable:
        meta = self.get_meta(name)
        key = f"{name}::{ep_spec}"
        if key in self._modules:
            return self._modules[key]
        file_part, symbol = ep_spec.rsplit(":", 1)
        file_path = Path(meta.kernel_dir) / file_part
        module = self._import_file(file_path, f"tribench.kernels.{name}.{file_path.stem}")
        func = getattr(module, symbol)
        self._modules[key] = func
        return func

    def load_make_inputs(self, name: str) -> Callable:
        return self.load_symbol(name, self.get_meta(name).entrypoints.make_inputs)

    def load_reference(self, name: str) -> Callable:
        return self.load_symbol(name, self.get_meta(name).entrypoints.reference)

    def load_triton(self, name: str) -> Callable | None:
        spec = self.get_meta(name).entrypoints.triton
        return None if spec is None else self.load_symbol(name, spec)

    def load_backward(self, name: str) -> Callable | None:
        spec = self.get_meta(name).entrypoints.backward
        return None if spec is None else self.load_symbol(name, spec)

    def load_variant(self, name: str, variant_name: str) -> Callable:
        spec = self.get_meta(name).entrypoints.variants.get(variant_name)
        if spec is None:
            raise KeyError(f"Variant '{variant_name}' not found in kernel '{name}'")
        return self.load_symbol(name, spec)

    def load_estimate(self, name: str) -> Callable | None:
        spec = self.get_meta(name).entrypoints.estimate
        return None if spec is None else self.load_symbol(name, spec)

    def implementations(self, name: str) -> list[tuple[str, Callable]]:
        """[("triton", fn)] if the pack has a main entrypoint, then its variants."""
        impls: list[tuple[str, Callable]] = []
        main = self.load_triton(name)
        if main is not None:
            impls.append(("triton", main))
        for v in self.get_meta(name).entrypoints.variants:
            impls.append((v, self.load_variant(name, v)))
        return impls

    def validate_all(self) -> dict[str, list[str]]:
        report: dict[str, list[str]] = {}
        for name, meta in self._metas.items():
            with open(Path(meta.kernel_dir) / "meta.json", "r") as f:
                raw = json.load(f)
            errors = validate_meta(raw) + validate_entrypoints(meta)
            if errors:
                report[name] = errors
        for path, err in self.scan_errors.items():
            report[path] = [err]
        return report

    @staticmethod
    def _import_file(file_path: Path, module_name: str) -> ModuleType:
        spec = importlib.util.spec_from_file_location(module_name, str(file_path))
        if spec is None or spec.loader is None:
            raise ImportError(f"Cannot load {file_path}")
        module = importlib.util.module_from_spec(spec)
        sys.modules[module_name] = module
        spec.loader.exec_module(module)
        return module
