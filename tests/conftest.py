"""Shared test setup: the `gpu` marker, repo-root imports, pack loaders."""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACK = ROOT / "tribench_amd" / "kernels" / "sage_attn"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


def load_pack_module(stem: str):
    """Import a kernel-pack file by path, the way the harness registry does."""
    name = f"tribench.kernels.sage_attn.{stem}"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PACK / f"{stem}.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pack_ref():
    return load_pack_module("reference")


@pytest.fixture(scope="session")
def hip_impl():
    return load_pack_module("hip_impl")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    return torch.device("cuda:0")
