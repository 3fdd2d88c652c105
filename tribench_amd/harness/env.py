"""Environment snapshot for run records (counterpart of tribench/env.py), ROCm-aware."""
from __future__ import annotations

import datetime as _dt
import os
import subprocess

from .types import EnvInfo


def _git(args: list[str]) -> str:
    try:
        return subprocess.run(["git", *args], capture_output=True, text=True, timeout=5).stdout.strip()
    except Exception:
        return ""


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: the model name string in full,
    with its family / model / stepping numbers (a virtualised host may give a
    short model name), or the platform's processor string."""
    fields: dict[str, str] = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block is enough
                key, _, val = line.partition(":")
                fields[key.strip()] = val.strip()
    except OSError:
        pass
    name = fields.get("model name")
    if not name:
        import platform

        return platform.processor() or "unknown"
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def capture_env(cmdline: str = "") -> EnvInfo:
    import torch

    env = EnvInfo(cmdline=cmdline, torch_version=torch.__version__,
                  hip_version=str(getattr(torch.version, "hip", "") or ""),
                  timestamp_utc=_dt.datetime.now(_dt.timezone.utc).isoformat())
    try:
        if torch.cuda.is_available():
            env.gpu_count = torch.cuda.device_count()
            props = torch.cuda.get_device_properties(0)
            env.gpu_name = props.name
            env.rocm_arch = getattr(props, "gcnArchName", "")
    except Exception:
        pass
    try:
        env.cpu_threads = len(os.sched_getaffinity(0))
    except AttributeError:
        env.cpu_threads = os.cpu_count() or 0
    env.cpu_model = cpu_model()
    env.git_commit = _git(["rev-parse", "HEAD"])
    env.git_dirty = bool(_git(["status", "--porcelain"]))
    return env
