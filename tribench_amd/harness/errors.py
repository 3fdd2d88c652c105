"""Hints for common failures (counterpart of tribench/errors.py:get_triton_hint)."""
from __future__ import annotations


def get_hint(e: Exception) -> str | None:
    """A human-readable hint for an exception text, or None."""
    msg = str(e).lower()
    if "out of bounds" in msg or "memory access" in msg or "illegal" in msg or "page fault" in msg:
        return "Possible out-of-bounds access. Check tensor shapes and strides against the kernel's assumptions."
    if "shape mismatch" in msg or "invalid configuration" in msg or "invalid argument" in msg or "invalid value" in msg:
        return "Shape mismatch or invalid configuration. Check grid/block sizes vs tensor shapes."
    if "invalid device function" in msg or "no kernel image" in msg:
        return "Kernel not compiled for this architecture (build for gfx950)."
    if "libsage_attn.so not found" in msg:
        return "Build the HIP library first: python -m tribench_amd.build"
    if "rocm gpu device" in msg:
        return "The HIP variant needs a ROCm device; pass --device cuda:0 on a GPU host."
    return None
