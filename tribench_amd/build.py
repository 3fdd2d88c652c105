"""Build the gfx950 C-ABI library ``tribench_amd/lib/libsage_attn.so``.

Every ``csrc/*.hip`` translation unit is compiled with ``hipcc
--offload-arch=gfx950`` and linked into one shared library.  Builds in-tree
(the ``.so`` travels with the source tree) and always recompiles.

Usage: ``python -m tribench_amd.build [-j N] [--peak] [--trace]``.
``--peak`` also builds the roofline measurement programs of
``tribench_amd/peak`` (MFMA and HBM peaks); ``--trace`` also builds
``lib/libsage_attn_trace.so``, the same sources with the attention kernel's
phase trace compiled in (SAGE_TRACE=2, include/sage_trace.h), for
``tribench_amd/trace_phases.py``.  The library and the device checks the GPU
tests run are always built.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libsage_attn.so"
TRACE_LIB = LIBDIR / "libsage_attn_trace.so"
ARCH = "gfx950"

# Common flags.  Packed-FP32 instructions are disabled for all device code.
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]
# Per-unit flags.  The pre-pass must round exactly like the reference, so no
# contraction of multiplies and adds into FMAs there.
UNIT_FLAGS = {
    "sage_prepass.hip": ["-ffp-contract=off"],
    # LLVM's max-ilp machine-scheduler strategy for the attention kernels:
    # measured faster than the default at every configuration (A/B, one box:
    # config 2 +1.0 %, config 3 +1.2 %, config 4 +0.3 %, config 5 +2.2 %)
    "sage_attn_fwd.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "sage_abi.hip": [],
    "sage_vtiles.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")
    return exe


def _compile(src: Path, obj: Path, extra: tuple[str, ...] = ()) -> None:
    cmd = [hipcc(), *COMMON, *UNIT_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns about the device-only target feature; drop that noise
    noise = ("packed-fp32-ops", "not a recognized feature")
    msgs = [ln for ln in res.stderr.splitlines() if ln.strip() and not any(x in ln for x in noise)]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)


def _build_lib(out: Path, objdir: Path, jobs: int | None, extra: tuple[str, ...] = ()) -> Path:
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_compile, s, o, extra) for s, o in zip(srcs, objs)]:
            f.result()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(jobs: int | None = None, verbose: bool = True, peak: bool = False, trace: bool = False) -> Path:
    """Compile every HIP unit for gfx950 and link ``libsage_attn.so``, then
    the device checks of ``tests/native`` (and, with ``peak``, the roofline
    measurement programs; with ``trace``, the phase-trace library)."""
    _build_lib(LIB, PKG / "_build", jobs)
    if verbose:
        print(f"built {LIB}")
    build_checks(verbose)
    if peak:
        build_peak(verbose)
    if trace:
        _build_lib(TRACE_LIB, PKG / "_build" / "trace", jobs, ("-DSAGE_TRACE=2",))
        if verbose:
            print(f"built {TRACE_LIB}")
    return LIB


# Roofline measurement programs (tribench_amd/peak/*.hip ->
# tribench_amd/lib/<stem>): mfma_peak measures the dense MFMA peaks the
# roofline figures divide by, hbm_peak what streaming kernels move through
# HBM.  The device checks of tests/native/*.hip (run by the GPU tests) are
# built the same way, with the pre-pass's floating-point flags.
PEAK_DIR = PKG / "peak"
CHECK_DIR = PKG.parent / "tests" / "native"


def build_checks(verbose: bool = True) -> list[Path]:
    """The device checks the GPU tests run (``tests/native/*.hip``)."""
    return _build_exes([(s, ["-ffp-contract=off"]) for s in sorted(CHECK_DIR.glob("*.hip"))], verbose)


def build_peak(verbose: bool = True) -> list[Path]:
    """The roofline measurement programs (``tribench_amd/peak/*.hip``)."""
    return _build_exes([(s, []) for s in sorted(PEAK_DIR.glob("*.hip"))], verbose)


def _build_exes(srcs: list[tuple[Path, list[str]]], verbose: bool) -> list[Path]:
    LIBDIR.mkdir(exist_ok=True)
    exes = []
    for src, extra in srcs:
        exe = LIBDIR / src.stem
        tmp = exe.with_name(exe.name + ".tmp")
        cmd = [hipcc(), *COMMON, *extra, str(src), "-o", str(tmp)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
        os.replace(tmp, exe)
        exes.append(exe)
        if verbose:
            print(f"built {exe}")
    return exes


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("-j", "--jobs", type=int, default=None)
    p.add_argument("--peak", action="store_true", help="also build the roofline measurement programs")
    p.add_argument("--trace", action="store_true", help="also build the phase-trace library")
    args = p.parse_args(argv)
    build(args.jobs, peak=args.peak, trace=args.trace)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
