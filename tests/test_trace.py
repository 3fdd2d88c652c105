"""The phase-trace measurement build (include/sage_trace.h) on a host without a GPU.

* the product library does not export the trace entry point, the trace
  library (when built: ``python -m tribench_amd.build --trace``) exports it
  next to every entry point of include/sage_attn.h;
* ``trace_phases.analyse`` on a synthetic trace whose phases, barrier waits
  and clock are known.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from tribench_amd import trace_phases as tp

ROOT = Path(__file__).resolve().parents[1]


def _declared(header: str) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(sage_[a-z_0-9]+)\s*\(", text)))


def test_trace_header_declares_one_entry_point():
    assert _declared("sage_trace.h") == ["sage_trace_attach"]


def test_product_library_has_no_trace_entry_point():
    lib = ctypes.CDLL(str(tp.PRODUCT_LIB))
    assert not hasattr(lib, "sage_trace_attach")


@pytest.mark.skipif(not tp.TRACE_LIB.is_file(), reason="trace library not built (build --trace)")
def test_trace_library_exports_everything():
    lib = ctypes.CDLL(str(tp.TRACE_LIB))
    for name in _declared("sage_attn.h") + _declared("sage_trace.h"):
        assert hasattr(lib, name), name
    attach = lib.sage_trace_attach
    attach.argtypes, attach.restype = [ctypes.c_void_p, ctypes.c_int64], ctypes.c_int
    assert attach(None, 0) == 0  # detach needs no device
    buf = (ctypes.c_ulonglong * 4)()
    assert attach(ctypes.cast(buf, ctypes.c_void_p), 0) != 0  # a buffer with no words is an argument error


def test_analyse_synthetic_trace():
    grid, cus = 512, 256
    T = np.zeros((grid, tp.NW, tp.WORDS), dtype=np.uint64)
    for g in range(grid):
        gen, cu = divmod(g, cus)
        for w in range(tp.NW):
            base = 10_000_000 + gen * 250_000
            T[g, w, :6] = [base, base + 18_000, base + 21_000, base + 181_000, base + 193_000, base + 196_000]
            T[g, w, 6], T[g, w, 7] = 30_000, 25_000 if w < 4 else 5_000
            T[g, w, 8] = (60 << 32) | 66
            T[g, w, 9] = gen * 10_000          # 100 MHz: 100 us per generation
            T[g, w, 10] = gen * 10_000 + 9_800  # 98 us of wall time -> 196000 cycles: 2.0 GHz
            T[g, w, 11] = ((w % 4) << 4) | ((cu % 16) << 8) | (((cu // 16) % 2) << 12) | ((cu // 32) << 32)
            T[g, w, 13], T[g, w, 14] = base + 15_000, base + 16_000
    out = tp.analyse(T)
    assert "shader clock 2.000 GHz" in out
    assert "| prologue | 18000 | 9.2 % |" in out and "| mask-free loops | 160000 | 81.6 % |" in out
    assert "| mask-free loops: cycles per iteration | 2667 |" in out
    assert "entry to Q quantized (Q rows awaited) 15000" in out
    assert "the wave that issues ahead 3.1 %, the other 15.6 %" in out
    assert "gap between consecutive work-groups on one CU 2.00 us median (256 CUs seen)" in out


def test_dispatch_replay_by_hand():
    """In-order dispatch to engines in turn, one CU per engine: the long first
    work-group holds back the second round on every engine."""
    n = 8  # work-groups of XCD 0: blockIdx 0, 8, 16, ...
    T = np.zeros((8 * n, tp.NW, tp.WORDS), dtype=np.uint64)
    durs = [4, 1, 1, 1, 1, 1, 1, 1]
    for i, d in enumerate(durs):
        g = 8 * i
        T[g, :, 9], T[g, :, 10] = 0, d * 100
        T[g, :, 11] = (i % 4) << 13
    sim, meas, idle = tp.simulate_dispatch(T, xcd=0, cus_per_engine=1)
    assert abs(sim - 5.25) < 1e-9 and meas == 4.0 and abs(idle - 9.7 / 4) < 1e-9
