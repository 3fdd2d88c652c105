"""Phase split of the attention kernel, from the trace build (measurement only).

Runs one benchmark configuration through ``hip_impl.run`` with
``lib/libsage_attn_trace.so`` (``python -m tribench_amd.build --trace``: the
same sources with SAGE_TRACE=2, include/sage_trace.h), settles the clock
with untimed forwards, then traces one attention launch and prints, as
markdown:

* per work-group, in shader cycles (s_memtime, per wave, averaged over the
  8 waves): the prologue (Q load and quantization, tiles 0-2 requested, 0-1
  awaited, S of block 0), iteration 0, the mask-free loops, the generic
  iterations (masked blocks, the last three without prefetch, the final P.V),
  the epilogue, and the cycles each phase spends waiting at the
  per-iteration barrier;
* the barrier wait of the two waves of each SIMD in the mask-free loops
  (the wave that reaches the barrier first waits for the other);
* the work-groups' wall times (s_memrealtime, 100 MHz): the clock per wave,
  the gap between consecutive work-groups on one CU, the spread of the
  XCDs' end times.

The trace build keeps its stamps in LDS and its barrier counters in SGPRs;
its launch time is printed next to the product library's for the same
configuration (alternating launches), so the perturbation is visible.

  python -m tribench_amd.trace_phases [--case cfg2] [--settle-ms 300] [--dtype bf16]
"""
from __future__ import annotations

import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
PACK = PKG / "kernels" / "sage_attn"
TRACE_LIB = PKG / "lib" / "libsage_attn_trace.so"
PRODUCT_LIB = PKG / "lib" / "libsage_attn.so"
WORDS = 16  # per wave, include/sage_trace.h
NW = 8      # waves per work-group


def _load(stem: str, lib: Path):
    """The pack file ``stem`` under a module name of its own, bound to ``lib``
    (the library override variable is set only while it binds)."""
    name = f"tribench.kernels.sage_attn.{stem}.{lib.stem}"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PACK / f"{stem}.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    if hasattr(mod, "_load"):
        old = os.environ.get("TRIBENCH_SAGE_HIP_LIB")
        os.environ["TRIBENCH_SAGE_HIP_LIB"] = str(lib)
        try:
            mod._load()  # bind now, while the variable names this library
        finally:
            if old is None:
                del os.environ["TRIBENCH_SAGE_HIP_LIB"]
            else:
                os.environ["TRIBENCH_SAGE_HIP_LIB"] = old
    return mod


def _case(prefix: str) -> tuple[str, dict]:
    cases = json.loads((PACK / "meta.json").read_text())["cases"]
    for c in cases:
        if c["name"] == prefix or c["name"].startswith(prefix + "_"):
            return c["name"], {k: v for k, v in c.items() if k != "name"}
    raise SystemExit(f"no case {prefix!r} in {PACK / 'meta.json'}")


def simulate_dispatch(T: np.ndarray, xcd: int = 0, cus_per_engine: int = 8) -> tuple[float, float, float]:
    """The dispatch rule the traces show, replayed on one XCD's traced
    work-group lengths: work-groups start in order (blockIdx = 8 * local + xcd),
    local index i goes to shader engine engine[i mod 4], and each waits for a
    free CU in its engine (0.05 us to start).  Returns (simulated span,
    measured span, simulated idle time per CU), in us."""
    rt0 = T[:, :, 9].astype(np.int64).min(axis=1)
    rt1 = T[:, :, 10].astype(np.int64).max(axis=1)
    dur = (rt1 - rt0) / 100.0
    hw = (T[:, 0, 11] & 0xFFFFFFFF).astype(np.int64)
    engine_of = (hw >> 13) & 7
    idx = np.arange(xcd, T.shape[0], 8)  # this XCD's work-groups in dispatch order
    engine = [int(engine_of[idx[i]]) for i in range(min(4, len(idx)))]
    free = {e: [0.0] * cus_per_engine for e in set(engine)}
    t = idle = end = 0.0
    for i, g in enumerate(idx):
        f = free[engine[i % len(engine)]]
        c = int(np.argmin(f))
        start = max(t, f[c]) + 0.05
        idle += start - f[c]
        f[c] = start + dur[g]
        t, end = start, max(end, f[c])
    span = (rt1[idx].max() - rt0[idx].min()) / 100.0
    return end, float(span), idle / (len(free) * cus_per_engine)


def analyse(T: np.ndarray) -> str:
    """Markdown summary of a trace array [grid, 8, 16] (uint64)."""
    t = T[:, :, :6].astype(np.float64)
    ph = np.diff(t, axis=2)  # prologue, iteration 0, mask-free loops, generic, epilogue
    total = t[:, :, 5] - t[:, :, 0]
    rt0, rt1 = T[:, :, 9].astype(np.float64), T[:, :, 10].astype(np.float64)
    wait_all, wait_fast = T[:, :, 6].astype(np.float64), T[:, :, 7].astype(np.float64)
    n_all, n_fast = (T[:, :, 8] & 0xFFFFFFFF).astype(np.float64), (T[:, :, 8] >> 32).astype(np.float64)
    hw = T[:, :, 11] & 0xFFFFFFFF
    xcc = (T[:, :, 11] >> 32) & 0xF
    simd = (hw >> 4) & 3
    cu = (hw >> 8) & 0xF
    sh = (hw >> 12) & 1
    se = (hw >> 13) & 7
    grid = T.shape[0]
    clock = total / ((rt1 - rt0) / 100e6)  # Hz, per wave
    wg_cycles = total.mean(axis=1)
    names = ["prologue", "iteration 0", "mask-free loops", "generic iterations", "epilogue"]
    per = ph.mean(axis=(0, 1))
    out = [f"work-groups: {grid}; waves: {grid * NW}; mean cycles per work-group (per wave, s_memtime): "
           f"{wg_cycles.mean():.0f}; shader clock {np.median(clock) / 1e9:.3f} GHz (median over waves, "
           f"{np.percentile(clock, 5) / 1e9:.3f}-{np.percentile(clock, 95) / 1e9:.3f} for 90 %)", "",
           "| phase | cycles per wave | share |", "|---|---|---|"]
    for nm, v in zip(names, per):
        out.append(f"| {nm} | {v:.0f} | {100 * v / per.sum():.1f} % |")
    out.append(f"| total | {per.sum():.0f} | 100 % |")
    if (T[:, :, 13] > 0).all():  # the prologue's parts (Q quantized in the attention kernel)
        q_done = (T[:, :, 13].astype(np.float64) - t[:, :, 0]).mean()
        tiles = (T[:, :, 14].astype(np.float64) - T[:, :, 13].astype(np.float64)).mean()
        rest = (t[:, :, 1] - T[:, :, 14].astype(np.float64)).mean()
        out += ["", f"prologue parts (cycles per wave): entry to Q quantized (Q rows awaited) {q_done:.0f}, "
                f"then tiles 0-1 awaited {tiles:.0f}, then S of block 0 and the score grid {rest:.0f}"]
    gen_wait = wait_all - wait_fast
    out += ["", "| barrier | per wave | share of the phase |", "|---|---|---|",
            f"| mask-free loops: waits | {n_fast.mean():.1f} barriers, {wait_fast.mean():.0f} cycles | "
            f"{100 * wait_fast.mean() / max(per[2], 1):.1f} % |",
            f"| everywhere else: waits | {(n_all - n_fast).mean():.1f} barriers, {gen_wait.mean():.0f} cycles | "
            f"{100 * gen_wait.mean() / max(per.sum() - per[2], 1):.1f} % |"]
    if n_fast.mean() > 0:
        out.append(f"| mask-free loops: cycles per iteration | {per[2] / n_fast.mean():.0f} | |")
    # the two waves of each SIMD in a work-group: the one waiting less at the barrier issues first
    firsts, seconds = [], []
    for g in range(grid):
        for s in range(4):
            w = np.nonzero(simd[g] == s)[0]
            if len(w) != 2:
                continue
            f = wait_fast[g, w] / np.maximum(ph[g, w, 2], 1)
            firsts.append(f.min())
            seconds.append(f.max())
    if firsts:
        out += ["", f"two waves of a SIMD, share of the mask-free loops spent at the barrier: the wave that "
                f"issues ahead {100 * np.mean(firsts):.1f} %, the other {100 * np.mean(seconds):.1f} % "
                f"({len(firsts)} SIMD pairs)"]
    # wall time: gaps between consecutive work-groups on one CU, XCD end spread
    start, end = rt0.min(axis=1), rt1.max(axis=1)
    key = xcc[:, 0] * 4096 + se[:, 0] * 512 + sh[:, 0] * 64 + cu[:, 0]
    gaps = []
    for k in np.unique(key):
        idx = np.nonzero(key == k)[0]
        o = idx[np.argsort(start[idx])]
        gaps += list((start[o[1:]] - end[o[:-1]]) / 100.0)  # us
    gen = np.zeros(grid, dtype=np.int64)
    for k in np.unique(key):
        idx = np.nonzero(key == k)[0]
        gen[idx[np.argsort(start[idx])]] = np.arange(len(idx))
    if gen.max() > 0:
        rows = []
        for g in range(min(gen.max() + 1, 12)):
            sel = gen == g
            rows.append(f"{g}: {ph[sel, :, 0].mean():.0f}")
        out += ["", "prologue cycles per wave by the work-group's place on its CU (0 = first): " + ", ".join(rows)]
    span = (end.max() - start.min()) / 100.0
    xe = [end[xcc[:, 0] == x].max() for x in np.unique(xcc[:, 0])]
    out += ["", f"launch (s_memrealtime): {span:.1f} us from the first work-group's start to the last one's end; "
            f"work-group wall time {np.mean(end - start) / 100.0:.1f} us mean; gap between consecutive "
            f"work-groups on one CU {np.median(gaps) if gaps else float('nan'):.2f} us median "
            f"({len(np.unique(key))} CUs seen); XCD end times spread over {(max(xe) - min(xe)) / 100.0:.1f} us"]
    sim, meas, idle = simulate_dispatch(T)
    out += ["", f"XCD 0 replayed with in-order dispatch to its four shader engines in turn (from the traced "
            f"lengths): {sim:.1f} us against {meas:.1f} us measured, {idle:.1f} us idle per CU"]
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--case", default="cfg2", help="a case name of the sage_attn pack, or its cfgN prefix")
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "fp16"])
    ap.add_argument("--settle-ms", type=float, default=300.0)
    ap.add_argument("--compare", type=int, default=20, help="alternating timed launches of each library")
    ap.add_argument("--save", default=None, help="also write the raw trace [grid, 8, 16] to this .npy file")
    args = ap.parse_args(argv)
    import torch

    if not TRACE_LIB.is_file():
        raise SystemExit(f"{TRACE_LIB} not built: python -m tribench_amd.build --trace")
    name, case = _case(args.case)
    prod = _load("hip_impl", PRODUCT_LIB)
    trc = _load("hip_impl", TRACE_LIB)
    R = _load("reference", PRODUCT_LIB)
    dev = torch.device("cuda:0")
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    inp = R.make_inputs(case, "cpu", 0, dtype)
    q, k, v = (inp[x].to(dev) for x in ("q", "k", "v"))
    causal = inp["causal"]
    opts = {key: case[key] for key in ("pv_dtype", "q_gran") if key in case}
    B, Hq, N, D = q.shape
    grid = ((N + 255) // 256) * Hq * B
    buf = torch.zeros(grid * NW * WORDS, dtype=torch.int64, device=dev)
    attach = trc._load().sage_trace_attach
    attach.argtypes, attach.restype = [ctypes.c_void_p, ctypes.c_int64], ctypes.c_int

    def fwd(mod):
        return mod.run(q, k, v, causal=causal, **opts)

    # settle the clock, then alternate the two libraries with events around each forward
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.settle_ms:
        for _ in range(4):
            fwd(prod)
        torch.cuda.synchronize()
    ms = {"product": [], "trace": []}
    for _ in range(args.compare):
        for label, mod in (("product", prod), ("trace", trc)):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fwd(mod)
            e1.record()
            torch.cuda.synchronize()
            ms[label].append(e0.elapsed_time(e1))
    if attach(ctypes.c_void_p(buf.data_ptr()), buf.numel()) != 0:
        raise SystemExit("sage_trace_attach failed")
    fwd(trc)
    torch.cuda.synchronize()
    attach(None, 0)
    T = buf.cpu().numpy().view(np.uint64).reshape(grid, NW, WORDS)
    if not (T[:, :, 5] > 0).all():
        raise SystemExit("trace incomplete: some waves wrote no record")
    if args.save:
        np.save(args.save, T)
    print(f"### {name} ({args.dtype}, {'causal' if causal else 'non-causal'}, {opts or 'defaults'})\n")
    print(f"forward (pre-pass + attention), median of {args.compare} alternating: product "
          f"{np.median(ms['product']):.4f} ms, trace build {np.median(ms['trace']):.4f} ms\n")
    print(analyse(T))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
