"""Benchmark of the sage_attn hot path on one MI355X (driver contract).

One step = one SageAttention forward (HIP pre-pass + fused attention; Q is
quantized where hip_impl.run puts it, in the attention kernel's prologue at
D = 128, see --q-quant) over the
BASELINE.json configuration 2 workload with the inputs already resident in
HBM:  B=4, H=32, N=4096, D=128, bf16, non-causal, K channel offset ~N(0,2),
INT8 Q/K per block (BLKQ 128, BLKK 64), fp16 P.V, fp32 accumulation.

Prints one JSON line.  ``value`` is the headline metric of BASELINE.json,
effective TOPS = 4*B*H*N^2*D / t.  ``roofline`` is the attention kernel's
algorithmic rate (HIP events around its launches, on its stream) against the
MI355X dense INT8 MFMA peak; ``cpu_baseline`` times the CPU oracle's fp32
SDPA (a restatement of reference.py:ref) on a bounded sample of the same
workload on this host's cores.  The metric is quoted at N = 4096 and 16384:
after the headline configuration the same run times configuration 3 (B=2,
H=32, N=16384, causal) and reports it as the nested ``n16384`` object, with
its own step time, effective and algorithmic TOPS and roofline.  ``prepass``
gives the pre-pass's algorithmic bytes per second (K and V read once, K8 and
the V tiles written once; Q too where the pre-pass quantizes it) as a
fraction of the published 8 TB/s (``hbm_frac``) and of a plain 1 GiB device
copy timed on the same box first (``copy_gbps``, ``frac_of_copy``).

Before the W warmup steps of each configuration the step runs untimed for
``--settle-ms`` of wall time (default 200 ms, TriBench's own warmup time,
tribench/cli.py:47 and tribench/bench.py:119): the GPU's clock ramps up from
idle over the first ~25 steps of this workload (0.9-1.07 ms per attention
launch against 0.81 ms settled), so without it a short run times the ramp.
``--settle-ms 0`` gives the W-steps-only warmup; the JSON line reports the
settle steps run.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2] [--also cfg3|none]
                  [--no-cpu-baseline] [--copy-probe-gib G] [--q-quant auto|prologue|pre-pass]
                  [--settle-ms MS]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
PACK = ROOT / "tribench_amd" / "kernels" / "sage_attn"
INT8_PEAK_TOPS = 5000.0  # MI355X dense INT8 MFMA, 5.0 POP/s
HBM_PEAK_GBPS = 8000.0

CONFIGS = {
    # BASELINE.json configs (configs[0] is the CPU plumbing case)
    "cfg2": dict(batch_size=4, num_heads=32, seq_len=4096, head_dim=128, k_offset_std=2.0, pv_dtype="fp16",
                 desc="B=4 H=32 N=4096 D=128 bf16 non-causal, INT8 QK per block (128/64), fp16 P.V"),
    "cfg3": dict(batch_size=2, num_heads=32, seq_len=16384, head_dim=128, causal=True, k_offset_std=4.0,
                 pv_dtype="fp16", desc="B=2 H=32 N=16384 D=128 bf16 causal, INT8 QK, fp16 P.V"),
    "cfg4": dict(batch_size=2, num_heads=48, num_kv_heads=8, seq_len=17776, head_dim=64, k_offset_std=2.0,
                 pv_dtype="fp16", desc="B=2 Hq=48 Hkv=8 N=17776 D=64 bf16 non-causal GQA, INT8 QK, fp16 P.V"),
    "cfg5": dict(batch_size=1, num_heads=32, seq_len=32768, head_dim=128, causal=True, k_offset_std=2.0,
                 v_dist="student_t", v_df=3, pv_dtype="fp8", q_gran="wave",
                 desc="B=1 H=32 N=32768 D=128 bf16 causal, INT8 QK per-wave Q scales, FP8 P.V"),
}


def _load(stem: str):
    name = f"tribench.kernels.sage_attn.{stem}"
    spec = importlib.util.spec_from_file_location(name, PACK / f"{stem}.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _traffic_from_profiles(cfg: str):
    """HBM bytes per attention launch of a configuration and the file they
    come from: measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (copy-
    calibrated) in the committed summary of that configuration, not in this
    run; (None, None) if there is none."""
    rel = f"profiles/attn_fwd_{cfg}_hbm_traffic.md"
    f = ROOT / rel
    if not f.exists():
        return None, None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return (float(m.group(1)), rel) if m else (None, None)


def cpu_baseline(R, case, budget_s: float = 15.0) -> dict:
    """fp32 SDPA of the CPU oracle on whole (batch, head) slices of the
    workload, cycling through them until ``budget_s`` of wall time is spent;
    TOPS by the metric's formula on the slices done."""
    from oracle import sage_oracle as O
    from tribench_amd.harness.env import cpu_model

    threads = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_limits
        limiter = threadpool_limits(limits=threads)
    except Exception:  # pragma: no cover - threadpoolctl is optional
        limiter = None
    torch.set_num_threads(threads)
    inp = R.make_inputs(case, "cpu", 0, torch.bfloat16)
    q, k, v = (inp[x].float().numpy() for x in ("q", "k", "v"))
    B, Hq, N, D = q.shape
    G = Hq // k.shape[1]
    causal = bool(inp["causal"])
    heads = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s:  # cycle through the slices
        b, h = divmod(heads % (B * Hq), Hq)
        O.sdpa(q[b:b + 1, h:h + 1], k[b:b + 1, h // G:h // G + 1], v[b:b + 1, h // G:h // G + 1],
               causal=causal, dtype=np.float32)
        heads += 1
    dt = time.perf_counter() - t0
    if limiter is not None:
        limiter.unregister()
    ops = 4.0 * heads * N * N * D
    return {
        "value": ops / dt / 1e12, "unit": "TOPS", "cores": threads, "cpu_model": cpu_model(), "kind": "port",
        "sample": f"oracle.sdpa fp32 (numpy BLAS) on {heads} (batch, head) slices of the {B * Hq} "
                  f"(cycled), N={N} D={D}{' causal' if causal else ''}: {dt:.1f} s",
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS))
    ap.add_argument("--also", default="cfg3", choices=sorted(CONFIGS) + ["none"],
                    help="a second configuration timed in the same run and reported as a nested object "
                         "keyed by its sequence length (default cfg3: the metric's N = 16384 case)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--q-quant", default="auto", choices=["auto", "prologue", "pre-pass"],
                    help="where Q is quantized: as hip_impl.run does by default (auto), in the attention "
                         "kernel's prologue, or in the pre-pass")
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed steps for this much wall time before the warmup steps of each configuration "
                         "(the clock's ramp from idle; TriBench warms up for 200 ms by default)")
    ap.add_argument("--copy-probe-gib", type=float, default=0.0,
                    help="first run one plain device copy of this many GiB (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against a known byte count)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the sage_attn path shards over (batch, kv-head) with no communication, "
              "so the multi-GPU figure is N x the one-GPU figure by construction and is not measured.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1

    if args.copy_probe_gib > 0:
        n = int(args.copy_probe_gib * (1 << 30)) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    copy_gbps = copy_rate_gbps()
    R = _load("reference")
    H = _load("hip_impl")
    head = measure(R, H, args.config, args.steps, args.warmup, args.q_quant, args.settle_ms)
    _with_copy_rate(head, copy_gbps)
    case = CONFIGS[args.config]
    res = {
        "metric": "sage_attn effective TOPS (4*B*H*N^2*D/t)",
        "value": head["value"],
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": head["config"],
        **{key: head[key] for key in ("pct_int8_peak", "algo_tops", "algo_pct_int8_peak", "latency_ms", "settle",
                                       "prepass", "roofline")},
    }
    if args.also != "none" and args.also != args.config:
        # the metric's N = 16384 half: the same measurement on configuration 3
        other = measure(R, H, args.also, args.steps, args.warmup, args.q_quant, args.settle_ms)
        _with_copy_rate(other, copy_gbps)
        res[f"n{CONFIGS[args.also]['seq_len']}"] = other
    if not args.no_cpu_baseline:
        if str(ROOT) not in sys.path:
            sys.path.insert(0, str(ROOT))
        res["cpu_baseline"] = cpu_baseline(R, case, args.cpu_budget_s)
    print(json.dumps(res), flush=True)
    return 0


def copy_rate_gbps(gib: int = 1, reps: int = 5) -> float:
    """What a plain device-to-device copy moves on this box (read + written
    bytes per second, median of ``reps`` copies of ``gib`` GiB): the practical
    scale for the pre-pass's rate beside the published 8 TB/s."""
    n = gib << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    del src, dst
    torch.cuda.empty_cache()
    return 2.0 * n / (float(np.median(times)) * 1e-3) / 1e9


def _with_copy_rate(res: dict, copy_gbps: float) -> None:
    pre = res["prepass"]
    pre["copy_gbps"] = round(copy_gbps, 1)
    pre["frac_of_copy"] = round(pre["gbps"] / copy_gbps, 4)


def measure(R, H, name: str, steps: int, warmup: int, q_quant: str, settle_ms: float = 0.0) -> dict:
    """Untimed steps for ``settle_ms`` of wall time, ``warmup`` untimed and
    ``steps`` timed forwards of configuration ``name`` with its inputs
    resident in HBM: step time (one pair of events around all steps),
    effective TOPS (the metric) and algorithmic TOPS, p50/p95 of per-step
    events, the pre-pass's HBM rate, and the attention kernel's roofline from
    events around its launches on its stream."""
    case = CONFIGS[name]
    dev = torch.device("cuda:0")
    inp = R.make_inputs(case, "cpu", 0, torch.bfloat16)
    q, k, v = (inp[x].to(dev) for x in ("q", "k", "v"))
    del inp
    causal = bool(case.get("causal", False))
    pv = case.get("pv_dtype", "fp16")
    q_sub = H.q_sub_of(case.get("q_gran", "block"))
    B, Hq, N, D = q.shape
    est = R.estimate(case)
    metric_ops, algo_ops = float(est["flops"]), float(est["algo_flops"])

    out = torch.empty_like(q)
    stream = torch.cuda.current_stream(dev)
    fused_q = H.fuse_q_default(D) if q_quant == "auto" else q_quant == "prologue"

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        pre = H.prepass(q, k, v, q_sub=q_sub, smooth_k=True, pv_dtype=pv, quant_q=not fused_q)
        if ev is not None:
            ev[1].record(stream)
        if fused_q:
            H.attention_q(q, k, v, pre, causal, pv_dtype=pv, q_sub=q_sub, out=out)
        else:
            H.attention(q, k, v, pre, causal, pv_dtype=pv, q_sub=q_sub, out=out)
        if ev is not None:
            ev[2].record(stream)

    # the clock's ramp from idle: steps in groups of 4, the host kept within a
    # group of the GPU, until settle_ms of wall time have passed
    torch.cuda.synchronize()
    n_settle, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(4):
            step()
        n_settle += 4
        torch.cuda.synchronize()
    settle_wall_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(steps):
        step(evs[i])
    t_end.record(stream)
    torch.cuda.synchronize()
    ms = t_start.elapsed_time(t_end) / steps
    pre_ms = np.array([e[0].elapsed_time(e[1]) for e in evs])
    attn_ms = np.array([e[1].elapsed_time(e[2]) for e in evs])
    step_ms = np.array([e[0].elapsed_time(e[2]) for e in evs])
    del q, k, v, out
    torch.cuda.empty_cache()

    value = metric_ops / (ms * 1e-3) / 1e12
    traffic, traffic_src = _traffic_from_profiles(name)
    # Q (unless the attention kernel quantizes it) and K quantization + V tiles
    pre_bytes = est["prepass_bytes_k" if fused_q else "prepass_bytes"] + est["vtile_bytes"]
    pre_gbps = pre_bytes / (float(pre_ms.mean()) * 1e-3) / 1e9
    achieved = algo_ops / (float(attn_ms.mean()) * 1e-3) / 1e12
    return {
        "config": {"workload": f"{name}: {case['desc']}", "batch": B, "heads": Hq, "kv_heads": int(case.get(
                   "num_kv_heads", Hq)), "seq_len": N, "head_dim": D, "causal": causal, "pv_dtype": pv,
                   "q_gran": case.get("q_gran", "block"), "smooth_k": True,
                   "q_quant": "attention prologue" if fused_q else "pre-pass"},
        "value": round(value, 2),
        "ms_per_step": round(ms, 4),
        "pct_int8_peak": round(100.0 * value / INT8_PEAK_TOPS, 2),
        "algo_tops": round(algo_ops / (ms * 1e-3) / 1e12, 2),
        "algo_pct_int8_peak": round(100.0 * algo_ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 2),
        **({"note": "causal: value and pct_int8_peak follow the metric's 4*B*H*N^2*D, which counts the "
                    "masked pairs; algo_tops and algo_pct_int8_peak count the unmasked pairs only"}
           if causal else {}),
        "latency_ms": {"p50": round(float(np.percentile(step_ms, 50)), 4),
                       "p95": round(float(np.percentile(step_ms, 95)), 4)},
        "settle": {"ms": round(settle_wall_ms, 1), "steps": n_settle},
        "prepass": {"ms": round(float(pre_ms.mean()), 4), "bytes": pre_bytes, "gbps": round(pre_gbps, 1),
                    "hbm_frac": round(pre_gbps / HBM_PEAK_GBPS, 4)},
        "roofline": {"kernel": "attn_fwd_kernel", "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s", "frac": round(achieved / INT8_PEAK_TOPS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "launch_ms": round(float(attn_ms.mean()), 4), "algo_ops_per_launch": algo_ops},
    }


if __name__ == "__main__":
    raise SystemExit(main())
