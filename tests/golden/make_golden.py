"""Write the golden fixtures of the sage_attn path (tests/golden/*.npz).

The reference (H1yori233/TriBench kernels/sage_attn) ships no golden vectors
or known-answer tests.  These fixtures are produced by this repository's CPU
oracle (oracle/sage_oracle.py) from the pack's own seeded inputs and pin the
oracle and the HIP path against regressions:

  sage_cfg1.npz   BASELINE.json config 1: B=1, H=2, N=256, D=64, fp32,
                  non-causal, K channel offset N(0,2), seed 0.  Inputs, the
                  pre-pass outputs (Q8, q_scale, K8, k_scale, km) and the
                  outputs of fp64 SDPA and of the exact SageAttention
                  emulation, both causal and non-causal.
  sage_fp8v.npz   Student-t(3) V, B=1, H=2, N=200, D=64, bf16 values in fp32:
                  per-channel FP8 e4m3 codes and scales.

Usage: python tests/golden/make_golden.py   (from the repository root)
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import sage_oracle as O  # noqa: E402


def _pack_ref():
    spec = importlib.util.spec_from_file_location(
        "tribench.kernels.sage_attn.reference", ROOT / "tribench_amd/kernels/sage_attn/reference.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


CFG1 = dict(batch_size=1, num_heads=2, seq_len=256, head_dim=64, k_offset_std=2.0)
FP8V = dict(batch_size=1, num_heads=2, seq_len=200, head_dim=64, v_dist="student_t", v_df=3)


def cfg1_arrays() -> dict:
    R = _pack_ref()
    inp = R.make_inputs(CFG1, "cpu", 0, torch.float32)
    q, k, v = (inp[x].numpy() for x in ("q", "k", "v"))
    pre = O.prepass(q, k, smooth_k=True)
    out = dict(q=q, k=k, v=v, q8=pre["q8"], q_scale=pre["q_scale"], k8=pre["k8"], k_scale=pre["k_scale"],
               km=pre["km"])
    for causal in (False, True):
        tag = "causal" if causal else "full"
        out[f"o_sdpa_{tag}"] = O.sdpa(q, k, v, causal=causal).astype(np.float32)
        out[f"o_emul_{tag}"] = O.sage_emulate(pre["q8"], pre["q_scale"], pre["k8"], pre["k_scale"], v,
                                              causal=causal).astype(np.float32)
    return out


def fp8v_arrays() -> dict:
    R = _pack_ref()
    inp = R.make_inputs(FP8V, "cpu", 0, torch.bfloat16)
    v = inp["v"].float().numpy()
    v8, vs = O.quant_v_fp8(v)
    return dict(v=v, v8=v8, v_scale=vs)


def main() -> int:
    d = Path(__file__).resolve().parent
    np.savez_compressed(d / "sage_cfg1.npz", **cfg1_arrays())
    np.savez_compressed(d / "sage_fp8v.npz", **fp8v_arrays())
    for f in ("sage_cfg1.npz", "sage_fp8v.npz"):
        print(f, (d / f).stat().st_size, "bytes")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
