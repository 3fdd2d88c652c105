"""Seeded random shapes through both attention paths (GPU, C-ABI).

Each case draws batch, heads (GQA ratio 1-3), sequence lengths (1-1500, Nq !=
Nkv for non-causal flash cases), head dim, causality, input dtype, P.V type,
Q granularity and layout, and in about a third of the cases scores that rise
from key block to key block (running-max moves and redone blocks).  The
draws are fixed by the seed, so a failure names a reproducible case.

INT8 path: against the exact emulation on the kernel's own q8/k8/scales with
the bound of test_gpu_attn.py (2e-3 + output rounding, plus 2^-9 * max|v|
for bf16 P), and cosine >= 0.999 against fp64 SDPA.  Flash path: against
fp64 SDPA with the flash_attn pack's gate (atol = rtol = 1e-2) and cosine
>= 0.9999; causal rows that see no key (Nq > Nkv is not drawn causal) do not
occur.
"""
from __future__ import annotations

import importlib.util
import random
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
OUT_EPS = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -10}
LOG2E = 1.4426950408889634


def _draw_qkv(rnd, g, B, Hq, Hkv, Nq, Nkv, D):
    q = torch.randn(B, Hq, Nq, D, generator=g)
    k = torch.randn(B, Hkv, Nkv, D, generator=g) + 2.0 * torch.randn(B, Hkv, 1, D, generator=g)
    v = torch.randn(B, Hkv, Nkv, D, generator=g)
    rising = rnd.random() < 0.3
    if rising:  # scores rise by about 2.5 log2 units per 64 keys
        u = torch.randn(D, generator=g)
        u /= u.norm()
        q = q + 4.0 * u
        k = k + 2.5 * (torch.arange(Nkv, dtype=torch.float32)[None, None, :, None] / 64) * D ** 0.5 / (4 * LOG2E) * u
    return q, k, v, rising


def _int8_cases(seed, n):
    rnd = random.Random(seed)
    out = []
    for i in range(n):
        D, Hkv, G, B = rnd.choice([64, 128]), rnd.choice([1, 2]), rnd.choice([1, 2, 3]), rnd.choice([1, 2])
        N, causal = rnd.randint(1, 1500), rnd.random() < 0.5
        pv, qg = rnd.choice(["fp16", "fp16", "bf16"]), rnd.choice(["block", "wave", "thread"])
        dt, lay = rnd.choice([torch.bfloat16, torch.float16]), rnd.choice(["HND", "NHD"])
        out.append((seed * 1000 + i, B, Hkv * G, Hkv, N, D, causal, pv, qg, dt, lay))
    return out


@pytest.mark.parametrize("case", _int8_cases(7, 12), ids=lambda c: f"int8-{c[0]}")
def test_int8_random_shapes(case, hip_impl, gpu_device):
    cid, B, Hq, Hkv, N, D, causal, pv, qg, dt, lay = case
    rnd, g = random.Random(cid), torch.Generator().manual_seed(cid)
    q, k, v, rising = _draw_qkv(rnd, g, B, Hq, Hkv, N, N, D)
    print(f"[int8-random {cid}] B{B} Hq{Hq} Hkv{Hkv} N{N} D{D} causal={causal} pv={pv} q={qg} {dt} {lay} "
          f"rising={rising}", flush=True)
    q, k, v = (t.to(dt) for t in (q, k, v))
    tq, tk, tv = (t.transpose(1, 2).contiguous() if lay == "NHD" else t for t in (q, k, v))
    o, pre = hip_impl.run(tq.to(gpu_device), tk.to(gpu_device), tv.to(gpu_device), causal=causal, pv_dtype=pv,
                          q_gran=qg, tensor_layout=lay, return_intermediates=True)
    torch.cuda.synchronize()
    o, q8, k8 = o.float().cpu(), pre["q8"].cpu(), pre["k8"].cpu()
    if lay == "NHD":
        o, q8, k8 = o.transpose(1, 2), q8.transpose(1, 2), k8.transpose(1, 2)
    got = o.numpy().astype(np.float64)
    assert np.isfinite(got).all()
    vf = v.float().numpy()
    emu = O.sage_emulate(q8.numpy(), pre["q_scale"].cpu().numpy(), k8.numpy(), pre["k_scale"].cpu().numpy(), vf,
                         causal=causal, q_sub=hip_impl.q_sub_of(qg))
    p_term = 2.0 ** -9 * float(np.abs(vf).max()) if pv == "bf16" else 0.0
    err = float((np.abs(got - emu) - OUT_EPS[dt] * np.abs(emu)).max()) - p_term
    want = O.sdpa(q.float().numpy(), k.float().numpy(), vf, causal=causal)
    cos = float((got * want).sum() / np.linalg.norm(got) / np.linalg.norm(want))
    print(f"  vs emulation {err:.2e}, cosine vs SDPA {cos:.6f}")
    assert err <= 2e-3 and cos >= 0.999


def _flash_module():
    name = "tribench.kernels.flash_attn.hip_impl"
    spec = importlib.util.spec_from_file_location(name, ROOT / "tribench_amd" / "kernels" / "flash_attn" /
                                                  "hip_impl.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _flash_cases(seed, n):
    rnd = random.Random(seed)
    out = []
    for i in range(n):
        D, Hkv, G, B = rnd.choice([64, 128]), rnd.choice([1, 2]), rnd.choice([1, 2, 3]), rnd.choice([1, 2])
        causal = rnd.random() < 0.5
        Nq = rnd.randint(1, 1500)
        Nkv = Nq if causal or rnd.random() < 0.6 else rnd.randint(1, 1500)
        dt = rnd.choice([torch.bfloat16, torch.float16])
        out.append((seed * 1000 + i, B, Hkv * G, Hkv, Nq, Nkv, D, causal, dt))
    return out


@pytest.mark.parametrize("case", _flash_cases(5, 12), ids=lambda c: f"flash-{c[0]}")
def test_flash_random_shapes(case, gpu_device):
    cid, B, Hq, Hkv, Nq, Nkv, D, causal, dt = case
    rnd, g = random.Random(cid), torch.Generator().manual_seed(cid)
    q, k, v, rising = _draw_qkv(rnd, g, B, Hq, Hkv, Nq, Nkv, D)
    print(f"[flash-random {cid}] B{B} Hq{Hq} Hkv{Hkv} Nq{Nq} Nkv{Nkv} D{D} causal={causal} {dt} rising={rising}",
          flush=True)
    q, k, v = (t.to(dt) for t in (q, k, v))
    o = _flash_module().run(q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), causal=causal)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy().astype(np.float64)
    want = O.sdpa(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal)
    cos = float((got * want).sum() / np.linalg.norm(got) / np.linalg.norm(want))
    print(f"  max_abs {np.abs(got - want).max():.2e}, cosine {cos:.7f}")
    assert np.allclose(got, want, atol=1e-2, rtol=1e-2) and cos >= 0.9999
