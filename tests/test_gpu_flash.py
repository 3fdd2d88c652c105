"""GPU parity of the unquantized attention (flash_attn pack, C-ABI sage_flash_fwd).

1. Exactness: small-integer q and k (exact in fp16 / bf16; Q K^T exact in the
   fp32 MFMA accumulators), a score multiplier of exactly 1 (sm_scale =
   1/1.44269504) and integer v: every P is a power of two, exact in the P.V
   type, so the kernel must equal the exact base-2 emulation
   (oracle.sage_emulate with unit scales) up to fp32 accumulation.  This pins
   the fp16/bf16 QK operand layouts, masking, GQA and the V tile order.
2. Random inputs against fp64 SDPA with the reference pack's gate
   (kernels/flash_attn/meta.json: atol 1e-2, rtol 1e-2) and cosine >= 0.9999.
3. The reference pack's two cases at full size against the fp32 reference.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
ATOL = RTOL = 1e-2


def _flash_module(stem):
    name = f"tribench.kernels.flash_attn.{stem}"
    if name not in sys.modules:
        spec = importlib.util.spec_from_file_location(name, ROOT / "tribench_amd" / "kernels" / "flash_attn" /
                                                      f"{stem}.py")
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
    return sys.modules[name]


@pytest.fixture(scope="module")
def flash():
    return _flash_module("hip_impl")


@pytest.fixture(scope="module")
def flash_ref():
    return _flash_module("reference")


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_exact(dtype, D, causal, flash, gpu_device):
    B, Hq, Hkv, N = 2, 4, 2, 200  # GQA, four 64-key blocks, the last ragged
    print(f"[flash-exact] {dtype} D={D} causal={causal}", flush=True)
    g = np.random.default_rng(D + 2 * int(causal))
    qi = np.zeros((B, Hq, N, D), np.int8)
    ki = np.zeros((B, Hkv, N, D), np.int8)
    qi[..., :4] = g.integers(-1, 2, size=(B, Hq, N, 4))
    ki[..., :4] = g.integers(-1, 2, size=(B, Hkv, N, 4))
    vi = g.integers(-8, 9, size=(B, Hkv, N, D)).astype(np.float32)
    t = DT[dtype]
    q = torch.from_numpy(qi.astype(np.float32)).to(t).to(gpu_device)
    k = torch.from_numpy(ki.astype(np.float32)).to(t).to(gpu_device)
    v = torch.from_numpy(vi).to(t).to(gpu_device)
    sm_scale = 1.0 / 1.44269504
    assert np.float32(sm_scale * 1.44269504) == np.float32(1.0)
    o = flash.run(q, k, v, causal=causal, sm_scale=sm_scale)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy().astype(np.float64)
    nq, nk = -(-N // 128), -(-N // 64)
    emu = O.sage_emulate(qi, np.ones((B, Hq, nq)), ki, np.ones((B, Hkv, nk)), vi, causal=causal)
    # the output is rounded to the input type: 2^-11 (fp16) / 2^-8 (bf16) relative
    eps = 2.0 ** -11 if dtype == "fp16" else 2.0 ** -8
    err = np.abs(got - emu)
    print(f"  max |o - emu| = {err.max():.3e}")
    assert np.isfinite(got).all() and (err <= 1e-5 + eps * np.abs(emu)).all()


# (B, Hq, Hkv, Nq, Nkv, D, dtype, causal)
SMALL = [
    (1, 2, 2, 256, 256, 64, "fp16", False),
    (2, 4, 2, 300, 300, 128, "bf16", True),
    (1, 6, 1, 777, 777, 64, "bf16", True),
    (1, 3, 3, 1000, 1000, 128, "fp16", False),
    (1, 2, 1, 130, 700, 128, "bf16", False),
    (1, 2, 2, 1, 500, 64, "fp16", False),
    # D = 64: 10 and 18 mask-free iterations (one 10-block trip; one trip and
    # 8 single iterations)
    (1, 2, 2, 896, 896, 64, "fp16", False),
    (1, 2, 1, 1408, 1408, 64, "bf16", False),
]


@pytest.mark.parametrize("case", SMALL, ids=lambda c: f"B{c[0]}Hq{c[1]}Hkv{c[2]}Nq{c[3]}Nkv{c[4]}D{c[5]}-{c[6]}-c{int(c[7])}")
def test_flash_small_vs_sdpa(case, flash, gpu_device):
    B, Hq, Hkv, Nq, Nkv, D, dtype, causal = case
    print(f"[flash-small] {case}", flush=True)
    gen = torch.Generator().manual_seed(Nq + 3 * Nkv + D)
    q = torch.randn(B, Hq, Nq, D, generator=gen).to(DT[dtype])
    k = torch.randn(B, Hkv, Nkv, D, generator=gen).to(DT[dtype])
    v = torch.randn(B, Hkv, Nkv, D, generator=gen).to(DT[dtype])
    o = flash.run(q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), causal=causal)
    torch.cuda.synchronize()
    assert o.dtype == q.dtype and o.shape == q.shape
    got = o.float().cpu().numpy().astype(np.float64)
    want = O.sdpa(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal)
    cos = float((got * want).sum() / np.linalg.norm(got) / np.linalg.norm(want))
    print(f"  max_abs={np.abs(got - want).max():.3e} cos={cos:.7f}")
    assert np.allclose(got, want, atol=ATOL, rtol=RTOL) and cos >= 0.9999


@pytest.mark.parametrize("dtype,D,causal", [("fp16", 128, False), ("bf16", 64, True)])
def test_flash_rising_scores(dtype, D, causal, flash, gpu_device):
    """Scores rising by about 2.5 log2 units per 64-key block (the queries
    share a direction the keys drift along): the running max moves again and
    again, so the mask-free loop redoes blocks whose P exceed its shortcut's
    bound and rescales O lazily throughout; the reference pack's gate holds."""
    print(f"[flash-rising] {dtype} D={D} causal={causal}", flush=True)
    from test_gpu_attn import rising_inputs
    q, k, v = (t.to(DT[dtype]) for t in rising_inputs(1, 2, 1000, D, 2.5, seed=D))
    o = flash.run(q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), causal=causal)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy().astype(np.float64)
    want = O.sdpa(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal)
    cos = float((got * want).sum() / np.linalg.norm(got) / np.linalg.norm(want))
    print(f"  max_abs={np.abs(got - want).max():.3e} cos={cos:.7f}")
    assert np.allclose(got, want, atol=ATOL, rtol=RTOL) and cos >= 0.9999


def test_flash_nhd_matches_hnd(flash, gpu_device):
    gen = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(2, 4, 333, 64, generator=gen).to(torch.bfloat16).to(gpu_device) for _ in range(3))
    o1 = flash.run(q, k, v)
    o2 = flash.run(q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous(), v.transpose(1, 2).contiguous(),
                   tensor_layout="NHD")
    torch.cuda.synchronize()
    assert torch.equal(o1, o2.transpose(1, 2))


@pytest.mark.parametrize("name,case", [
    ("s4k_d64", dict(batch_size=8, num_heads=16, seq_len=4096, head_dim=64)),
    ("s8k_d64", dict(batch_size=4, num_heads=16, seq_len=8192, head_dim=64)),
])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_flash_pack_cases(name, case, dtype, flash, flash_ref, gpu_device):
    print(f"[flash-full] {name} {dtype}", flush=True)
    inp = flash_ref.make_inputs(case, "cpu", 0, DT[dtype])
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    o = flash.run(q, k, v, causal=inp["causal"])
    want = flash_ref.ref(q, k, v, causal=inp["causal"])
    torch.cuda.synchronize()
    of = o.float()
    cos = float(torch.nn.functional.cosine_similarity(of.flatten(), want.flatten(), dim=0))
    print(f"  max_abs={float((of - want).abs().max()):.3e} cos={cos:.7f}")
    assert torch.allclose(of, want, atol=ATOL, rtol=RTOL) and cos >= 0.9999
