"""GPU parity of the P.V variants of the fused attention, FP8 e4m3 in particular.

1. Exactness (every P.V mode): integer scores with unit scales make every
   probability an exact power of two and the V values are exact in fp16,
   bf16 and e4m3, so the kernel must equal the exact-arithmetic emulation
   (oracle.sage_emulate) up to fp32 accumulation rounding.  This pins the
   operand layouts, the V transposition, the key order in LDS, masking, GQA
   and the per-channel V scales of each mode with no quantization noise.

2. FP8 P.V accuracy (config 5's path): P is rounded to e4m3 (relative error
   up to 2^-4, rms about 2.6 %) and V is per-channel e4m3.  The north star's
   cosine gate (>= 0.999 against fp32 SDPA) applies; its max-abs 2e-2 gate is
   not attainable by FP8 V itself on heavy-tailed V (a single e4m3 rounding of
   a Student-t value of 20 is off by up to 0.6), so the max-abs bound here is
   against the emulation of the same FP8 V with exact P, relative to the
   row's scale: |o - emu| <= 2^-4 * max|v| over the keys the row sees, which
   bounds sum_i p_i * delta_i * v_i / sum_i p_i for |delta_i| <= 2^-4.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu


def _exact_case(B, Hq, Hkv, N, D, seed):
    """Sparse int8 Q/K (4 channels in {-1,0,1}): scores are integers in [-4, 4]."""
    g = np.random.default_rng(seed)
    q8 = np.zeros((B, Hq, N, D), np.int8)
    k8 = np.zeros((B, Hkv, N, D), np.int8)
    q8[..., :4] = g.integers(-1, 2, size=(B, Hq, N, 4))
    k8[..., :4] = g.integers(-1, 2, size=(B, Hkv, N, 4))
    vint = g.integers(-8, 9, size=(B, Hkv, N, D)).astype(np.float32)
    return q8, k8, vint


@pytest.mark.parametrize("pv", ["fp16", "bf16", "fp8"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_pv_modes_exact(pv, D, causal, hip_impl, gpu_device):
    B, Hq, Hkv, N = 2, 4, 2, 200  # GQA, four 64-key blocks, the last ragged
    print(f"[pv-exact] pv={pv} D={D} causal={causal}", flush=True)
    q8, k8, vint = _exact_case(B, Hq, Hkv, N, D, seed=D + int(causal))
    q_sub = hip_impl.WAVE_ROWS
    nqs = -(-N // 128) * (128 // q_sub)
    pre = {
        "q8": torch.from_numpy(q8).to(gpu_device),
        "k8": torch.from_numpy(k8).to(gpu_device),
        "q_scale": torch.ones((B, Hq, nqs), dtype=torch.float32, device=gpu_device),
        "k_scale": torch.ones((B, Hkv, -(-N // 64)), dtype=torch.float32, device=gpu_device),
    }
    q = torch.zeros((B, Hq, N, D), dtype=torch.float32, device=gpu_device)
    k = torch.zeros((B, Hkv, N, D), dtype=torch.float32, device=gpu_device)
    if pv == "fp8":
        # v = codes' values times power-of-two channel scales: the V tiles hold exactly these codes
        codes = O.e4m3_encode(vint)
        assert np.array_equal(O.e4m3_decode(codes), vint)
        vs = (2.0 ** (np.arange(D) % 3 - 1)).astype(np.float32)
        v_scale = np.broadcast_to(vs, (B, Hkv, D)).copy()
        pre["v_scale"] = torch.from_numpy(v_scale).to(gpu_device)
        v = torch.from_numpy(vint * vs).to(gpu_device)
        emu = O.sage_emulate(q8, np.ones((B, Hq, nqs)), k8, np.ones((B, Hkv, -(-N // 64))), codes,
                             causal=causal, q_sub=q_sub, v_scale=v_scale)
    else:
        v = torch.from_numpy(vint).to(gpu_device)
        emu = O.sage_emulate(q8, np.ones((B, Hq, nqs)), k8, np.ones((B, Hkv, -(-N // 64))), vint,
                             causal=causal, q_sub=q_sub)
    o = hip_impl.attention(q, k, v, pre, causal, pv_dtype=pv, q_sub=q_sub)
    torch.cuda.synchronize()
    got = o.cpu().numpy().astype(np.float64)
    err = np.abs(got - emu)
    tol = 1e-5 * (1.0 + np.abs(emu))
    print(f"  max |o - emu| = {err.max():.3e}")
    assert np.isfinite(got).all() and (err <= tol).all()


def _row_vmax(v, Hq, causal):
    """max |v| over the keys each query row sees, per (b, h, row), for GQA-expanded v."""
    a = np.abs(v).max(axis=-1)  # [B, Hkv, N]
    if causal:
        a = np.maximum.accumulate(a, axis=-1)
    else:
        a = np.broadcast_to(a.max(axis=-1, keepdims=True), a.shape)
    return np.repeat(a, Hq // v.shape[1], axis=1)


FP8_SMALL = [
    # (B, Hq, Hkv, N, D, causal)
    (1, 2, 1, 1000, 128, True),
    (1, 4, 2, 777, 64, False),
    (2, 2, 2, 333, 128, False),
]


@pytest.mark.parametrize("case", FP8_SMALL, ids=lambda c: f"B{c[0]}Hq{c[1]}Hkv{c[2]}N{c[3]}D{c[4]}c{int(c[5])}")
def test_fp8_pv_small(case, pack_ref, hip_impl, gpu_device):
    B, Hq, Hkv, N, D, causal = case
    print(f"[pv-fp8] {case}", flush=True)
    inp = pack_ref.make_inputs(dict(batch_size=B, num_heads=Hq, num_kv_heads=Hkv, seq_len=N, head_dim=D,
                                    k_offset_std=2.0, v_dist="student_t", v_df=3), "cpu", 0, torch.bfloat16)
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    o, pre = hip_impl.run(q, k, v, causal=causal, pv_dtype="fp8", q_gran="wave", return_intermediates=True)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    v8, vsc = O.quant_v_fp8(inp["v"].float().numpy())
    assert np.array_equal(pre["v_scale"].cpu().numpy(), vsc)  # the pre-pass's per-channel scales, bit-exact
    emu = O.sage_emulate(pre["q8"].cpu().numpy(), pre["q_scale"].cpu().numpy(), pre["k8"].cpu().numpy(),
                         pre["k_scale"].cpu().numpy(), v8, causal=causal, q_sub=hip_impl.WAVE_ROWS, v_scale=vsc)
    want = O.sdpa(inp["q"].float().numpy(), inp["k"].float().numpy(), inp["v"].float().numpy(), causal=causal)
    vdec = O.e4m3_decode(v8) * vsc[:, :, None, :]
    bound = 2.0 ** -4 * _row_vmax(vdec, Hq, causal)[..., None] + 2.0 ** -8 * np.abs(emu)
    e = np.abs(got - emu)
    cos_e = float((got * emu).sum() / np.linalg.norm(got) / np.linalg.norm(emu))
    cos = float((got * want).sum() / np.linalg.norm(got) / np.linalg.norm(want))
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    print(f"  vs emulation: max_abs={e.max():.3e} (worst e/bound {(e / bound).max():.3f}) cos={cos_e:.6f}")
    print(f"  vs fp64 SDPA: max_abs={np.abs(got - want).max():.3e} cos={cos:.6f} rel_l2={rel:.4f}")
    assert (e <= bound).all()
    assert cos_e >= 0.999 and cos >= 0.999


def test_fp8_pv_config5(pack_ref, hip_impl, gpu_device):
    """Config 5 at full size against the fp32 reference (cosine gate)."""
    case = dict(batch_size=1, num_heads=32, seq_len=32768, head_dim=128, causal=True, k_offset_std=2.0,
                v_dist="student_t", v_df=3)
    print(f"[pv-fp8-cfg5] {case}", flush=True)
    inp = pack_ref.make_inputs(case, "cpu", 0, torch.bfloat16)
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    o = hip_impl.run(q, k, v, causal=True, pv_dtype="fp8", q_gran="wave")
    want = pack_ref.ref(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    of = o.float()
    cos = float(torch.nn.functional.cosine_similarity(of.flatten(), want.flatten(), dim=0))
    rel = float((of - want).norm() / want.norm())
    print(f"  cos={cos:.6f} rel_l2={rel:.4f} max_abs={float((of - want).abs().max()):.3e}")
    assert cos >= 0.999
