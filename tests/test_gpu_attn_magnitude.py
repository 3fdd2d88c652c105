"""Attention on inputs of growing magnitude against the exact emulation.

Multiplying Q and K by a factor multiplies their block scales, so the INT8
score scale c = q_scale * k_scale grows with its square (about 1.8e-4 at
unit-variance inputs, 0.16 at 30 times that, 2e-8 at a hundredth).  The kernel forms every score as
one FMA on the accumulator read as kMagicF + S, minus a bias kMagicF * c + m.
Rounding that bias would shift each block's scores by up to 0.75 c log2 units,
differently from block to block, and at c of 1e-2 and above the output would
leave the emulation bound (three to ten times over at 10x and 30x inputs).
The kernel keeps that bias exact (c trimmed to 21 bits, the running max on a
grid of at most 1 log2 unit), which covers c up to about 0.16: from 0.01x to
30x inputs the bounds hold, fp16 and bf16 P with those of test_gpu_attn.py
(the emulation consumes V as the P.V MFMAs do, rounded to bf16 for bf16 P),
FP8 P with that of test_gpu_attn_pv.py, Q quantized in the attention prologue
and in the pre-pass, D 64 and 128, causal and not.  At 100x (c near 2, one
INT8 score unit a factor of 4 in weight) the bias is within an ulp of
kMagicF * c, about one score unit, and the outputs are held to a cosine
against the emulation: 0.9999 for 16-bit P, 0.999 (the north star's gate)
for FP8 P.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O
from test_gpu_attn import DT, EMUL_ABS, _vs_emulation

pytestmark = pytest.mark.gpu

SCALES = [0.01, 1, 3, 10, 30, 100]
EXACT_UP_TO = 30  # scales whose c stays within the grid's exact range
# (name, B, Hq, Hkv, N, D, dtype, causal, pv, q_gran, fuse_q)
CASES = [
    ("d128_fusedq", 1, 2, 2, 2048, 128, "bf16", False, "fp16", "block", True),
    ("d128_prepassq_causal", 1, 2, 2, 1500, 128, "bf16", True, "fp16", "block", False),
    ("d64_gqa_causal", 1, 4, 2, 1777, 64, "bf16", True, "fp16", "block", None),
    ("d128_bf16p_thread", 1, 2, 1, 1300, 128, "fp16", False, "bf16", "thread", None),
    ("d128_fp8p_wave_causal", 1, 2, 2, 2048, 128, "bf16", True, "fp8", "wave", None),
]


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_attn_vs_emulation_at_magnitude(case, scale, pack_ref, hip_impl, gpu_device):
    name, B, Hq, Hkv, N, D, dtype, causal, pv, q_gran, fuse_q = case
    print(f"[magnitude] {name} x{scale}", flush=True)
    inp = pack_ref.make_inputs(dict(batch_size=B, num_heads=Hq, num_kv_heads=Hkv, seq_len=N, head_dim=D),
                               "cpu", SCALES.index(scale), torch.float32)
    q = (inp["q"] * scale).to(DT[dtype]).to(gpu_device)
    k = (inp["k"] * scale).to(DT[dtype]).to(gpu_device)
    v = inp["v"].to(DT[dtype]).to(gpu_device)
    o, pre = hip_impl.run(q, k, v, causal=causal, pv_dtype=pv, q_gran=q_gran, fuse_q=fuse_q,
                          return_intermediates=True)
    torch.cuda.synchronize()
    q8, qs = pre["q8"].cpu().numpy(), pre["q_scale"].cpu().numpy()
    k8, ks = pre["k8"].cpu().numpy(), pre["k_scale"].cpu().numpy()
    rows = np.unique(np.concatenate([np.arange(0, min(N, 96)), np.arange(0, N, 7), np.arange(max(0, N - 64), N)]))
    q_sub = hip_impl.q_sub_of(q_gran)
    if pv == "fp8":
        codes, vsc = O.quant_v_fp8(v.float().cpu().numpy())
        assert np.array_equal(pre["v_scale"].cpu().numpy(), vsc)  # the pre-pass's scales, bit-exact
        emu = O.sage_emulate(q8, qs, k8, ks, codes, causal=causal, q_sub=q_sub, v_scale=vsc, rows=rows)
    else:
        # the V the P.V MFMAs consume: converted to the P.V type (bf16 here rounds fp16 V)
        vv = v.to(torch.bfloat16 if pv == "bf16" else torch.float16).float().cpu().numpy()
        emu = O.sage_emulate(q8, qs, k8, ks, vv, causal=causal, q_sub=q_sub, rows=rows)
    got = o.float().cpu().numpy()[:, :, rows].astype(np.float64)
    assert np.isfinite(got).all()
    c_max = float(qs.max() * ks.max())
    cos = float((got * emu).sum() / np.linalg.norm(got) / np.linalg.norm(emu))
    print(f"  cos vs emulation {cos:.6f}, max|o-emu| {np.abs(got - emu).max():.3e}", flush=True)
    if pv == "fp8":
        G = Hq // Hkv
        worst = 0.0
        for h in range(Hq):
            vdec = O.e4m3_decode(codes[0, h // G]).astype(np.float64) * vsc[0, h // G][None, :]
            vmax = np.abs(vdec).max(axis=-1)
            row_vmax = np.maximum.accumulate(vmax)[rows] if causal else np.full(len(rows), vmax.max())
            bound = 2.0 ** -4 * row_vmax[:, None] + 2.0 ** -8 * np.abs(emu[0, h])
            worst = max(worst, float((np.abs(got[0, h] - emu[0, h]) / bound).max()))
        print(f"  c_max={c_max:.2e} worst e/bound={worst:.3f}", flush=True)
        if scale <= EXACT_UP_TO:
            assert worst <= 1.0
        else:
            assert cos >= 0.999
    else:
        excess = _vs_emulation(got, emu, DT[dtype], pv, v.float().cpu().numpy())
        print(f"  c_max={c_max:.2e} max(|o-emu| - eps|emu|)={excess:.3e} (bound {EMUL_ABS})", flush=True)
        if scale <= EXACT_UP_TO:
            assert excess <= EMUL_ABS
        else:
            assert cos >= 0.9999
