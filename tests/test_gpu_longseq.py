"""Long sequences, beyond the benchmark configurations, against the CPU oracle.

The largest benchmark configuration has N = 32768.  These cases go to
N = 131071 and 65537, ragged (not a multiple of the 64-key block):
- the K statistics then use 8192-token chunks (16 per head);
- a head has 2048 k-scale blocks;
- the attention sweeps up to 2048 key blocks per work-group.

Checks, as in test_gpu_fullsize.py:
1. the pre-pass outputs bit for bit against the oracle (per_block_int8,
   triton_impl.py:7-33, 35-82, and the K channel mean), as ``run`` returns
   them;
2. sampled query rows against the exact emulation of the same INT8 data,
   within 2e-3 + 2^-8 |emu| (the bf16 rounding of the output), the part
   beyond half an ulp of the bf16 output within 0.3 of that;
3. the north star's gate against the fp32 reference (reference.py:15-24) on
   the GPU: max-abs <= 2e-2 (rows >= 128 when causal) and cosine >= 0.999.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O
from parity_util import emulation_split, split_line

pytestmark = pytest.mark.gpu

CASES = [
    # D = 64: Q quantized in the pre-pass, GQA 2:1, non-causal, ragged tail
    ("n131071_d64_gqa", dict(batch_size=1, num_heads=4, num_kv_heads=2, seq_len=131071, head_dim=64,
                             k_offset_std=2.0), False),
    # D = 128: Q quantized in the attention prologue, causal, ragged tail
    ("n65537_d128_causal", dict(batch_size=1, num_heads=2, seq_len=65537, head_dim=128, k_offset_std=4.0), True),
]
SAMPLE = 128


@pytest.mark.parametrize("name,case,causal", CASES, ids=[c[0] for c in CASES])
def test_long_sequence(name, case, causal, pack_ref, hip_impl, gpu_device):
    print(f"[longseq] {name} {case} causal={causal}", flush=True)
    inp = pack_ref.make_inputs(case, "cpu", 0, torch.bfloat16)
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    o, inter = hip_impl.run(q, k, v, causal=causal, return_intermediates=True)
    torch.cuda.synchronize()
    got = {key: inter[key].cpu().numpy() for key in ("q8", "q_scale", "k8", "k_scale", "km")}
    qn, kn, vn = (inp[x].float().numpy() for x in ("q", "k", "v"))

    # 1. bit-exact pre-pass outputs, every kv head with its query heads
    for hk in range(Hkv):
        hs = slice(hk * G, (hk + 1) * G)
        want = O.prepass(qn[:, hs], kn[:, hk:hk + 1], vn[:, hk:hk + 1], smooth_k=True)
        for key in ("q8", "q_scale"):
            assert np.array_equal(got[key][:, hs], want[key]), f"{name} hk{hk}: {key}"
        for key in ("k8", "k_scale", "km"):
            assert np.array_equal(got[key][:, hk:hk + 1], want[key]), f"{name} hk{hk}: {key}"

    # 2. sampled rows of the first and last head against the exact emulation
    want_o = pack_ref.ref(q, k, v, causal=causal)
    for h in (0, Hq - 1):
        sp = emulation_split(o, want_o, got, vn, 0, h, G, causal=causal, q_sub=hip_impl.q_sub_of("block"),
                             sample=SAMPLE)
        print("  " + split_line(f"{name} h={h}", sp), flush=True)
        assert np.isfinite(sp["got"]).all() and (sp["err"] <= sp["bound"]).all(), f"{name} h{h}"
        assert sp["arith_ratio"] <= 0.3, f"{name} h{h}"

    # 3. the north star's gate against the fp32 reference
    of = o.float()
    diff = (of - want_o).abs()
    max_abs = float(diff[:, :, 128:].max() if causal else diff.max())
    cos = float(torch.nn.functional.cosine_similarity(of.flatten(), want_o.flatten(), dim=0))
    print(f"  vs fp32 reference: max_abs={max_abs:.3e}{' (rows >= 128)' if causal else ''} cos={cos:.6f}",
          flush=True)
    assert max_abs <= 2e-2 and cos >= 0.999, name
