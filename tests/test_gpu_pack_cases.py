"""The sage_attn pack's own benchmark cases, through the INT8 path, as TriBench runs them.

``tribench test --kernel sage_attn`` (tribench/cli.py:315) runs the cases of
kernels/sage_attn/meta.json:29-44, s4k_d64 (B=8 H=16 N=4096 D=64) and
s8k_d64 (B=4 H=16 N=8192 D=64), by calling the implementation as
``run(q, k, v)`` (non-causal, no other keys) and gating the output against
reference.py:ref with atol = rtol = 5e-2 (meta.json:45-48).  Here, in fp16
and bf16:

1. the call exactly as the harness makes it, under the pack's gate
   (``check_correctness`` with the pack's tolerances), plus max-abs and
   cosine against the fp32 reference;
2. the same call returning its intermediates: the pre-pass outputs (Q8,
   q_scale, K8, k_scale, km) bit-exact against the CPU oracle in every
   (batch, kv head) slice, and the output identical to the plain call;
3. sampled rows of the first and last (batch, head) against the exact
   emulation of the same INT8 data, with the emulation's and the kernel's
   distance to the fp32 reference printed ([record]).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from parity_util import emulation_split, prepass_mismatches, split_line
from tribench_amd.harness.correctness import check_correctness
from tribench_amd.harness.types import CorrectnessSpec

pytestmark = pytest.mark.gpu

PACK = Path(__file__).resolve().parents[1] / "tribench_amd" / "kernels" / "sage_attn"
META = json.loads((PACK / "meta.json").read_text())
CASES = ["s4k_d64", "s8k_d64"]
PARAMS = [(c, d) for c in CASES for d in (torch.float16, torch.bfloat16)]


def _case(name):
    cases = {c["name"]: c for c in META["cases"]}
    return {k: v for k, v in cases[name].items() if k != "name"}


@pytest.mark.parametrize("name,dtype", PARAMS, ids=[f"{n}-{str(d)[6:]}" for n, d in PARAMS])
def test_pack_case_through_int8_path(name, dtype, pack_ref, hip_impl, gpu_device):
    case = _case(name)
    print(f"[pack case] {name} {dtype} {case}", flush=True)
    torch.manual_seed(0)
    inp = pack_ref.make_inputs(case, "cpu", 0, dtype)
    assert set(inp) == {"q", "k", "v", "causal"} and inp["causal"] is False
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    B, Hq, N, D = q.shape
    G = Hq // k.shape[1]

    # 1. as the harness calls it, under the pack's gate
    o = hip_impl.run(q, k, v)
    want_o = pack_ref.ref(q, k, v, causal=False)
    torch.cuda.synchronize()
    tol = META["correctness"]
    res = check_correctness(want_o, o, "fp16" if dtype == torch.float16 else "bf16",
                            CorrectnessSpec(atol=tol["atol"], rtol=tol["rtol"]))
    of = o.float()
    max_abs = float((of - want_o).abs().max())
    cos = float(torch.nn.functional.cosine_similarity(of.flatten(), want_o.flatten(), dim=0))
    print(f"  [record] {name} {dtype}: gate {'PASS' if res.passed else 'FAIL'} max_abs={max_abs:.3e} "
          f"cos={cos:.6f}", flush=True)
    assert res.passed, res.error_msg
    assert max_abs <= 2e-2 and cos >= 0.999

    # 2. the same call with its intermediates: bit-exact pre-pass, same output
    o2, inter = hip_impl.run(q, k, v, return_intermediates=True)
    torch.cuda.synchronize()
    assert torch.equal(o2, o)
    host = {key: inter[key].cpu().numpy() for key in ("q8", "q_scale", "k8", "k_scale", "km")}
    qn, kn, vn = (inp[x].float().numpy() for x in ("q", "k", "v"))
    errors = prepass_mismatches(host, qn, kn, vn, q_sub=hip_impl.q_sub_of("block"))
    assert not errors, "\n".join(errors[:8])

    # 3. sampled rows against the exact emulation, and the split of the distance to the fp32 reference
    for b, h in ((0, 0), (B - 1, Hq - 1)):
        sp = emulation_split(o, want_o, host, vn, b, h, G, causal=False, q_sub=hip_impl.q_sub_of("block"),
                             out_dtype="bf16" if dtype == torch.bfloat16 else "fp16")
        print("  " + split_line(f"{name} {dtype} (b={b}, h={h})", sp), flush=True)
        assert np.isfinite(sp["got"]).all() and (sp["err"] <= sp["bound"]).all()
        assert sp["arith_ratio"] <= 0.3
