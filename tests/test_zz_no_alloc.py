"""sage_prepass_vt_noalloc (the pre-pass without a workspace argument: its
partial sums live in the library's fixed per-GPU scratch array) against
sage_prepass_vt with a caller workspace: every output bit for bit, on two
calls in a row, the second with a smaller input, through the C ABI."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, N, D, pv_dtype, q_gran): FP8 first (K sums and V maxima both
# in the scratch array), then a smaller fp16 problem that reuses it
CALLS = [
    (2, 8, 4, 3000, 128, "fp8", "wave"),
    (1, 4, 2, 777, 64, "fp16", "block"),
]
OUT_KEYS = ("q8", "q_scale", "k8", "k_scale", "km", "vt")


def _inputs(pack_ref, B, Hq, Hkv, N, D, pv, seed):
    case = dict(batch_size=B, num_heads=Hq, num_kv_heads=Hkv, seq_len=N, head_dim=D, k_offset_std=2.0,
                v_dist="student_t" if pv == "fp8" else "normal", v_df=3)
    return pack_ref.make_inputs(case, "cpu", seed, torch.bfloat16)


def test_noalloc_prepass_equals_workspace_entry_point(pack_ref, hip_impl, gpu_device):
    for i, (B, Hq, Hkv, N, D, pv, q_gran) in enumerate(CALLS):
        print(f"[noalloc] call {i}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} pv={pv} q_gran={q_gran}", flush=True)
        inp = _inputs(pack_ref, B, Hq, Hkv, N, D, pv, seed=i)
        q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
        kw = dict(q_sub=hip_impl.q_sub_of(q_gran), smooth_k=True, pv_dtype=pv)
        want = hip_impl.prepass(q, k, v, **kw)
        got = hip_impl.prepass(q, k, v, static_scratch=True, **kw)
        torch.cuda.synchronize()
        assert "workspace" not in got
        keys = OUT_KEYS + (("v_scale",) if pv == "fp8" else ())
        for key in keys:
            assert torch.equal(got[key], want[key]), f"call {i}: {key} differs"


def test_noalloc_prepass_rejects_problems_beyond_the_scratch(pack_ref, hip_impl, gpu_device):
    lib = hip_impl._load()
    B, Hkv, N, D = 16, 64, 4096, 128
    need = lib.sage_prepass_workspace_bytes(B, Hkv, N, D, 1, 0)
    assert need > 4 << 20
    q = torch.zeros((B, Hkv, N, D), dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(RuntimeError, match="invalid argument.*scratch"):
        hip_impl.prepass(q, q, q, pv_dtype="fp16", static_scratch=True)
