"""GPU parity of the HIP pre-pass against the CPU oracle: bit-exact.

INT8 Q/K, the fp32 block scales, the K channel mean and FP8 V must equal the
oracle's values bit for bit (the reference's quantization,
triton_impl.py:7-82, restated in oracle/sage_oracle.py).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}

# (B, Hq, Hkv, N, D, dtype, q_sub, smooth_k, v_fp8, k_offset_std, v_dist)
CASES = [
    (1, 2, 2, 256, 64, "fp32", 128, True, False, 2.0, "normal"),      # config 1 shape
    (1, 2, 2, 256, 64, "fp32", 128, False, False, 2.0, "normal"),     # reference semantics (no smoothing)
    (2, 4, 2, 300, 128, "bf16", 128, True, False, 2.0, "normal"),     # ragged tail, GQA
    (1, 3, 3, 1000, 64, "fp16", 32, True, False, 4.0, "normal"),      # per-wave Q scales
    (2, 6, 1, 777, 128, "bf16", 32, True, True, 2.0, "student_t"),    # FP8 V, GQA 6:1
    (1, 4, 4, 4096, 128, "bf16", 128, True, False, 2.0, "normal"),    # 16 K-stat chunks
    (1, 2, 2, 17776, 64, "bf16", 128, True, True, 2.0, "normal"),     # config-4 length, 14 chunks
    (2, 4, 2, 300, 128, "bf16", 1, True, False, 2.0, "normal"),       # per-row Q scales, ragged
    (1, 3, 3, 1000, 64, "fp16", 1, True, False, 4.0, "student_t"),    # per-row Q scales, D=64
]


def _ids(c):
    return f"B{c[0]}Hq{c[1]}Hkv{c[2]}N{c[3]}D{c[4]}-{c[5]}-qsub{c[6]}-smooth{int(c[7])}-fp8v{int(c[8])}"


def _inputs(pack_ref, B, Hq, Hkv, N, D, dtype, off, vdist, seed=0):
    case = dict(batch_size=B, num_heads=Hq, num_kv_heads=Hkv, seq_len=N, head_dim=D,
                k_offset_std=off, v_dist=vdist, v_df=3)
    return pack_ref.make_inputs(case, "cpu", seed, DT[dtype])


def _np32(t):
    return t.float().cpu().numpy()


def _eq_bits(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype == np.float32:
        # identical values; +0.0 and -0.0 count as equal
        return bool(np.array_equal(a, b))
    return bool(np.array_equal(a, b))


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_prepass_bitexact(case, pack_ref, hip_impl, gpu_device):
    B, Hq, Hkv, N, D, dtype, q_sub, smooth, vfp8, off, vdist = case
    print(f"[prepass] {_ids(case)}", flush=True)
    inp = _inputs(pack_ref, B, Hq, Hkv, N, D, dtype, off, vdist)
    want = O.prepass(_np32(inp["q"]), _np32(inp["k"]), _np32(inp["v"]), q_sub=q_sub, smooth_k=smooth,
                     v_fp8=vfp8)
    got = hip_impl.prepass(inp["q"].to(gpu_device), inp["k"].to(gpu_device), inp["v"].to(gpu_device),
                           q_sub=q_sub, smooth_k=smooth, v_fp8=vfp8)
    torch.cuda.synchronize()
    keys = ["q8", "q_scale", "k8", "k_scale"] + (["km"] if smooth else []) + (["v8", "v_scale"] if vfp8 else [])
    for key in keys:
        g = got[key].cpu().numpy()
        w = want[key]
        if not _eq_bits(g, w):
            diff = np.argwhere(g != w)
            raise AssertionError(f"{key}: {len(diff)} mismatches, first at {diff[:3].tolist()}: "
                                 f"got {g[tuple(diff[0])]} want {w[tuple(diff[0])]}")


def test_prepass_nhd_layout(pack_ref, hip_impl, gpu_device):
    """The reference's NHD layout (triton_impl.py:49-55) through strides."""
    inp = _inputs(pack_ref, 2, 4, 4, 200, 64, "bf16", 2.0, "normal")
    q = inp["q"].transpose(1, 2).contiguous()  # [B, N, H, D]
    k = inp["k"].transpose(1, 2).contiguous()
    want = O.prepass(_np32(inp["q"]), _np32(inp["k"]), smooth_k=True)
    got = hip_impl.prepass(q.to(gpu_device), k.to(gpu_device), k.to(gpu_device), smooth_k=True,
                           tensor_layout="NHD")
    torch.cuda.synchronize()
    assert tuple(got["q8"].shape) == tuple(q.shape)
    assert np.array_equal(got["q8"].cpu().transpose(1, 2).numpy(), want["q8"])
    assert np.array_equal(got["k8"].cpu().transpose(1, 2).numpy(), want["k8"])
    assert np.array_equal(got["q_scale"].cpu().numpy(), want["q_scale"])
    assert np.array_equal(got["k_scale"].cpu().numpy(), want["k_scale"])
    assert np.array_equal(got["km"].cpu().numpy(), want["km"])


def test_per_block_int8_mirror(pack_ref, hip_impl, gpu_device):
    """per_block_int8(q, k, km) semantics: k - km in k's dtype, then quantize."""
    inp = _inputs(pack_ref, 1, 2, 2, 333, 128, "fp16", 2.0, "normal")
    q, k = inp["q"].to(gpu_device), inp["k"].to(gpu_device)
    km = k.float().mean(dim=2, keepdim=True).to(k.dtype)
    q8, qs, k8, ks = hip_impl.per_block_int8(q, k, km=km)
    torch.cuda.synchronize()
    k_s = (k - km).float().cpu().numpy()
    wq8, wqs = O.quant_per_block_int8(_np32(q), 128, mul=O.q_multiplier(128))
    wk8, wks = O.quant_per_block_int8(k_s, 64)
    assert np.array_equal(q8.cpu().numpy(), wq8) and np.array_equal(qs.cpu().numpy(), wqs)
    assert np.array_equal(k8.cpu().numpy(), wk8) and np.array_equal(ks.cpu().numpy(), wks)


def test_per_block_int8_sm_scale_and_block_sizes(pack_ref, hip_impl, gpu_device):
    """Explicit sm_scale (triton_impl.py:60-61, 69) and non-default BLKQ / BLKK
    (the function's arguments, triton_impl.py:35), NHD layout: bit-exact."""
    inp = _inputs(pack_ref, 2, 4, 2, 300, 64, "bf16", 2.0, "normal")
    q, k = inp["q"].to(gpu_device), inp["k"].to(gpu_device)
    qn, kn = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    q8, qs, k8, ks = hip_impl.per_block_int8(qn, kn, BLKQ=64, BLKK=128, sm_scale=0.0371, tensor_layout="NHD")
    torch.cuda.synchronize()
    assert q8.shape == qn.shape and qs.shape == (2, 4, 5) and ks.shape == (2, 2, 3)
    wq8, wqs = O.quant_per_block_int8(_np32(q), 64, mul=O.q_multiplier(64, 0.0371))
    wk8, wks = O.quant_per_block_int8(_np32(k), 128)
    assert np.array_equal(q8.transpose(1, 2).cpu().numpy(), wq8) and np.array_equal(qs.cpu().numpy(), wqs)
    assert np.array_equal(k8.transpose(1, 2).cpu().numpy(), wk8) and np.array_equal(ks.cpu().numpy(), wks)


def test_prepass_special_blocks(hip_impl, gpu_device):
    """All-zero block, exact ties, the 0x3EFFFFFF quirk, -0.0, tiny values."""
    D = 64
    N = 256
    k = torch.zeros((1, 1, N, D), dtype=torch.float32)
    # block 0 all zero; block 1 has amax 127 so scale is exactly 1.0
    blk1 = k[0, 0, 64:128]
    blk1[0, 0] = 127.0
    blk1[0, 1] = 0.5
    blk1[0, 2] = -0.5
    blk1[0, 3] = 1.5
    blk1[0, 4] = -2.5
    blk1[0, 5] = float(np.uint32(0x3EFFFFFF).view(np.float32))
    blk1[0, 6] = -float(np.uint32(0x3EFFFFFF).view(np.float32))
    blk1[0, 7] = -0.0
    blk1[0, 8] = 1e-30
    blk1[0, 9] = -126.5
    # block 2: tiny values (scale near the fast-division limit)
    k[0, 0, 128:192] = torch.randn((64, D)) * 1e-33
    # block 3: large values
    k[0, 0, 192:256] = torch.randn((64, D)) * 1e30
    q = k.clone()
    got = hip_impl.prepass(q.to(gpu_device), k.to(gpu_device), k.to(gpu_device), smooth_k=False)
    torch.cuda.synchronize()
    wk8, wks = O.quant_per_block_int8(k.numpy(), 64)
    gk8 = got["k8"].cpu().numpy()
    assert np.array_equal(got["k_scale"].cpu().numpy(), wks)
    assert np.array_equal(gk8, wk8)
    assert wks[0, 0, 0] == 0.0 and wks[0, 0, 1] == 1.0
    row = gk8[0, 0, 64]
    assert list(row[:10]) == [127, 1, -1, 2, -3, 1, -1, 0, 0, -127]


# V tiles (sage_vtiles): the reference's v.to(torch.float16) (triton_impl.py:189),
# in the attention kernel's tile layout; bit-exact against numpy's conversion
# (round to nearest even) and the oracle's layout, or the oracle's FP8 codes.
VT_CASES = [
    (1, 2, 256, 64, "fp32", "fp16"),
    (2, 2, 300, 128, "bf16", "fp16"),   # ragged tail: zero keys past N
    (1, 3, 1000, 128, "fp16", "bf16"),
    (1, 2, 777, 64, "bf16", "bf16"),
    (2, 1, 333, 128, "bf16", "fp8"),
    (1, 2, 200, 64, "fp16", "fp8"),
]


@pytest.mark.parametrize("case", VT_CASES, ids=lambda c: f"B{c[0]}H{c[1]}N{c[2]}D{c[3]}-{c[4]}-to-{c[5]}")
def test_vtiles_bitexact(case, pack_ref, hip_impl, gpu_device):
    B, H, N, D, dtype, pv = case
    print(f"[vtiles] {case}", flush=True)
    inp = _inputs(pack_ref, B, H, H, N, D, dtype, 0.0, "student_t" if pv == "fp8" else "normal")
    v = inp["v"].to(gpu_device)
    v32 = _np32(inp["v"])
    if pv == "fp8":
        codes, vs = O.quant_v_fp8(v32)
        out = hip_impl.vtiles(v, "fp8", torch.from_numpy(vs).to(gpu_device))
        want = O.vtiles(codes)
        got = out.cpu().numpy()
    else:
        out = hip_impl.vtiles(v, pv)
        if pv == "fp16":
            want = O.vtiles(v32.astype(np.float16)).view(np.uint16)
        else:  # bf16: round to nearest even through torch's own conversion
            want = O.vtiles(torch.from_numpy(v32).to(torch.bfloat16).view(torch.int16).numpy()).view(np.uint16)
        got = out.cpu().numpy().view(np.uint16)
    torch.cuda.synchronize()
    assert got.size == want.size
    assert np.array_equal(got.reshape(want.shape), want)


def test_vtiles_nhd_matches_hnd(pack_ref, hip_impl, gpu_device):
    inp = _inputs(pack_ref, 2, 3, 3, 250, 128, "bf16", 0.0, "normal", seed=2)
    v = inp["v"].to(gpu_device)
    a = hip_impl.vtiles(v, "fp16")
    b = hip_impl.vtiles(v.transpose(1, 2).contiguous(), "fp16", tensor_layout="NHD")
    torch.cuda.synchronize()
    assert torch.equal(a, b)


# The pre-pass with the V tiles in its own launches (sage_prepass_vt, what
# run() uses): every output equals the separate calls' (and so the oracle's,
# which the tests above pin), the tiles byte for byte, for each placement of
# the tile role: launch A beside the statistics (fp16/bf16 with Q quantized in
# the pre-pass), launch B beside the K quantization (FP8, and fp16/bf16 when
# Q is left to the attention prologue: quant_q False), the single launch
# without statistics.
# (B, Hq, Hkv, N, D, dtype, pv, smooth_k, q_sub, layout, quant_q)
VT_CASES = [
    (1, 2, 2, 256, 64, "fp32", "fp16", True, 128, "HND", True),
    (2, 4, 2, 300, 128, "bf16", "fp16", True, 128, "HND", True),
    (2, 4, 2, 300, 128, "bf16", "bf16", False, 128, "HND", True),
    (1, 3, 3, 1000, 64, "fp16", "fp8", True, 32, "HND", True),
    (1, 6, 1, 777, 128, "bf16", "fp8", False, 1, "NHD", True),
    (1, 4, 4, 4096, 128, "bf16", "fp16", True, 128, "HND", True),
    (2, 4, 2, 300, 128, "bf16", "fp16", True, 128, "HND", False),
    (1, 4, 4, 4096, 128, "bf16", "bf16", True, 128, "HND", False),
    (1, 2, 2, 257, 64, "fp32", "fp16", True, 128, "NHD", False),
    (1, 2, 1, 1000, 128, "fp16", "fp16", False, 128, "HND", False),
]


@pytest.mark.parametrize("case", VT_CASES, ids=lambda c: f"B{c[0]}Hq{c[1]}Hkv{c[2]}N{c[3]}D{c[4]}-{c[5]}-{c[6]}"
                         f"-smooth{int(c[7])}-qsub{c[8]}-{c[9]}-q{int(c[10])}")
def test_prepass_vt_equals_separate_calls(case, pack_ref, hip_impl, gpu_device):
    B, Hq, Hkv, N, D, dtype, pv, smooth, q_sub, layout, quant_q = case
    print(f"[prepass-vt] {case}", flush=True)
    inp = _inputs(pack_ref, B, Hq, Hkv, N, D, dtype, 2.0, "student_t" if pv == "fp8" else "normal")
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    if layout == "NHD":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    kw = dict(q_sub=q_sub, smooth_k=smooth, tensor_layout=layout)
    fused = hip_impl.prepass(q, k, v, pv_dtype=pv, quant_q=quant_q, **kw)
    plain = hip_impl.prepass(q, k, v, v_fp8=pv == "fp8", **kw)
    tiles = hip_impl.vtiles(v, pv, plain.get("v_scale"), tensor_layout=layout)
    torch.cuda.synchronize()
    assert torch.equal(fused["vt"], tiles)
    keys = (("q8", "q_scale") if quant_q else ()) + ("k8", "k_scale")
    for key in keys + (("km",) if smooth else ()) + (("v_scale",) if pv == "fp8" else ()):
        assert torch.equal(fused[key], plain[key]), key


def test_vtiles_of_another_pv_type_are_rejected(pack_ref, hip_impl, gpu_device):
    """fp16 and bf16 V tiles have the same size: a pre-pass result made for one
    P.V type must not be read as the other (an "invalid argument" error)."""
    inp = _inputs(pack_ref, 1, 2, 2, 128, 64, "bf16", 2.0, "normal")
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    pre = hip_impl.prepass(q, k, v, pv_dtype="fp16")
    assert pre["vt_pv"] == "fp16"
    with pytest.raises(ValueError, match="invalid argument"):
        hip_impl.attention(q, k, v, pre, pv_dtype="bf16")
    with pytest.raises(ValueError, match="invalid argument"):
        hip_impl.attention_q(q, k, v, pre, pv_dtype="bf16")
    hip_impl.attention(q, k, v, pre, pv_dtype="fp16")  # the matching type is accepted
    torch.cuda.synchronize()
