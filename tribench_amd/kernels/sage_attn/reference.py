"""sage_attn kernel pack: inputs, reference and work estimate.

Counterpart of kernels/sage_attn/reference.py of TriBench (same three entry
points and calling convention, reference.py:4-34), extended with what the
benchmark configurations need: grouped KV heads, a per-channel K offset,
Student-t V, causal cases, and options passed through to the HIP variant.

This file is loaded by file path (no parent package), so it imports nothing
relative.
"""
from __future__ import annotations

import math

import torch

# case keys that are passed through to the implementation as keyword options
_IMPL_OPTION_KEYS = ("pv_dtype", "q_gran", "smooth_k")


def _gen(shape, g):
    return torch.randn(shape, generator=g, dtype=torch.float32)


def make_inputs(case: dict, device: str, seed: int, dtype: torch.dtype, **kwargs):
    """Seeded synthetic q, k, v (reference.py:4-13).

    Draws happen on the CPU in fp32 from ``torch.Generator().manual_seed(seed)``
    in a fixed order — q, k, v, the K channel offset, then the Student-t
    denominators — and are then cast to ``dtype`` and moved to ``device``, so a
    CPU baseline and the GPU see identical values.

    Case keys (defaults follow the reference): batch_size 8, num_heads 16,
    num_kv_heads (= num_heads), seq_len 4096, head_dim 64, causal False,
    k_offset_std (0: no offset; the offset is N(0, std) per channel, constant
    over tokens), v_dist "normal" | "student_t" with v_df.
    """
    B = case.get("batch_size", 8)
    H = case.get("num_heads", 16)
    Hkv = case.get("num_kv_heads", H)
    N = case.get("seq_len", 4096)
    D = case.get("head_dim", 64)
    g = torch.Generator().manual_seed(seed)
    q = _gen((B, H, N, D), g)
    k = _gen((B, Hkv, N, D), g)
    v = _gen((B, Hkv, N, D), g)
    off_std = float(case.get("k_offset_std", 0.0))
    if off_std > 0:
        k = k + _gen((B, Hkv, 1, D), g) * off_std
    if case.get("v_dist", "normal") == "student_t":
        df = int(case.get("v_df", 3))
        chi2 = torch.zeros((B, Hkv, N, D), dtype=torch.float32)
        for _ in range(df):
            chi2 += _gen((B, Hkv, N, D), g) ** 2
        v = v / torch.sqrt(chi2 / df)
    out = {
        "q": q.to(dtype).to(device),
        "k": k.to(dtype).to(device),
        "v": v.to(dtype).to(device),
        "causal": bool(case.get("causal", False)),
    }
    for key in _IMPL_OPTION_KEYS:
        if key in case:
            out[key] = case[key]
    return out


def ref(q, k, v, causal=False, sm_scale=None, q_chunk: int = 1024, **kwargs):
    """fp32 scaled-dot-product attention (reference.py:15-24).

    softmax(q k^T * sm_scale) v with the reference's causal mask (key j hidden
    from query i iff j > i, torch.tril of reference.py:19-22).  Unlike the
    reference, which multiplies in the input dtype and cannot broadcast
    grouped heads, this computes in fp32 on the inputs' device, repeats KV
    heads for GQA (repeat_interleave), and works on chunks of q rows so the
    score matrix never exists whole.  Returns fp32 [B, Hq, Nq, D].
    """
    B, Hq, Nq, D = q.shape
    Hkv, Nkv = k.shape[1], k.shape[2]
    if sm_scale is None:
        sm_scale = D ** -0.5
    G = Hq // Hkv
    out = torch.empty((B, Hq, Nq, D), dtype=torch.float32, device=q.device)
    kcol = torch.arange(Nkv, device=q.device)
    for b in range(B):
        for hk in range(Hkv):
            kk = k[b, hk].float()
            vv = v[b, hk].float()
            for h in range(hk * G, (hk + 1) * G):
                for i0 in range(0, Nq, q_chunk):
                    i1 = min(i0 + q_chunk, Nq)
                    s = (q[b, h, i0:i1].float() @ kk.t()) * sm_scale
                    if causal:
                        rows = torch.arange(i0, i1, device=q.device)
                        s.masked_fill_(kcol[None, :] > rows[:, None], float("-inf"))
                    out[b, h, i0:i1] = torch.softmax(s, dim=-1) @ vv
    return out


def estimate(case: dict):
    """Work of one call (reference.py:26-34).

    ``flops`` is the reference's 4*B*H*N^2*D (the headline metric counts this
    even for causal cases); ``bytes`` is the reference's q, k, v, o at 2 bytes.
    Added: ``algo_flops`` (4*B*Hq*D*unmasked pairs), ``prepass_bytes`` (the
    HBM floor of the quantization pre-pass), ``prepass_bytes_k`` (the same
    without Q, when the attention kernel quantizes Q itself) and
    ``vtile_bytes`` (the HBM floor of converting V to the 16-bit P.V type,
    the reference's v.to(float16) of triton_impl.py:189; 0 for FP8 P.V, whose
    V codes are in prepass_bytes).
    """
    B = case.get("batch_size", 8)
    H = case.get("num_heads", 16)
    Hkv = case.get("num_kv_heads", H)
    N = case.get("seq_len", 4096)
    D = case.get("head_dim", 64)
    causal = bool(case.get("causal", False))
    flops = 4 * B * H * N * N * D
    pairs = N * (N + 1) // 2 if causal else N * N
    in_bytes = 2
    eq, ek = B * H * N * D, B * Hkv * N * D
    q_sub = {"wave": 32, "thread": 1}.get(case.get("q_gran"), 128)  # rows per Q scale
    q_part = in_bytes * eq + eq + 4 * B * H * math.ceil(N / 128) * (128 // q_sub)
    pre_k = in_bytes * ek + ek + 4 * B * Hkv * math.ceil(N / 64)
    if case.get("smooth_k", True):
        pre_k += 4 * B * Hkv * D
    fp8 = case.get("pv_dtype") == "fp8"
    if fp8:
        pre_k += in_bytes * ek + ek + 4 * B * Hkv * D
    pre = q_part + pre_k
    return {
        "flops": flops,
        "bytes": 4 * B * H * N * D * 2,
        "algo_flops": 4 * B * H * D * pairs,
        "prepass_bytes": pre,
        "prepass_bytes_k": pre_k,
        "vtile_bytes": 0 if fp8 else (in_bytes + 2) * ek,
    }
