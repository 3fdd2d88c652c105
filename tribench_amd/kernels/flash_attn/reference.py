"""flash_attn kernel pack: inputs, reference and work estimate.

Counterpart of kernels/flash_attn/reference.py of TriBench (same three entry
points, reference.py:4-38).  The inputs and the fp32 reference are those of
this repository's sage_attn pack (seeded CPU draws in a fixed order, fp32
softmax attention with GQA and the top-left causal mask), loaded from the
sibling pack by file path: packs are imported without a parent package.
"""
from __future__ import annotations

import importlib.util
from pathlib import Path


def _sage_reference():
    path = Path(__file__).resolve().parent.parent / "sage_attn" / "reference.py"
    spec = importlib.util.spec_from_file_location("tribench.kernels.sage_attn._shared_reference", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


_SAGE = _sage_reference()


def make_inputs(case: dict, device: str, seed: int, dtype, **kwargs):
    """Seeded q, k, v [B, H, N, D] and causal (reference.py:4-13); defaults
    batch 8, heads 16, seq 4096, dim 64 as in the reference."""
    return _SAGE.make_inputs(case, device, seed, dtype, **kwargs)


def ref(q, k, v, causal=False, sm_scale=None, **kwargs):
    """softmax(q k^T * sm_scale [causal]) v (reference.py:15-29), in fp32."""
    return _SAGE.ref(q, k, v, causal=causal, sm_scale=sm_scale)


def estimate(case: dict):
    """Work of one call (reference.py:31-38): flops = 4*B*H*N^2*D, bytes =
    q, k, v, o at 2 bytes; added: algo_flops (4*B*H*D*unmasked pairs) and
    vtile_bytes (V converted to the attention kernel's tile layout)."""
    B = case.get("batch_size", 8)
    H = case.get("num_heads", 16)
    Hkv = case.get("num_kv_heads", H)
    N = case.get("seq_len", 4096)
    D = case.get("head_dim", 64)
    pairs = N * (N + 1) // 2 if case.get("causal", False) else N * N
    return {
        "flops": 4 * B * H * N * N * D,
        "bytes": 4 * B * H * N * D * 2,
        "algo_flops": 4 * B * H * D * pairs,
        "vtile_bytes": 4 * B * Hkv * N * D,
    }
