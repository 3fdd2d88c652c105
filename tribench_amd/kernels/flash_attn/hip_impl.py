"""HIP variant of the flash_attn kernel pack (MI355X / gfx950).

``run`` has the call signature of ``run_flash_attn`` (kernels/flash_attn/
triton_impl.py:103) and is registered as ``variants: {"hip": "hip_impl.py:run"}``.
It runs the attention kernel of libsage_attn.so on unquantized fp16/bf16 Q
and K (C-ABI ``sage_flash_fwd``): S = Q K^T in fp32 from fp16/bf16 MFMAs, an
online softmax, P rounded to V's dtype as the reference does (:87-88), P.V
accumulated in fp32.  V first goes through ``sage_vtiles`` (the 16-bit V^T
tile layout the kernel copies into LDS).

The library loader, argument checks and ``vtiles`` are the sage_attn pack's
(loaded from the sibling pack by file path; packs have no parent package).
There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import importlib.util
from pathlib import Path

import numpy as np
import torch


def _sage_hip():
    path = Path(__file__).resolve().parent.parent / "sage_attn" / "hip_impl.py"
    spec = importlib.util.spec_from_file_location("tribench.kernels.sage_attn._shared_hip_impl", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


_H = _sage_hip()
_PV_OF = {torch.float16: "fp16", torch.bfloat16: "bf16"}


@_H._on_tensor_device
def run(q, k, v, causal=False, sm_scale=None, *, tensor_layout="HND", **kw):
    """FlashAttention forward on MI355X: q [B,Hq,Nq,D], k/v [B,Hkv,Nkv,D]
    (HND, or NHD with ``tensor_layout``), fp16 or bf16; returns o with q's
    shape and dtype.  ``causal`` uses the top-left mask (key j visible to
    query i iff j <= i), as the reference's ``offs_m >= start_n + offs_n``
    (triton_impl.py:71-72)."""
    lib = _H._load()
    B, Hq, Hkv, Nq, Nkv, D = _H._check_inputs(q, k, v, tensor_layout)
    if q.dtype not in _PV_OF:
        raise ValueError(f"sage_attn hip: invalid argument: flash_attn takes fp16 or bf16, not {q.dtype}")
    if sm_scale is None:
        sm_scale = D ** -0.5  # triton_impl.py:104-105
    qk_mul = float(np.float32(sm_scale * _H.LOG2E_REF))
    vt = _H.vtiles(v, _PV_OF[q.dtype], tensor_layout=tensor_layout)
    o = _H._empty_like_layout(q, q.dtype)
    rc = lib.sage_flash_fwd(
        _H._ptr(q), _H._strides(q, tensor_layout), _H._ptr(k), _H._strides(k, tensor_layout),
        _H._ptr(vt), _H.DTYPE_VTILES, None, _H._ptr(o), _H._strides(o, tensor_layout),
        _H._TORCH_CODES[q.dtype], B, Hq, Hkv, Nq, Nkv, D, ctypes.c_float(qk_mul), int(bool(causal)),
        _H._stream(q.device),
    )
    _H._check(rc, "sage_flash_fwd")
    return o
