"""HIP variant of the sage_attn kernel pack (MI355X / gfx950).

``run`` has the call signature of ``run_sage_attn`` (triton_impl.py:162) and
is registered as ``variants: {"hip": "hip_impl.py:run"}`` in meta.json, so the
harness's ``test`` and ``run`` commands drive it unchanged.  It allocates every
buffer with torch on the inputs' device and calls the C ABI of
``libsage_attn.so`` (include/sage_attn.h) through ctypes, on torch's current
stream:

    sage_prepass     per_block_int8 (triton_impl.py:35-82) + K smoothing (+ FP8 V scales)
    sage_vtiles      v.to(torch.float16) (triton_impl.py:189), in the attention's V tile layout
    sage_prepass_vt  both, in the pre-pass's launches (what run() uses)
    sage_attn_fwd    _attn_fwd launch (triton_impl.py:186-199); sage_attn_fwd_q quantizes Q itself

There is no CPU or PyTorch fallback: without a ROCm device or without the
library the call raises.  The module is loaded by file path (no parent
package), so it finds the library from its own location:
``$TRIBENCH_SAGE_HIP_LIB`` when set (which must then name the file), else
``./libsage_attn.so`` next to this file, or ``tribench_amd/lib/libsage_attn.so``
of this repository.
"""
from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import numpy as np
import torch

ABI_VERSION = 6
LOG2E_REF = 1.44269504  # triton_impl.py:69
WAVE_ROWS = 32          # q rows per wavefront of the attention kernel (q_gran="wave")
# rows per Q scale for each q_gran: one block of 128 rows (the reference), one
# wavefront's 32 rows, or one row (the rows one lane of the kernel's MFMA
# operand holds, the counterpart of SageAttention's per-thread granularity)
Q_GRAN_ROWS = {"block": 128, "wave": WAVE_ROWS, "thread": 1}

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_FP8E4M3, DTYPE_VTILES = 0, 1, 2, 3, 4
V_NONE, V_FP8, V_FP8_SCALE = 0, 1, 2
PV_MODES = {"fp16": 0, "bf16": 1, "fp8": 2}
_TORCH_CODES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

_LIB = None


def library_path() -> Path:
    """Where the C-ABI library is looked up: $TRIBENCH_SAGE_HIP_LIB when set
    (it must name a file: an explicit choice never falls back to another
    library), else the first existing default candidate."""
    here = Path(__file__).resolve().parent
    env = os.environ.get("TRIBENCH_SAGE_HIP_LIB")
    if env:
        if not Path(env).is_file():
            raise RuntimeError(f"sage_attn hip: TRIBENCH_SAGE_HIP_LIB={env} is not a file")
        return Path(env)
    cands = []
    cands.append(here / "libsage_attn.so")
    cands.append(here.parents[1] / "lib" / "libsage_attn.so")
    for c in cands:
        if c.is_file():
            return c
    raise RuntimeError(
        "sage_attn hip: libsage_attn.so not found (looked in: "
        + ", ".join(str(c) for c in cands) + "); build it with `python -m tribench_amd.build`"
    )


def _load():
    global _LIB
    if _LIB is not None:
        return _LIB
    lib = ctypes.CDLL(str(library_path()))
    i64, i32, f32, vp, sz = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
    p64 = ctypes.POINTER(ctypes.c_int64)
    lib.sage_abi_version.restype = i32
    lib.sage_abi_version.argtypes = []
    ver = lib.sage_abi_version()  # before binding the rest: an older library may lack newer symbols
    if ver != ABI_VERSION:
        raise RuntimeError(f"sage_attn hip: library ABI {ver}, expected {ABI_VERSION} "
                           f"({library_path()}; rebuild with `python -m tribench_amd.build`)")
    lib.sage_last_error.restype = ctypes.c_char_p
    lib.sage_last_error.argtypes = []
    lib.sage_prepass_workspace_bytes.restype = sz
    lib.sage_prepass_workspace_bytes.argtypes = [i64, i64, i64, i64, i32, i32]
    lib.sage_prepass.restype = i32
    lib.sage_prepass.argtypes = [
        vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, p64, p64, p64, f32, i32, i32, i32, i32, i32,
        vp, p64, vp, vp, p64, vp, vp, vp, p64, vp, vp, sz, vp,
    ]
    lib.sage_prepass_vt.restype = i32
    lib.sage_prepass_vt.argtypes = lib.sage_prepass.argtypes[:-1] + [i32, vp, sz, vp]
    lib.sage_prepass_vt_noalloc.restype = i32
    lib.sage_prepass_vt_noalloc.argtypes = lib.sage_prepass.argtypes[:-3] + [i32, vp, sz, vp]
    lib.sage_vtile_bytes.restype = sz
    lib.sage_vtile_bytes.argtypes = [i64, i64, i64, i64, i32]
    lib.sage_vtiles.restype = i32
    lib.sage_vtiles.argtypes = [vp, i32, i64, i64, i64, i64, p64, i32, vp, vp, sz, vp]
    lib.sage_attn_fwd.restype = i32
    lib.sage_attn_fwd.argtypes = [
        vp, p64, vp, vp, p64, vp, vp, i32, p64, vp, vp, i32, p64, i64, i64, i64, i64, i64, i64, i32,
        i32, i32, i32, i32, vp,
    ]
    lib.sage_attn_fwd_q.restype = i32
    lib.sage_attn_fwd_q.argtypes = [
        vp, p64, i32, f32, vp, vp, vp, p64, vp, vp, i32, p64, vp, vp, p64, i64, i64, i64, i64, i64, i64, i32,
        i32, i32, i32, i32, vp,
    ]
    lib.sage_flash_fwd.restype = i32
    lib.sage_flash_fwd.argtypes = [vp, p64, vp, p64, vp, i32, p64, vp, p64, i32, i64, i64, i64, i64, i64, i64, f32,
                                   i32, vp]
    _LIB = lib
    return lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _load().sage_last_error().decode(errors="replace")
        raise RuntimeError(f"sage_attn hip: {what} failed: {msg}")


def _strides(t: torch.Tensor, layout: str):
    """(batch, head, seq) element strides of a 4-D tensor in the given layout."""
    s = t.stride()
    if layout == "HND":
        vals = (s[0], s[1], s[2])
    elif layout == "NHD":
        vals = (s[0], s[2], s[1])
    else:
        raise ValueError(f"sage_attn hip: invalid argument: tensor_layout {layout!r}")
    return (ctypes.c_int64 * 3)(*vals)


def _dims(t: torch.Tensor, layout: str):
    if layout == "HND":
        b, h, n, d = t.shape
    else:
        b, n, h, d = t.shape
    return b, h, n, d


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _on_tensor_device(fn):
    """Run ``fn`` with the device of its first tensor argument current.

    The library launches on torch's current stream of that device and keeps
    per-device state (the no-allocation entry point's scratch array, found
    with hipGetDevice), so the data's device must be the current one
    whatever device the caller left current.
    """
    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        dev = next((a.device for a in args if isinstance(a, torch.Tensor)), None)
        if dev is None or dev.type != "cuda":
            return fn(*args, **kwargs)
        with torch.cuda.device(dev):
            return fn(*args, **kwargs)
    return wrapper


def _check_inputs(q, k, v, layout):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"sage_attn hip: invalid argument: {name} is not a tensor")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"sage_attn hip: {name} is on {t.device}; this variant runs only on a ROCm GPU device")
        if t.dim() != 4 or t.stride(3) != 1:
            raise ValueError(f"sage_attn hip: invalid argument: {name} must be 4-D with a unit head-dim stride")
        if t.dtype not in _TORCH_CODES:
            raise ValueError(f"sage_attn hip: invalid argument: {name} dtype {t.dtype}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("sage_attn hip: invalid argument: q, k, v dtypes differ")
    if not (q.device == k.device == v.device):
        raise ValueError("sage_attn hip: invalid argument: q, k, v devices differ")
    B, Hq, Nq, D = _dims(q, layout)
    Bk, Hkv, Nkv, Dk = _dims(k, layout)
    if _dims(v, layout) != (Bk, Hkv, Nkv, Dk) or Bk != B or Dk != D:
        raise ValueError(f"sage_attn hip: invalid argument: shape mismatch q{tuple(q.shape)} "
                         f"k{tuple(k.shape)} v{tuple(v.shape)}")
    if Hq % Hkv:
        raise ValueError(f"sage_attn hip: invalid argument: {Hq} query heads not a multiple of {Hkv} kv heads")
    return B, Hq, Hkv, Nq, Nkv, D


def _empty_like_layout(t: torch.Tensor, dtype) -> torch.Tensor:
    return torch.empty_like(t, dtype=dtype, memory_format=torch.preserve_format)


@_on_tensor_device
def vtiles(v, pv_dtype="fp16", v_scale=None, *, tensor_layout="HND"):
    """V in the attention kernel's tile layout (uint8 buffer), converted to
    the P.V type: the counterpart of the reference's v.to(torch.float16)
    (triton_impl.py:189).  ``pv_dtype`` "fp8" needs the per-channel v_scale
    [B,Hkv,D] of :func:`prepass`."""
    lib = _load()
    if pv_dtype not in PV_MODES:
        raise ValueError(f"sage_attn hip: invalid argument: pv_dtype {pv_dtype!r}")
    B, Hkv, Nkv, D = _dims(v, tensor_layout)
    mode = PV_MODES[pv_dtype]
    if pv_dtype == "fp8" and v_scale is None:
        raise ValueError("sage_attn hip: invalid argument: fp8 V tiles need v_scale")
    nbytes = lib.sage_vtile_bytes(B, Hkv, Nkv, D, mode)
    out = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=v.device)
    rc = lib.sage_vtiles(_ptr(v), _TORCH_CODES[v.dtype], B, Hkv, Nkv, D, _strides(v, tensor_layout), mode,
                         _ptr(v_scale), _ptr(out), ctypes.c_size_t(nbytes), _stream(v.device))
    _check(rc, "sage_vtiles")
    return out


@_on_tensor_device
def prepass(q, k, v=None, sm_scale=None, *, blkq=128, blkk=64, q_sub=None, smooth_k=True,
            v_fp8=False, pv_dtype=None, quant_q=True, tensor_layout="HND", static_scratch=False):
    """Run the HIP pre-pass; returns a dict of device tensors.

    q8/k8 (int8, same layout as q/k), q_scale [B,Hq,ceil(Nq/blkq)*(blkq/q_sub)],
    k_scale [B,Hkv,ceil(Nkv/blkk)], km [B,Hkv,D] (smooth_k), v8 (row-major e4m3
    codes as uint8) + v_scale [B,Hkv,D] (v_fp8), and with ``pv_dtype`` the V
    tiles ``vt`` that :func:`attention` reads (v_scale too for "fp8").  With
    ``quant_q=False`` Q is left to :func:`attention_q` (no q8 / q_scale).
    ``static_scratch=True`` (needs ``pv_dtype``) calls sage_prepass_vt_noalloc,
    whose partial sums live in the library's fixed per-GPU scratch array
    instead of a workspace tensor (calls that overlap on one GPU race on it).
    """
    lib = _load()
    B, Hq, Hkv, Nq, Nkv, D = _check_inputs(q, k, v if v is not None else k, tensor_layout)
    if pv_dtype is not None and pv_dtype not in PV_MODES:
        raise ValueError(f"sage_attn hip: invalid argument: pv_dtype {pv_dtype!r}")
    v_mode = V_FP8 if v_fp8 else (V_FP8_SCALE if pv_dtype == "fp8" else V_NONE)
    q_sub = blkq if q_sub is None else q_sub
    if sm_scale is None:
        sm_scale = D ** -0.5
    q_mul = float(np.float32(sm_scale * LOG2E_REF))
    dev = q.device
    q8 = _empty_like_layout(q, torch.int8) if quant_q else None
    k8 = _empty_like_layout(k, torch.int8)
    nqs = -(-Nq // blkq) * (blkq // q_sub)
    q_scale = torch.empty((B, Hq, nqs), dtype=torch.float32, device=dev) if quant_q else None
    k_scale = torch.empty((B, Hkv, -(-Nkv // blkk)), dtype=torch.float32, device=dev)
    km = torch.empty((B, Hkv, D), dtype=torch.float32, device=dev) if smooth_k else None
    v8 = v_scale = None
    if v_mode != V_NONE:
        v_scale = torch.empty((B, Hkv, D), dtype=torch.float32, device=dev)
    if v_fp8:
        v8 = _empty_like_layout(v, torch.uint8)
    if static_scratch and pv_dtype is None:
        raise ValueError("sage_attn hip: invalid argument: static_scratch needs pv_dtype (sage_prepass_vt_noalloc)")
    ws_bytes = 0 if static_scratch else lib.sage_prepass_workspace_bytes(B, Hkv, Nkv, D, int(smooth_k), v_mode)
    ws = None if static_scratch else torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    uses_v = v_mode != V_NONE or pv_dtype is not None
    args = [
        _ptr(q) if quant_q else None, _ptr(k), _ptr(v) if uses_v else None, _TORCH_CODES[q.dtype], B, Hq, Hkv,
        Nq, Nkv, D, _strides(q, tensor_layout) if quant_q else None, _strides(k, tensor_layout),
        _strides(v, tensor_layout) if uses_v else None,
        q_mul, blkq, blkk, q_sub, int(smooth_k), v_mode,
        _ptr(q8), _strides(q8, tensor_layout) if quant_q else None, _ptr(q_scale), _ptr(k8),
        _strides(k8, tensor_layout),
        _ptr(k_scale), _ptr(km), _ptr(v8), _strides(v8, tensor_layout) if v_fp8 else None, _ptr(v_scale),
    ]
    vt = None
    if pv_dtype is None:
        rc = lib.sage_prepass(*args, _ptr(ws), ctypes.c_size_t(ws_bytes), _stream(dev))
        _check(rc, "sage_prepass")
    else:
        # the V tiles of vtiles(), written by the pre-pass's own launches
        nbytes = lib.sage_vtile_bytes(B, Hkv, Nkv, D, PV_MODES[pv_dtype])
        vt = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
        tail = [PV_MODES[pv_dtype], _ptr(vt), ctypes.c_size_t(nbytes), _stream(dev)]
        if static_scratch:
            rc = lib.sage_prepass_vt_noalloc(*args, *tail)
            _check(rc, "sage_prepass_vt_noalloc")
        else:
            rc = lib.sage_prepass_vt(*args, _ptr(ws), ctypes.c_size_t(ws_bytes), *tail)
            _check(rc, "sage_prepass_vt")
    out = {"k8": k8, "k_scale": k_scale}
    if ws is not None:
        out["workspace"] = ws
    if quant_q:
        out["q8"] = q8
        out["q_scale"] = q_scale
    if smooth_k:
        out["km"] = km
    if v_fp8:
        out["v8"] = v8
    if v_scale is not None:
        out["v_scale"] = v_scale
    if vt is not None:
        out["vt"] = vt
        out["vt_pv"] = pv_dtype  # the tiles' element type: attention() checks it against its pv_dtype
    return out


def q_sub_of(q_gran):
    """Rows per Q scale for a q_gran option (raises on an unknown one)."""
    if q_gran not in Q_GRAN_ROWS:
        raise ValueError(f"sage_attn hip: invalid argument: q_gran {q_gran!r}")
    return Q_GRAN_ROWS[q_gran]


def fuse_q_default(head_dim):
    """Where Q is quantized when the caller does not say: in the attention
    kernel's prologue at D = 128 (measured 1-2 % faster per forward at
    configurations 2 and 3, even at 5), in the pre-pass at D = 64 (the
    prologue costs more than it saves there: 2 % slower at configuration 4)."""
    return head_dim == 128


@_on_tensor_device
def prepass_stage(q, k, v, causal=False, sm_scale=None, *, pv_dtype="fp16", q_gran="block", smooth_k=True,
                  fuse_q=None, tensor_layout="HND", **kw):
    """The pre-pass of :func:`run` alone, with run's arguments (the harness
    times it as the ``prepass`` stage to report its HBM rate)."""
    q_sub = q_sub_of(q_gran)
    if fuse_q is None:
        fuse_q = fuse_q_default(_dims(q, tensor_layout)[3])
    return prepass(q, k, v, sm_scale, q_sub=q_sub, smooth_k=smooth_k, pv_dtype=pv_dtype, quant_q=not fuse_q,
                   tensor_layout=tensor_layout)


@_on_tensor_device
def per_block_int8(q, k, km=None, BLKQ=128, BLKK=64, sm_scale=None, tensor_layout="HND"):
    """HIP counterpart of per_block_int8 (triton_impl.py:35-82).

    Returns (q_int8, q_scale, k_int8, k_scale).  A caller-supplied ``km`` is
    subtracted from k in k's dtype first, as the reference does (:39-40).
    """
    if km is not None:
        k = k - km
    r = prepass(q, k, k, sm_scale, blkq=BLKQ, blkk=BLKK, smooth_k=False, tensor_layout=tensor_layout)
    return r["q8"], r["q_scale"], r["k8"], r["k_scale"]


def _tiles_for(pre, v, pv_dtype, B, Hkv, Nkv, D, tensor_layout):
    """The V tiles the attention kernel reads: ``pre["vt"]`` when present (it
    must hold ``pv_dtype`` elements: fp16 and bf16 tiles have the same size,
    so a mismatch would otherwise be read as the wrong type), else built from v."""
    vt = pre.get("vt")
    if vt is None:
        return vtiles(v, pv_dtype, pre.get("v_scale"), tensor_layout=tensor_layout)
    if pre.get("vt_pv") != pv_dtype:
        raise ValueError(f"sage_attn hip: invalid argument: pre['vt'] holds {pre.get('vt_pv')!r} tiles, "
                         f"the attention was asked for pv_dtype {pv_dtype!r}")
    if vt.numel() < _load().sage_vtile_bytes(B, Hkv, Nkv, D, PV_MODES[pv_dtype]):
        raise ValueError(f"sage_attn hip: invalid argument: pre['vt'] is not a {pv_dtype} tile buffer")
    return vt


@_on_tensor_device
def attention(q, k, v, pre, causal=False, *, pv_dtype="fp16", q_sub=128, blkq=128, blkk=64, tensor_layout="HND",
              out=None):
    """Launch the fused attention kernel on the outputs of :func:`prepass`.

    Replaces the _attn_fwd launch of triton_impl.py:186-199.  V is read from
    ``pre["vt"]`` (built here from ``v`` when absent).  Returns o with q's
    shape and dtype (written into ``out`` when given).
    """
    lib = _load()
    if pv_dtype not in PV_MODES:
        raise ValueError(f"sage_attn hip: invalid argument: pv_dtype {pv_dtype!r}")
    B, Hq, Hkv, Nq, Nkv, D = _check_inputs(q, k, v, tensor_layout)
    o = _empty_like_layout(q, q.dtype) if out is None else out
    vt = _tiles_for(pre, v, pv_dtype, B, Hkv, Nkv, D, tensor_layout)
    rc = lib.sage_attn_fwd(
        _ptr(pre["q8"]), _strides(pre["q8"], tensor_layout), _ptr(pre["q_scale"]),
        _ptr(pre["k8"]), _strides(pre["k8"], tensor_layout), _ptr(pre["k_scale"]),
        _ptr(vt), DTYPE_VTILES, None, _ptr(pre.get("v_scale")),
        _ptr(o), _TORCH_CODES[o.dtype], _strides(o, tensor_layout),
        B, Hq, Hkv, Nq, Nkv, D, int(bool(causal)), blkq, blkk, q_sub, PV_MODES[pv_dtype], _stream(q.device),
    )
    _check(rc, "sage_attn_fwd")
    return o


@_on_tensor_device
def attention_q(q, k, v, pre, causal=False, sm_scale=None, *, pv_dtype="fp16", q_sub=128, blkk=64,
                tensor_layout="HND", out=None, q8_out=None, q_scale_out=None):
    """The fused attention with the Q quantization of the pre-pass done in its
    prologue (C-ABI sage_attn_fwd_q; BLKQ 128): ``pre`` from
    :func:`prepass` with ``quant_q=False``.  ``q8_out`` / ``q_scale_out``
    (optional) receive Q8 and q_scale.  Returns o with q's shape and dtype.
    """
    lib = _load()
    if pv_dtype not in PV_MODES:
        raise ValueError(f"sage_attn hip: invalid argument: pv_dtype {pv_dtype!r}")
    B, Hq, Hkv, Nq, Nkv, D = _check_inputs(q, k, v, tensor_layout)
    if sm_scale is None:
        sm_scale = D ** -0.5
    q_mul = float(np.float32(sm_scale * LOG2E_REF))
    o = _empty_like_layout(q, q.dtype) if out is None else out
    vt = _tiles_for(pre, v, pv_dtype, B, Hkv, Nkv, D, tensor_layout)
    if q8_out is not None and (q8_out.dtype != torch.int8 or q8_out.stride() != q.stride()):
        raise ValueError("sage_attn hip: invalid argument: q8_out must be int8 with q's strides")
    rc = lib.sage_attn_fwd_q(
        _ptr(q), _strides(q, tensor_layout), _TORCH_CODES[q.dtype], ctypes.c_float(q_mul), _ptr(q8_out),
        _ptr(q_scale_out), _ptr(pre["k8"]), _strides(pre["k8"], tensor_layout), _ptr(pre["k_scale"]),
        _ptr(vt), DTYPE_VTILES, None, _ptr(pre.get("v_scale")), _ptr(o), _strides(o, tensor_layout),
        B, Hq, Hkv, Nq, Nkv, D, int(bool(causal)), 128, blkk, q_sub, PV_MODES[pv_dtype], _stream(q.device),
    )
    _check(rc, "sage_attn_fwd_q")
    return o


@_on_tensor_device
def run(q, k, v, causal=False, sm_scale=None, *, pv_dtype="fp16", q_gran="block", smooth_k=True,
        fuse_q=None, tensor_layout="HND", return_intermediates=False, **kw):
    """SageAttention forward on MI355X: INT8 QK^T, online softmax, P.V.

    Same call as run_sage_attn(q, k, v, causal=False, sm_scale=None)
    (triton_impl.py:162): q [B,Hq,N,D], k/v [B,Hkv,N,D] (HND), fp16/bf16/fp32,
    returns o with q's shape and dtype.  Unlike the reference, ``causal`` is
    honoured.  Options (case keys of meta.json arrive here):

    pv_dtype   "fp16" (the reference's P.V type), "bf16", or "fp8" (FP8 e4m3 P
               and per-channel FP8 V)
    q_gran     "block": one Q scale per 128 rows (reference); "wave": one per
               32 rows (the attention kernel's per-wavefront tile); "thread":
               one per row (each lane of the kernel holds one query row)
    smooth_k   subtract the per-channel K mean before quantizing (default on)
    fuse_q     quantize Q in the attention kernel's prologue (True) or in the
               pre-pass (False): the same Q8 and scales bit for bit; by
               default (None) as fuse_q_default(D) measured faster
    """
    if pv_dtype not in PV_MODES:
        raise ValueError(f"sage_attn hip: invalid argument: pv_dtype {pv_dtype!r}")
    q_sub = q_sub_of(q_gran)
    _check_inputs(q, k, v, tensor_layout)
    blkq, blkk = 128, 64  # BLOCK_M / BLOCK_N of triton_impl.py:166-167
    if fuse_q is None:
        fuse_q = fuse_q_default(_dims(q, tensor_layout)[3])
    pre = prepass(q, k, v, sm_scale, blkq=blkq, blkk=blkk, q_sub=q_sub, smooth_k=smooth_k,
                  pv_dtype=pv_dtype, quant_q=not fuse_q, tensor_layout=tensor_layout)
    if fuse_q:
        q8 = qs = None
        if return_intermediates:
            B, Hq, Nq, _ = _dims(q, tensor_layout)
            q8 = _empty_like_layout(q, torch.int8)
            qs = torch.empty((B, Hq, -(-Nq // blkq) * (blkq // q_sub)), dtype=torch.float32, device=q.device)
            pre["q8"], pre["q_scale"] = q8, qs
        o = attention_q(q, k, v, pre, causal, sm_scale, pv_dtype=pv_dtype, q_sub=q_sub, blkk=blkk,
                        tensor_layout=tensor_layout, q8_out=q8, q_scale_out=qs)
    else:
        o = attention(q, k, v, pre, causal, pv_dtype=pv_dtype, q_sub=q_sub, blkq=blkq, blkk=blkk,
                      tensor_layout=tensor_layout)
    if return_intermediates:
        for key in ("workspace", "vt", "vt_pv"):
            pre.pop(key, None)
        return o, pre
    return o
