"""CPU oracle of TriBench's sage_attn hot path — TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, what the reference computes on the path
``kernels/sage_attn`` of H1yori233/TriBench.  It is the checker the tests,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use;
the product path (``tribench_amd``) never imports it.

Functions and the reference lines they restate:

* :func:`q_multiplier`          triton_impl.py:60-61, 69
* :func:`quant_per_block_int8`  triton_impl.py:7-33 (kernel), 35-82 (scale
  shapes, Q/K calls); per-sub-block scales are the build's per-wave option
* :func:`k_channel_mean`        the K-smoothing hook triton_impl.py:39-40; the
  reduction order is the build's definition (sage_quant_math.h)
* :func:`e4m3_encode` / :func:`quant_v_fp8`  FP8 V (absent in the reference;
  OCP e4m3 as torch.float8_e4m3fn, RNE, saturating)
* :func:`vtiles`                the build's V tile layout of the attention
  kernel (V converted as triton_impl.py:189, v.to(torch.float16))
* :func:`sdpa`                  reference.py:15-24 (+ GQA, chunked)
* :func:`sage_emulate`          triton_impl.py:86-160 in exact arithmetic:
  dequantized int8 scores, exact softmax, fp64 P.V
* :func:`attention_flops`, :func:`prepass_bytes`  reference.py:26-34 and the
  build's algorithmic work

Pinning (tests/test_oracle.py): known-answer blocks, the 0x3EFFFFFF rounding
quirk, invariants of the quantizer, brute-force small SDPA, torch's
scaled_dot_product_attention, torch.float8_e4m3fn, and the committed fixtures
under tests/golden/.
"""
from __future__ import annotations

import math

import numpy as np

LOG2E_REF = 1.44269504  # the constant of triton_impl.py:69

# --------------------------------------------------------------------------
# quantization
# --------------------------------------------------------------------------


def q_multiplier(head_dim: int, sm_scale: float | None = None) -> np.float32:
    """fp32(sm_scale * 1.44269504), sm_scale defaulting to D**-0.5.

    triton_impl.py:60-61 computes the default in Python double and :69 passes
    the product to the kernel as an fp32 scalar.
    """
    if sm_scale is None:
        sm_scale = head_dim ** -0.5
    return np.float32(sm_scale * LOG2E_REF)


def quant_per_block_int8(x, blk: int, mul=None, q_sub: int | None = None, km=None):
    """Per-block INT8 quantization of x [B, H, N, D] (float32 values).

    triton_impl.py:25-33: x = fp32(in) * mul; scale = max|x| / 127.;
    t = x / scale; t += 0.5 * sign(t); q = trunc(t) (int8).  Rows past N are
    left out of the block max (they read as 0).  ``q_sub`` splits each block
    into sub-blocks of q_sub rows with a scale each (the build's per-wave
    option; q_sub == blk is the reference).  ``km`` [B, H, D] is subtracted in
    fp32 after the multiply (the build's K smoothing).  A block whose max is 0
    quantizes to 0 with scale 0 (the reference would compute 0/0).

    Returns (q8 int8 [B,H,N,D], scale float32 [B,H,ceil(N/blk)*(blk/q_sub)]).
    """
    x = np.asarray(x, dtype=np.float32)
    B, H, N, D = x.shape
    q_sub = blk if q_sub is None else q_sub
    assert blk % q_sub == 0
    nb = -(-N // blk)
    npad = nb * blk
    xs = np.zeros((B, H, npad, D), dtype=np.float32)
    xs[:, :, :N] = x
    if mul is not None:
        xs = xs * np.float32(mul)
    if km is not None:
        xs = xs - np.asarray(km, dtype=np.float32)[:, :, None, :]
        xs[:, :, N:] = 0.0  # padding rows stay out of the block max
    nsub = npad // q_sub
    xv = xs.reshape(B, H, nsub, q_sub * D)
    amax = np.abs(xv).max(axis=-1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = xv / scale[..., None]
    t = np.where(scale[..., None] > 0, t, np.float32(0.0)).astype(np.float32)
    half = np.where(t >= 0, np.float32(0.5), np.float32(-0.5)).astype(np.float32)
    u = (t + half).astype(np.float32)
    q8 = np.trunc(u).astype(np.int8)
    q8 = q8.reshape(B, H, npad, D)[:, :, :N]
    return np.ascontiguousarray(q8), scale


def kstat_token_lanes(D: int) -> int:
    """Token lanes of one K-statistics block (256 threads, 8 channels each)."""
    return 256 // (D // 8)


def kstat_chunk_tokens(N: int) -> int:
    """Tokens per K-statistics chunk: at most 16 chunks, multiples of 256."""
    return 256 * ((N + 4095) // 4096)


def k_channel_sum(k):
    """Channel sums of k [B, H, N, D] in the kernel's fixed order (float32).

    Per chunk of kstat_chunk_tokens(N) tokens: token lane tl adds tokens
    tl, tl+TL, ... left to right; the TL lane sums are combined by the
    halving tree acc[tl] += acc[tl + s]; the chunk partials are added left to
    right.
    """
    k = np.asarray(k, dtype=np.float32)
    B, H, N, D = k.shape
    TL = kstat_token_lanes(D)
    ch = kstat_chunk_tokens(N)
    total = None
    for n0 in range(0, N, ch):
        part = k[:, :, n0:min(n0 + ch, N)]
        L = part.shape[2]
        R = -(-L // TL)
        pad = np.zeros((B, H, R * TL, D), dtype=np.float32)
        pad[:, :, :L] = part
        pad = pad.reshape(B, H, R, TL, D)
        acc = np.zeros((B, H, TL, D), dtype=np.float32)
        for r in range(R):
            acc = (acc + pad[:, :, r]).astype(np.float32)
        s = TL
        while s > 1:
            s //= 2
            acc = (acc[:, :, :s] + acc[:, :, s:2 * s]).astype(np.float32)
        p = acc[:, :, 0]
        total = p if total is None else (total + p).astype(np.float32)
    return total


def k_channel_mean(k):
    """km[b,h,c] = channel sum / fp32(N) (IEEE division), float32 [B, H, D]."""
    k = np.asarray(k, dtype=np.float32)
    return (k_channel_sum(k) / np.float32(k.shape[2])).astype(np.float32)


# --------------------------------------------------------------------------
# FP8 e4m3 (OCP "e4m3fn": bias 7, max 448, 0x7F NaN)
# --------------------------------------------------------------------------


def e4m3_encode(x):
    """fp32 -> e4m3 codes, round-to-nearest-even, saturating at +-448."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint32)
    a = u & np.uint32(0x7FFFFFFF)
    af = a.view(np.float32)
    code = np.zeros(x.shape, dtype=np.uint32)
    sub = af < np.float32(2.0 ** -6)
    # only the subnormal lanes enter the cast (NaN, inf and large values would not fit uint32)
    sub_code = np.rint(np.where(sub, af, np.float32(0.0)) * np.float32(512.0)).astype(np.uint32)
    code = np.where(sub, sub_code, code)
    e = (a >> np.uint32(23)).astype(np.int64) - 127 + 7
    m = a & np.uint32(0x7FFFFF)
    m3 = m >> np.uint32(20)
    rem = m & np.uint32(0xFFFFF)
    up = (rem > 0x80000) | ((rem == 0x80000) & ((m3 & 1) == 1))
    norm = (np.clip(e, 0, 31).astype(np.uint32) << np.uint32(3)) + m3 + up.astype(np.uint32)
    norm = np.minimum(norm, np.uint32(0x7E))
    code = np.where(sub, code, norm)
    code = np.where(af >= np.float32(448.0), np.uint32(0x7E), code)
    code = np.where(a > np.uint32(0x7F800000), np.uint32(0x7F), code | sign)
    return code.astype(np.uint8)


_E4M3_TABLE = None


def e4m3_decode(codes):
    """e4m3 codes -> float32 values."""
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        t = np.zeros(256, dtype=np.float32)
        for c in range(256):
            s = -1.0 if c & 0x80 else 1.0
            e = (c >> 3) & 0xF
            m = c & 7
            if e == 15 and m == 7:
                t[c] = np.nan
            elif e == 0:
                t[c] = s * m * 2.0 ** -9
            else:
                t[c] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
        _E4M3_TABLE = t
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def quant_v_fp8(v):
    """Per-channel FP8 V: v_scale[b,h,c] = max_n |v| / 448; codes = e4m3(v / v_scale).

    Returns (codes uint8 [B,H,N,D], v_scale float32 [B,H,D]).
    """
    v = np.asarray(v, dtype=np.float32)
    amax = np.abs(v).max(axis=2)
    vs = (amax / np.float32(448.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = v / vs[:, :, None, :]
    t = np.where(vs[:, :, None, :] > 0, t, np.float32(0.0)).astype(np.float32)
    return e4m3_encode(t), vs


def vtile_positions() -> np.ndarray:
    """pos[k] of key k (0..63) inside a V tile: k = 32t + 8i + 4h + r -> 32h + 16t + 4i + r.

    The build's own layout (the order in which lane half h of a 32x32 MFMA C
    tile holds the keys of its column), documented in include/sage_attn.h.
    """
    k = np.arange(64)
    t, i, h, r = k >> 5, (k >> 3) & 3, (k >> 2) & 1, k & 3
    return 32 * h + 16 * t + 4 * i + r


def vtiles(v_elems):
    """Tile layout of per-element values [B, H, N, D] (any dtype, already
    converted): returns [B, H, ceil(N/64), D, 64] with keys at vtile_positions()
    and zeros past N.  The V conversion of triton_impl.py:189 (v.to(float16))
    is the caller's (e.g. numpy astype(float16)); this is only the layout."""
    v_elems = np.asarray(v_elems)
    B, H, N, D = v_elems.shape
    T = -(-N // 64)
    pad = np.zeros((B, H, T * 64, D), dtype=v_elems.dtype)
    pad[:, :, :N] = v_elems
    tiles = pad.reshape(B, H, T, 64, D).transpose(0, 1, 2, 4, 3)  # [B,H,T,D,key]
    out = np.zeros_like(tiles)
    out[..., vtile_positions()] = tiles
    return out


# --------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------


def _expand_kv(x, hq):
    h = x.shape[1]
    if h == hq:
        return x
    return np.repeat(x, hq // h, axis=1)


def sdpa(q, k, v, causal: bool = False, sm_scale: float | None = None, dtype=np.float64,
         q_chunk: int = 1024, rows=None):
    """softmax(q k^T * sm_scale [+ causal mask]) v (reference.py:15-24).

    The causal mask is the reference's torch.tril(ones(N, N)) == 0 (key j is
    masked for query i iff j > i).  KV heads are repeated for GQA
    (repeat_interleave over the head dim).  Computed in ``dtype`` per
    (batch, head, chunk of q rows) so the score matrix is never whole.
    ``rows`` (query indices) restricts the result to those rows, in that
    order: [B, Hq, len(rows), D].
    """
    q = np.asarray(q)
    B, Hq, Nq, D = q.shape
    Nkv = k.shape[2]
    if sm_scale is None:
        sm_scale = D ** -0.5
    rows = np.arange(Nq) if rows is None else np.asarray(rows, dtype=np.int64)
    out = np.empty((B, Hq, len(rows), D), dtype=dtype)
    G = Hq // k.shape[1]
    kj = np.arange(Nkv)[None, :]
    for b in range(B):
        for h in range(Hq):
            kk = np.asarray(k[b, h // G], dtype=dtype)
            vv = np.asarray(v[b, h // G], dtype=dtype)
            for i0 in range(0, len(rows), q_chunk):
                r = rows[i0:i0 + q_chunk]
                s = np.asarray(q[b, h, r], dtype=dtype) @ kk.T
                s *= dtype(sm_scale)
                if causal:
                    s = np.where(kj > r[:, None], -np.inf, s)
                s -= s.max(axis=1, keepdims=True)
                np.exp(s, out=s)
                s /= s.sum(axis=1, keepdims=True)
                out[b, h, i0:i0 + len(r)] = s @ vv
    return out


def sage_emulate(q8, q_scale, k8, k_scale, v, causal=False, blkq=128, q_sub=None, blkk=64,
                 v_scale=None, q_chunk: int = 1024, rows=None):
    """The SageAttention algorithm of triton_impl.py:86-160 in exact arithmetic.

    Scores are int8 dot products times q_scale * k_scale (log2 units: the
    log2(e) factor sits in q_scale), softmax is base 2 and exact, and P.V is
    fp64.  ``v`` is either real values or FP8 codes with ``v_scale``.  The
    difference between this and :func:`sdpa` is the quantization error; the
    difference between this and the kernel is the kernel's own arithmetic.
    ``rows`` (query indices) restricts the result to those rows, in that
    order: [B, Hq, len(rows), D].
    """
    q_sub = blkq if q_sub is None else q_sub
    B, Hq, Nq, D = q8.shape
    Hkv, Nkv = k8.shape[1], k8.shape[2]
    G = Hq // Hkv
    rows_all = np.arange(Nq) if rows is None else np.asarray(rows, dtype=np.int64)
    out = np.empty((B, Hq, len(rows_all), D), dtype=np.float64)
    kcol = np.arange(Nkv)
    for b in range(B):
        for hk in range(Hkv):
            if v_scale is not None:
                vv = e4m3_decode(v[b, hk]).astype(np.float64) * np.asarray(v_scale[b, hk], np.float64)[None, :]
            else:
                vv = np.asarray(v[b, hk], dtype=np.float64)
            kk = k8[b, hk].astype(np.float64)
            ks = np.asarray(k_scale[b, hk], np.float64)[kcol // blkk]
            for h in range(hk * G, (hk + 1) * G):
                for i0 in range(0, len(rows_all), q_chunk):
                    r = rows_all[i0:i0 + q_chunk]
                    qs = np.asarray(q_scale[b, h], np.float64)[r // q_sub]
                    s = (q8[b, h, r].astype(np.float64) @ kk.T) * qs[:, None] * ks[None, :]
                    if causal:
                        s = np.where(kcol[None, :] > r[:, None], -np.inf, s)
                    s -= s.max(axis=1, keepdims=True)
                    p = np.exp2(s)
                    p /= p.sum(axis=1, keepdims=True)
                    out[b, h, i0:i0 + len(r)] = p @ vv
    return out


def prepass(q, k, v=None, sm_scale=None, blkq=128, blkk=64, q_sub=None, smooth_k=True,
            v_fp8=False):
    """Every intermediate of the pre-pass for float32 inputs [B, H, N, D]."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    D = q.shape[-1]
    mul = q_multiplier(D, sm_scale)
    q8, qs = quant_per_block_int8(q, blkq, mul=mul, q_sub=q_sub)
    out = {"q8": q8, "q_scale": qs}
    km = k_channel_mean(k) if smooth_k else None
    k8, ks = quant_per_block_int8(k, blkk, km=km)
    out.update(k8=k8, k_scale=ks)
    if smooth_k:
        out["km"] = km
    if v_fp8:
        v8, vs = quant_v_fp8(v)
        out.update(v8=v8, v_scale=vs)
    return out


# --------------------------------------------------------------------------
# work counts
# --------------------------------------------------------------------------


def unmasked_pairs(nq: int, nkv: int, causal: bool) -> int:
    """Number of (query, key) pairs the softmax sees (top-left causal)."""
    if not causal:
        return nq * nkv
    full = min(nq, nkv)
    pairs = full * (full + 1) // 2
    if nq > nkv:
        pairs += (nq - nkv) * nkv
    return pairs


def attention_flops(B, Hq, Nq, Nkv, D, causal=False):
    """(metric ops 4*B*H*Nq*Nkv*D as reference.py:32, algorithmic ops)."""
    metric = 4 * B * Hq * Nq * Nkv * D
    algo = 4 * B * Hq * D * unmasked_pairs(Nq, Nkv, causal)
    return metric, algo


def prepass_bytes(B, Hq, Hkv, Nq, Nkv, D, in_bytes=2, blkq=128, blkk=64, q_sub=None,
                  smooth_k=True, v_fp8=False):
    """HBM bytes the pre-pass must move at minimum (reads once, writes once)."""
    q_sub = blkq if q_sub is None else q_sub
    eq, ek = B * Hq * Nq * D, B * Hkv * Nkv * D
    n = in_bytes * (eq + ek) + (eq + ek)
    n += 4 * (B * Hq * math.ceil(Nq / blkq) * (blkq // q_sub) + B * Hkv * math.ceil(Nkv / blkk))
    if smooth_k:
        n += 4 * B * Hkv * D
    if v_fp8:
        n += in_bytes * ek + ek + 4 * B * Hkv * D
    return n
