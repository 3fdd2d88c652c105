"""Checks shared by the full-size GPU parity tests (not a test module).

* ``prepass_mismatches``: the pre-pass outputs of a GPU call against the CPU
  oracle, bit for bit, per (batch, kv head) slice (the oracle runs on one
  slice with that kv head's query heads at a time, to bound host memory).
* ``emulation_split``: on sampled query rows of one (batch, head), the kernel
  output against the exact emulation of the same INT8 data (the kernel's own
  error, with its bound) and both against the fp32 reference (the
  quantization's share of the error and the kernel's total), so that the
  north star's max-abs / cosine budget splits into the algorithm's part and
  the kernel's part.
"""
from __future__ import annotations

import numpy as np

from oracle import sage_oracle as O

SAMPLE = 256


def sample_rows(N: int, seed: int, sample: int = SAMPLE) -> np.ndarray:
    """The first and last ``sample`` rows and ``sample`` seeded random ones, sorted."""
    rng = np.random.default_rng(seed)
    rows = np.concatenate([np.arange(min(sample, N)), np.arange(max(N - sample, 0), N),
                           rng.choice(N, size=min(sample, N), replace=False)])
    return np.unique(rows)


def first_mismatch(name, got, want):
    if np.array_equal(got, want):
        return None
    diff = np.argwhere(got != want)
    i = tuple(diff[0])
    return f"{name}: {len(diff)} mismatches, first at {list(i)}: got {got[i]} want {want[i]}"


def prepass_mismatches(outputs: dict, qn, kn, vn, *, q_sub, smooth_k=True, v_fp8=False, keys_q=("q8", "q_scale"),
                       keys_k=("k8", "k_scale", "km"), label="") -> list[str]:
    """Every mismatch between ``outputs`` (host arrays of a GPU call) and the
    oracle's pre-pass on the fp32 inputs ``qn, kn, vn``."""
    B, Hq = qn.shape[:2]
    Hkv = kn.shape[1]
    G = Hq // Hkv
    errors = []
    for b in range(B):
        for hk in range(Hkv):
            hs = slice(hk * G, (hk + 1) * G)
            want = O.prepass(qn[b:b + 1, hs], kn[b:b + 1, hk:hk + 1], vn[b:b + 1, hk:hk + 1], q_sub=q_sub,
                             smooth_k=smooth_k, v_fp8=v_fp8)
            checks = [(key, outputs[key][b:b + 1, hs], want[key]) for key in keys_q]
            checks += [(key, outputs[key][b:b + 1, hk:hk + 1], want[key]) for key in keys_k]
            for what, got, w in checks:
                msg = first_mismatch(f"b{b} hk{hk} {label}{what}", got, w)
                if msg:
                    errors.append(msg)
    return errors


def _rows(x, b: int, h: int, rows: np.ndarray) -> np.ndarray:
    """Rows ``rows`` of (b, h) of a [B,H,N,D] numpy array or torch tensor, as fp64 on the host."""
    if isinstance(x, np.ndarray):
        return x[b, h, rows].astype(np.float64)
    import torch

    idx = torch.as_tensor(rows, device=x.device, dtype=torch.long)
    return x[b, h].index_select(0, idx).double().cpu().numpy()


def half_ulp(x: np.ndarray, dtype: str) -> np.ndarray:
    """Half an ulp of the output type at |x| (the most its round-to-nearest
    moves a value): bf16 keeps 8 significant bits, fp16 11 (normal range;
    2^-25 below it), fp32 is treated as exact."""
    if dtype == "fp32":
        return np.zeros_like(x)
    bits, emin = (8, -126) if dtype == "bf16" else (11, -14)
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** emin)))
    return np.ldexp(1.0, (e - bits).astype(np.int64))


def _round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """``x`` rounded to the output type (round to nearest even), as fp64."""
    if dtype == "fp32":
        return x.astype(np.float32).astype(np.float64)
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float64))
    return t.to(torch.bfloat16 if dtype == "bf16" else torch.float16).double().numpy()


def _cos(a, b) -> float:
    a, b = a.ravel(), b.ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def emulation_split(got_o, ref_o, inter: dict, vn, b: int, h: int, G: int, *, causal: bool, q_sub,
                    fp8_v=None, seed: int | None = None, out_dtype: str = "bf16", sample: int = SAMPLE) -> dict:
    """Sampled rows of (b, h): the kernel (``got_o`` [B,Hq,N,D], host array or
    device tensor) against the exact emulation of the INT8 data in ``inter``
    (host q8, q_scale, k8, k_scale from the same call) and both against the
    fp32 reference ``ref_o`` (same shape).  ``fp8_v``: (codes, v_scale) of the FP8 V.  Returns the
    per-element error, the kernel-vs-emulation bound (fp16/bf16 P:
    2e-3 + 2^-8 |emu|, the 16-bit output rounding; FP8 P.V: 2^-4 max|v| over
    the row's keys + 2^-8 |emu|) and the summary figures.

    The kernel rounds its fp32 result to the output type ``out_dtype`` once,
    as the reference does; the emulation is not rounded.  ``arith`` is the
    part of |o - emu| beyond half an ulp of the output, i.e. what the
    kernel's arithmetic before that rounding must account for."""
    N = int(got_o.shape[2])
    hk = h // G
    rows = sample_rows(N, seed=h if seed is None else seed, sample=sample)
    sl = (slice(b, b + 1), slice(h, h + 1))
    kv = (slice(b, b + 1), slice(hk, hk + 1))
    if fp8_v is not None:
        codes, vsc = fp8_v[0][kv], fp8_v[1][kv]
    else:
        codes, vsc = vn[kv], None
    emu = O.sage_emulate(inter["q8"][sl], inter["q_scale"][sl], inter["k8"][kv], inter["k_scale"][kv], codes,
                         causal=causal, q_sub=q_sub, v_scale=vsc, rows=rows)[0, 0]
    got = _rows(got_o, b, h, rows)
    ref = _rows(ref_o, b, h, rows)
    if fp8_v is not None:
        vdec = O.e4m3_decode(codes[0, 0]).astype(np.float64) * vsc[0, 0][None, :]
        vmax = np.abs(vdec).max(axis=-1)
        row_vmax = np.maximum.accumulate(vmax)[rows] if causal else np.full(len(rows), vmax.max())
        bound = 2.0 ** -4 * row_vmax[:, None] + 2.0 ** -8 * np.abs(emu)
    else:
        bound = 2e-3 + 2.0 ** -8 * np.abs(emu)
    e = np.abs(got - emu)
    arith = np.maximum(e - half_ulp(got, out_dtype), 0.0)
    emu_rounded = _round_to(emu, out_dtype)
    late = rows >= 128
    return {
        "rows": rows, "err": e, "bound": bound, "got": got, "emu": emu, "ref": ref, "arith": arith,
        "kernel_vs_emu_max_abs": float(e.max()), "ratio": float((e / bound).max()),
        "arith_max_abs": float(arith.max()), "arith_ratio": float((arith / bound).max()),
        "eq_rounded": float((got == emu_rounded).mean()),
        "emu_vs_ref_max_abs": float(np.abs(emu - ref).max()), "emu_vs_ref_cos": _cos(emu, ref),
        "kernel_vs_ref_max_abs": float(np.abs(got - ref).max()), "kernel_vs_ref_cos": _cos(got, ref),
        "emu_vs_ref_max_abs_late": float(np.abs(emu - ref)[late].max()) if late.any() else 0.0,
        "kernel_vs_ref_max_abs_late": float(np.abs(got - ref)[late].max()) if late.any() else 0.0,
    }


def split_line(tag: str, s: dict) -> str:
    return (f"[record] {tag}: {len(s['rows'])} sampled rows; kernel vs emulation max_abs="
            f"{s['kernel_vs_emu_max_abs']:.3e} worst e/bound={s['ratio']:.3f} (beyond the output rounding: "
            f"max_abs={s['arith_max_abs']:.3e} worst {s['arith_ratio']:.3f}; equal to the emulation rounded to "
            f"the output type: {100 * s['eq_rounded']:.2f} %); emulation vs fp32 ref "
            f"max_abs={s['emu_vs_ref_max_abs']:.3e} (rows>=128 {s['emu_vs_ref_max_abs_late']:.3e}) "
            f"cos={s['emu_vs_ref_cos']:.6f}; kernel vs fp32 ref max_abs={s['kernel_vs_ref_max_abs']:.3e} "
            f"(rows>=128 {s['kernel_vs_ref_max_abs_late']:.3e}) cos={s['kernel_vs_ref_cos']:.6f}")
