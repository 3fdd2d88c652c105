"""Pins of the CPU oracle (oracle/sage_oracle.py) — no GPU.

The reference ships no golden vectors for this path, so each oracle function
is pinned by what fixes it independently of its own formula:

* quantization (triton_impl.py:25-33): hand-built blocks with known answers,
  the fp32 rounding quirk at 0x3EFFFFFF, invariants (|q8| <= 127, every
  nonzero block reaches +-127, |q8*scale - x| <= scale/2 up to the rounding
  of scale), an element-by-element restatement with Python scalars, and
  exactness on inputs that lie on the quantization grid;
* K channel mean: an independent pure-Python loop in the documented order,
  and the fp64 mean;
* FP8 e4m3: torch.float8_e4m3fn (the library definition of OCP e4m3) on a
  dense sweep and on every rounding boundary;
* SDPA (reference.py:15-24): torch.nn.functional.scaled_dot_product_attention,
  fp64 brute force, causal row 0 = v[0], uniform scores = mean(v), GQA =
  MHA after repeat_interleave;
* SageAttention emulation: equals SDPA when quantization is exact;
* work formulas: the ops and pre-pass bytes of the benchmark configurations
  (config 2: 2^40 ops and 402.8 MB; config 3: 2^43 metric, 4.398e12
  algorithmic ops; config 4: 7.766e12; config 5: 1208.1 MB).
"""
from __future__ import annotations

import math
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def f32(bits: int) -> np.float32:
    return np.uint32(bits).view(np.float32)


# ---------------------------------------------------------------------------
# quantization
# ---------------------------------------------------------------------------

def test_q_multiplier_constants():
    # fp32(D**-0.5 * 1.44269504) as triton_impl.py:60-61,69 passes it
    assert O.q_multiplier(128).view(np.uint32) == 0x3E0293EE
    assert O.q_multiplier(64).view(np.uint32) == 0x3E38AA3B
    assert O.q_multiplier(64, sm_scale=0.5) == np.float32(0.5 * 1.44269504)


def test_quant_known_block():
    x = np.zeros((1, 1, 64, 64), np.float32)
    vals = [127.0, 0.5, -0.5, 1.5, -2.5, f32(0x3EFFFFFF), -f32(0x3EFFFFFF), -0.0, 1e-30, -126.5, 63.49, -63.5]
    x[0, 0, 0, :len(vals)] = vals
    q8, sc = O.quant_per_block_int8(x, 64)
    assert sc.shape == (1, 1, 1) and sc[0, 0, 0] == np.float32(1.0)
    # ties go away from zero; 0.49999997 + 0.5 rounds to 1.0 in fp32 -> 1
    assert list(q8[0, 0, 0, :len(vals)]) == [127, 1, -1, 2, -3, 1, -1, 0, 0, -127, 63, -64]


def test_quant_all_zero_and_tail_blocks():
    x = np.zeros((1, 1, 100, 16), np.float32)
    x[0, 0, 64:100] = np.arange(36 * 16, dtype=np.float32).reshape(36, 16) - 100
    q8, sc = O.quant_per_block_int8(x, 64)
    assert sc.shape == (1, 1, 2)
    assert sc[0, 0, 0] == 0 and not q8[0, 0, :64].any()  # all-zero block: scale 0, q 0 (build-defined)
    amax = np.abs(x[0, 0, 64:]).max()
    assert sc[0, 0, 1] == np.float32(amax) / np.float32(127)
    assert q8.shape == x.shape


def _quant_scalar(xs, mul=None):
    """Element-by-element restatement with numpy fp32 scalars (one block)."""
    xs = [np.float32(v) for v in xs]
    if mul is not None:
        xs = [np.float32(v * np.float32(mul)) for v in xs]
    amax = max(abs(v) for v in xs)
    scale = np.float32(amax / np.float32(127.0))
    out = []
    for v in xs:
        t = np.float32(v / scale) if scale > 0 else np.float32(0)
        u = np.float32(t + (np.float32(0.5) if t >= 0 else np.float32(-0.5)))
        out.append(int(math.trunc(float(u))))
    return out, scale


@pytest.mark.parametrize("seed", range(5))
def test_quant_matches_scalar_restatement(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((1, 1, 128, 16)) * rng.uniform(0.01, 100)).astype(np.float32)
    mul = O.q_multiplier(16)
    q8, sc = O.quant_per_block_int8(x, 128, mul=mul)
    want, scale = _quant_scalar(x.ravel(), mul)
    assert sc[0, 0, 0] == scale
    assert q8.ravel().tolist() == want


def test_quant_invariants_and_error_bound():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((2, 3, 300, 64)) * 3 + rng.standard_normal((2, 3, 1, 64))).astype(np.float32)
    for blk, q_sub in ((128, 128), (128, 32), (64, 64), (128, 1)):
        q8, sc = O.quant_per_block_int8(x, blk, q_sub=q_sub)
        assert np.abs(q8.astype(np.int32)).max() <= 127
        nsub = sc.shape[-1]
        pad = np.zeros((2, 3, nsub * q_sub, 64), np.int8)
        pad[:, :, :300] = q8
        per = np.abs(pad.reshape(2, 3, nsub, -1).astype(np.int32)).max(-1)
        assert np.all(per[sc > 0] == 127)  # every nonzero (sub-)block reaches +-127
        s_rows = np.repeat(sc, q_sub, axis=-1)[:, :, :300, None].astype(np.float64)
        err = np.abs(q8 * s_rows - x)
        assert np.all(err <= s_rows * 0.5 * (1 + 2.0 ** -20) + 1e-38)


def test_quant_per_row_is_blocks_of_one_row():
    """One scale per row (q_sub = 1) inside 128-row blocks is the same
    quantization as blocks of a single row, and padded rows get scale 0."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((2, 3, 300, 64)) * 2 + rng.standard_normal((2, 3, 300, 1)) * 5).astype(np.float32)
    mul = O.q_multiplier(64)
    q8, sc = O.quant_per_block_int8(x, 128, mul=mul, q_sub=1)
    q8r, scr = O.quant_per_block_int8(x, 1, mul=mul)
    assert np.array_equal(q8, q8r)
    assert sc.shape == (2, 3, 384) and np.array_equal(sc[:, :, :300], scr) and np.all(sc[:, :, 300:] == 0)
    # a row's scale is its own max|x * mul| / 127, independent of the other rows
    xm = (x.astype(np.float32) * mul).astype(np.float32)
    assert np.array_equal(sc[:, :, :300], (np.abs(xm).max(-1) / np.float32(127)).astype(np.float32))


def test_quant_exact_on_grid():
    # values already on the quantization grid round-trip exactly
    rng = np.random.default_rng(3)
    ints = rng.integers(-127, 128, size=(1, 2, 64, 32)).astype(np.float32)
    ints[:, :, 0, 0] = 127
    step = np.float32(0.25)
    q8, sc = O.quant_per_block_int8(ints * step, 64)
    assert np.all(sc == step) and np.array_equal(q8, ints.astype(np.int8))


# ---------------------------------------------------------------------------
# K channel mean
# ---------------------------------------------------------------------------

def _kmean_loops(k):
    """The documented order, in plain Python loops over numpy fp32 scalars."""
    B, H, N, D = k.shape
    TL = 256 // (D // 8)
    ch = 256 * ((N + 4095) // 4096)
    km = np.zeros((B, H, D), np.float32)
    for b in range(B):
        for h in range(H):
            for c in range(D):
                total = None
                for n0 in range(0, N, ch):
                    n1 = min(n0 + ch, N)
                    lanes = []
                    for tl in range(TL):
                        acc = np.float32(0)
                        for n in range(n0 + tl, n1, TL):
                            acc = np.float32(acc + k[b, h, n, c])
                        lanes.append(acc)
                    s = TL
                    while s > 1:
                        s //= 2
                        lanes = [np.float32(lanes[i] + lanes[i + s]) for i in range(s)]
                    total = lanes[0] if total is None else np.float32(total + lanes[0])
                km[b, h, c] = np.float32(total / np.float32(N))
    return km


@pytest.mark.parametrize("N,D", [(300, 64), (4500, 128)])
def test_k_channel_mean_order(N, D):
    rng = np.random.default_rng(N)
    k = (rng.standard_normal((1, 1, N, D)) * 5 + 3).astype(np.float32)
    km = O.k_channel_mean(k)
    cols = slice(0, 8)  # a few channels through the slow loop
    assert np.array_equal(km[..., cols], _kmean_loops(k[..., cols].copy())[..., :8] if D == 8 else
                          _kmean_loops(np.ascontiguousarray(k))[..., cols])
    assert np.allclose(km, k.astype(np.float64).mean(2), rtol=0, atol=1e-5)


def test_k_chunking():
    assert O.kstat_chunk_tokens(256) == 256 and O.kstat_chunk_tokens(4096) == 256
    assert O.kstat_chunk_tokens(4097) == 512 and O.kstat_chunk_tokens(32768) == 2048
    for n in (1, 255, 4096, 17776, 32768, 100000):
        ch = O.kstat_chunk_tokens(n)
        assert -(-n // ch) <= 16 and ch % 256 == 0
    assert O.kstat_token_lanes(128) == 16 and O.kstat_token_lanes(64) == 32


# ---------------------------------------------------------------------------
# FP8 e4m3
# ---------------------------------------------------------------------------

def _torch_e4m3(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_matches_torch_dense_sweep():
    # every 97th fp32 bit pattern from 0 up to 464 (torch saturates to 448 below that and
    # returns NaN above it; the pre-pass never exceeds 448*(1+2^-23)), both signs
    hi = int(np.float32(464.0).view(np.uint32))
    bits = np.arange(0, hi + 1, 97, dtype=np.uint32)
    x = bits.view(np.float32)
    for sgn in (1, -1):
        xs = (x * sgn).astype(np.float32)
        assert np.array_equal(O.e4m3_encode(xs), _torch_e4m3(xs))


def test_e4m3_rounding_boundaries():
    # midpoints between consecutive codes and their fp32 neighbours
    vals = O.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    xs = []
    for m in mids:
        f = np.float32(m)
        xs += [f, np.nextafter(f, np.float32(0)), np.nextafter(f, np.float32(1000))]
    xs = np.array(xs, np.float32)
    assert np.array_equal(O.e4m3_encode(xs), _torch_e4m3(xs))
    assert O.e4m3_encode(np.array([448.0, 460.0, 1e30, np.inf], np.float32)).tolist() == [0x7E] * 4
    assert O.e4m3_encode(np.array([np.nan], np.float32))[0] == 0x7F
    assert np.array_equal(O.e4m3_decode(O.e4m3_encode(vals.astype(np.float32))), vals.astype(np.float32))


def test_quant_v_fp8_golden():
    g = np.load(GOLDEN / "sage_fp8v.npz")
    v8, vs = O.quant_v_fp8(g["v"])
    assert np.array_equal(v8, g["v8"]) and np.array_equal(vs, g["v_scale"])
    # codes equal torch's cast of v / v_scale
    t = (g["v"] / g["v_scale"][:, :, None, :]).astype(np.float32)
    assert np.array_equal(v8, _torch_e4m3(t))
    assert (O.e4m3_decode(v8) == 448).any() or (O.e4m3_decode(v8) == -448).any()


# ---------------------------------------------------------------------------
# SDPA and the SageAttention emulation
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_vs_torch(causal):
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(2, 3, 70, 32, generator=g, dtype=torch.float64) for _ in range(3))
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal).numpy()
    got = O.sdpa(q.numpy(), k.numpy(), v.numpy(), causal=causal, q_chunk=16)
    assert np.abs(got - want).max() < 1e-12


def test_sdpa_brute_force_and_special_cases():
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((1, 1, 5, 4)) for _ in range(3))
    got = O.sdpa(q, k, v, causal=True)
    for i in range(5):
        s = [float(q[0, 0, i] @ k[0, 0, j]) / 2.0 for j in range(i + 1)]
        w = [math.exp(x - max(s)) for x in s]
        o = sum(wj * v[0, 0, j] for j, wj in enumerate(w)) / sum(w)
        assert np.allclose(got[0, 0, i], o, atol=1e-14)
    assert np.allclose(got[0, 0, 0], v[0, 0, 0])  # causal row 0 is v[0]
    zq = np.zeros_like(q)
    assert np.allclose(O.sdpa(zq, k, v)[0, 0], v[0, 0].mean(0))  # uniform scores


def test_sdpa_gqa_equals_repeat():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 6, 20, 16))
    k, v = rng.standard_normal((1, 2, 20, 16)), rng.standard_normal((1, 2, 20, 16))
    a = O.sdpa(q, k, v, causal=True)
    b = O.sdpa(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1), causal=True)
    assert np.array_equal(a, b)


def test_emulation_is_base2_sdpa_of_dequantized_inputs():
    """The emulation's scores are q8.k8 * q_scale * k_scale in log2 units
    (log2 e is folded into q_scale, triton_impl.py:69, :99-104): it must equal
    natural-base SDPA of the dequantized q and k with scale ln 2, per-block
    and per-sub-block scale indexing included."""
    rng = np.random.default_rng(9)
    B, Hq, Hkv, N, D = 1, 4, 2, 200, 64
    q = rng.standard_normal((B, Hq, N, D)).astype(np.float32)
    k = (rng.standard_normal((B, Hkv, N, D)) + 2).astype(np.float32)
    v = rng.standard_normal((B, Hkv, N, D))
    for q_sub in (128, 32, 1):
        q8, qs = O.quant_per_block_int8(q, 128, mul=O.q_multiplier(D), q_sub=q_sub)
        k8, ks = O.quant_per_block_int8(k, 64)
        qd = q8 * np.repeat(qs, q_sub, axis=-1)[:, :, :N, None].astype(np.float64)
        kd = k8 * np.repeat(ks, 64, axis=-1)[:, :, :N, None].astype(np.float64)
        for causal in (False, True):
            emu = O.sage_emulate(q8, qs, k8, ks, v, causal=causal, q_sub=q_sub)
            ref = O.sdpa(qd, kd, v, causal=causal, sm_scale=math.log(2))
            assert np.abs(emu - ref).max() < 1e-12


def test_row_subsets_equal_the_full_result():
    """``rows=`` (the sampled-row checks at full size) picks the same rows as
    the full computation, in the given order, causal and GQA included, with
    the FP8-code form of V too (to rounding: BLAS may sum a product of
    another shape in another order; a wrong row is off by O(1))."""
    rng = np.random.default_rng(11)
    B, Hq, Hkv, N, D = 2, 4, 2, 150, 32
    q = rng.standard_normal((B, Hq, N, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    rows = np.array([149, 0, 3, 64, 127, 128, 77])
    q8, qs = O.quant_per_block_int8(q, 128, mul=O.q_multiplier(D), q_sub=32)
    k8, ks = O.quant_per_block_int8(k, 64)
    codes, vs = O.quant_v_fp8(v)
    for causal in (False, True):
        full = O.sdpa(q, k, v, causal=causal, q_chunk=16)
        assert np.abs(O.sdpa(q, k, v, causal=causal, q_chunk=16, rows=rows) - full[:, :, rows]).max() < 1e-12
        for vv, vsc in ((v, None), (codes, vs)):
            e = O.sage_emulate(q8, qs, k8, ks, vv, causal=causal, q_sub=32, v_scale=vsc, q_chunk=16)
            er = O.sage_emulate(q8, qs, k8, ks, vv, causal=causal, q_sub=32, v_scale=vsc, q_chunk=4, rows=rows)
            assert np.abs(er - e[:, :, rows]).max() < 1e-12


# ---------------------------------------------------------------------------
# fixtures and work formulas
# ---------------------------------------------------------------------------

def test_golden_cfg1_regression():
    g = np.load(GOLDEN / "sage_cfg1.npz")
    pre = O.prepass(g["q"], g["k"], smooth_k=True)
    for key in ("q8", "q_scale", "k8", "k_scale", "km"):
        assert np.array_equal(pre[key], g[key]), key
    for causal, tag in ((False, "full"), (True, "causal")):
        assert np.abs(O.sdpa(g["q"], g["k"], g["v"], causal=causal) - g[f"o_sdpa_{tag}"]).max() < 1e-6
        emu = O.sage_emulate(g["q8"], g["q_scale"], g["k8"], g["k_scale"], g["v"], causal=causal)
        assert np.abs(emu - g[f"o_emul_{tag}"]).max() < 1e-6
    # the quantization error of config 1 against SDPA (north-star bounds hold non-causal)
    err = np.abs(g["o_emul_full"] - g["o_sdpa_full"]).max()
    assert err <= 2e-2


def test_golden_inputs_match_pack_generator(pack_ref):
    g = np.load(GOLDEN / "sage_cfg1.npz")
    inp = pack_ref.make_inputs(dict(batch_size=1, num_heads=2, seq_len=256, head_dim=64, k_offset_std=2.0),
                               "cpu", 0, torch.float32)
    for x in ("q", "k", "v"):
        assert np.array_equal(inp[x].numpy(), g[x])


def test_work_formulas_at_the_benchmark_configurations():
    assert O.attention_flops(4, 32, 4096, 4096, 128) == (2 ** 40, 2 ** 40)
    m, a = O.attention_flops(2, 32, 16384, 16384, 128, causal=True)
    assert m == 2 ** 43 and abs(a / 4.398e12 - 1) < 1e-3
    assert abs(O.attention_flops(2, 48, 17776, 17776, 64)[0] / 7.766e12 - 1) < 1e-3
    assert abs(O.prepass_bytes(4, 32, 32, 4096, 4096, 128) / 402.8e6 - 1) < 1e-3
    assert abs(O.prepass_bytes(2, 32, 32, 16384, 16384, 128) / 805.4e6 - 1) < 1e-3
    assert abs(O.prepass_bytes(2, 48, 8, 17776, 17776, 64) / 382.3e6 - 1) < 1e-3
    b5 = O.prepass_bytes(1, 32, 32, 32768, 32768, 128, q_sub=32, v_fp8=True)
    assert abs(b5 / 1208.1e6 - 1) < 2e-3
    assert O.unmasked_pairs(5, 5, True) == 15 and O.unmasked_pairs(3, 5, True) == 6


def test_float32_struct_helper():
    assert struct.unpack("<f", struct.pack("<I", 0x3F800000))[0] == 1.0


def test_vtile_layout_round_trip_and_positions():
    """The V tile layout: positions are a permutation, every lane half holds
    its 32 keys contiguously, and the tiles decode back to the input with
    zeros past N."""
    pos = O.vtile_positions()
    assert sorted(pos.tolist()) == list(range(64))
    # register v of key tile t in lane half h holds key 32t + 8(v//4) + 4h + v%4 at column 32h + 16t + v
    for t in range(2):
        for h in range(2):
            for v in range(16):
                assert pos[32 * t + 8 * (v // 4) + 4 * h + v % 4] == 32 * h + 16 * t + v
    x = np.arange(2 * 3 * 130 * 8, dtype=np.float32).reshape(2, 3, 130, 8) + 1
    t = O.vtiles(x)
    assert t.shape == (2, 3, 3, 8, 64)
    back = np.zeros((2, 3, 192, 8), np.float32)
    for k in range(64):
        back[:, :, k::64, :][:, :, :3] = t[..., pos[k]]
    assert np.array_equal(back[:, :, :130], x) and not back[:, :, 130:].any()
