"""The pre-pass element arithmetic, compiled for the host and checked (no GPU).

tests/native/quant_math_check.cpp includes tribench_amd/csrc/sage_quant_math.h
— the same text the gfx950 kernels compile — and compares it against IEEE
arithmetic: Markstein's division (sage::div_rn) and the reference rounding
(triton_impl.py:29-31) exhaustively over the binades where int8 rounding
happens, plus random scales across the fast-path range; the FP8 e4m3
encoder against the numpy oracle (itself pinned to torch.float8_e4m3fn); and
the FP8 V path's quotient (div_rn_signed, which keeps -0) against IEEE
division, through the encoder, for every 16-bit input per scale.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import sage_oracle as O

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("qmc") / "quant_math_check"
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(HERE / "native" / "quant_math_check.cpp")], check=True)
    return exe


def _run(exe, *args, timeout=300):
    res = subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True, timeout=timeout)
    assert res.returncode == 0 and res.stdout.startswith("OK"), res.stdout + res.stderr
    return int(res.stdout.split()[1])


@pytest.mark.parametrize("scale_bits", ["3c010204", "3d8f5c29"])
def test_div_and_rounding_exhaustive_top_binades(checker, scale_bits):
    # every x with scale/256 <= |x| <= 127.5*scale, both signs
    assert _run(checker, "div", scale_bits, -8) > 1e8


def test_div_and_rounding_random_scales(checker):
    assert _run(checker, "divrand", 4000, 5000) == 20_000_000


def test_e4m3_encoder_matches_oracle(checker, tmp_path):
    out = tmp_path / "codes.bin"
    stride = 4099
    n = _run(checker, "e4m3", stride, out)
    codes = np.fromfile(out, dtype=np.uint8).reshape(-1, 2)
    assert codes.shape[0] == n
    bits = np.arange(0, 0x7F800001, stride, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    assert np.array_equal(codes[:, 0], O.e4m3_encode(x))
    assert np.array_equal(codes[:, 1], O.e4m3_encode(-x))


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_fp8_division_16bit_inputs(checker, dtype):
    # every x of the type against every 17th amax (the full sweep, stride 1:
    # 889,737,154 bf16 and 1,007,713,278 fp16 pairs, passes as well)
    assert _run(checker, "fp8div", dtype, 17) > 4e7


def test_fp8_division_random_fp32(checker):
    assert _run(checker, "fp8divrand", 2000, 20000) > 3e7
