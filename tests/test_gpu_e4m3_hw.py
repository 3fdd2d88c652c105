"""gfx950's fp32 -> FP8 e4m3 conversion instruction against the pre-pass's own
encoder, over all 2^32 fp32 inputs (tests/native/e4m3_hw_check.hip, built by
__graft_entry__.build()).  The V tiles and FP8 V rows use the instruction on
quotients v / v_scale, all of magnitude <= 448 * (1 + 2^-23): it must agree
there bit for bit (class 0) and up to 464 (class 1), where RNE still lands on
448.  Beyond 464 the instruction gives NaN codes where the encoder saturates,
and NaN inputs get another NaN code; the kernels never produce either
(NaN in V is outside the oracle's domain: its v_scale is NaN there)."""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parents[1] / "tribench_amd" / "lib" / "e4m3_hw_check"


def test_packed_e4m3_conversion_matches_the_encoder(gpu_device):
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built (run __graft_entry__.build())")
    print("[e4m3-hw] all 2^32 fp32 patterns", flush=True)
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    rec = json.loads(res.stdout.strip().splitlines()[-1])
    print(f"[record] e4m3 hw check {rec}", flush=True)
    assert sum(rec["patterns"]) == 1 << 32
    assert rec["patterns"][0] > 2_000_000_000
    assert rec["mismatches"][0] == 0 and rec["mismatches"][1] == 0, rec
