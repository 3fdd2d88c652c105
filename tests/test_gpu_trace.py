"""The phase-trace build on the GPU: same results as the product library, and sane stamps.

The trace library (``python -m tribench_amd.build --trace``, SAGE_TRACE=2)
adds s_memtime stamps and barrier counters to the attention kernel.  On a
small causal GQA case with a ragged tail and on a non-causal one, through
``hip_impl.run``: the output equals the product library's bit for bit, every
wave writes its record, the phase stamps of each wave are in order, each
wave meets exactly as many barriers as its work-group runs iterations plus
one (the prologue's), and the record's work-group index is a permutation
of the grid.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tribench_amd import trace_phases as tp

pytestmark = pytest.mark.gpu

CASES = [
    dict(batch_size=1, num_heads=4, num_kv_heads=2, seq_len=1000, head_dim=128, k_offset_std=2.0, causal=True),
    dict(batch_size=2, num_heads=2, seq_len=700, head_dim=64, k_offset_std=2.0),
]


@pytest.mark.skipif(not tp.TRACE_LIB.is_file(), reason="trace library not built (build --trace)")
@pytest.mark.parametrize("case", CASES, ids=["causal_gqa_d128", "d64"])
def test_trace_build_matches_product(case, gpu_device):
    print(f"[trace] {case}", flush=True)
    prod = tp._load("hip_impl", tp.PRODUCT_LIB)
    trc = tp._load("hip_impl", tp.TRACE_LIB)
    R = tp._load("reference", tp.PRODUCT_LIB)
    inp = R.make_inputs(case, "cpu", 0, torch.bfloat16)
    q, k, v = (inp[x].to(gpu_device) for x in ("q", "k", "v"))
    causal = bool(case.get("causal", False))
    B, Hq, N, D = q.shape
    grid = ((N + 255) // 256) * Hq * B
    buf = torch.zeros(grid * tp.NW * tp.WORDS, dtype=torch.int64, device=gpu_device)
    attach = trc._load().sage_trace_attach
    attach.argtypes, attach.restype = [ctypes.c_void_p, ctypes.c_int64], ctypes.c_int
    want = prod.run(q, k, v, causal=causal)
    assert attach(ctypes.c_void_p(buf.data_ptr()), buf.numel()) == 0
    try:
        got = trc.run(q, k, v, causal=causal)
        torch.cuda.synchronize()
    finally:
        attach(None, 0)
    assert torch.equal(got, want)
    T = buf.cpu().numpy().view(np.uint64).reshape(grid, tp.NW, tp.WORDS)
    assert (T[:, :, 5] > 0).all(), "a wave wrote no record"
    t = T[:, :, :6].astype(np.int64)
    assert (np.diff(t, axis=2) >= 0).all(), "phase stamps out of order"
    # barriers: the prologue's one plus one per iteration j = 0 .. nkb
    n_all = (T[:, :, 8] & 0xFFFFFFFF).astype(np.int64)
    assert (n_all == n_all[:, :1]).all(), "waves of one work-group met different barrier counts"
    nqb = (N + 255) // 256
    wg = T[:, 0, 12].astype(np.int64)
    assert sorted(wg.tolist()) == list(range(grid))
    for g in range(grid):
        if causal:  # the q-block this work-group ran, from its barrier count
            nkb = int(n_all[g, 0]) - 2
            assert 1 <= nkb <= (N + 63) // 64
        else:
            assert n_all[g, 0] == (N + 63) // 64 + 2
    assert nqb >= 1
