"""The C-ABI library on a host without a GPU: it loads, exports every symbol
of include/sage_attn.h, and rejects bad arguments before touching a device."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sage_attn.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sage_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib(hip_impl):
    return hip_impl._load()


def test_header_declares_the_entry_points():
    assert _declared_functions() == ["sage_abi_version", "sage_attn_fwd", "sage_attn_fwd_q", "sage_flash_fwd",
                                     "sage_last_error", "sage_prepass", "sage_prepass_vt",
                                     "sage_prepass_vt_noalloc", "sage_prepass_workspace_bytes",
                                     "sage_vtile_bytes", "sage_vtiles"]


def _declared_arg_counts():
    """Parameter count of every function declared in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(sage_[a-z_0-9]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_bindings_match_the_header_argument_counts(lib):
    """hip_impl binds every entry point with exactly the header's number of
    parameters: a signature change on one side without the other fails here
    instead of passing garbage through ctypes."""
    counts = _declared_arg_counts()
    assert set(counts) == set(_declared_functions())
    for name, n in counts.items():
        fn = getattr(lib, name)
        assert fn.argtypes is not None, name
        assert len(fn.argtypes) == n, f"{name}: header {n} parameters, binding {len(fn.argtypes)}"


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_matches_header(lib, hip_impl):
    m = re.search(r"#define SAGE_ABI_VERSION (\d+)", HEADER.read_text())
    assert lib.sage_abi_version() == int(m.group(1)) == hip_impl.ABI_VERSION


def test_workspace_bytes(lib):
    # smooth_k: B*Hkv*nch*D fp32 partial sums; FP8 V adds as many channel maxima
    nch = 16  # N = 4096 -> 16 chunks of 256 tokens
    assert lib.sage_prepass_workspace_bytes(4, 32, 4096, 128, 1, 0) == 4 * 32 * nch * 128 * 4
    assert lib.sage_prepass_workspace_bytes(4, 32, 4096, 128, 1, 1) == 2 * 4 * 32 * nch * 128 * 4
    assert lib.sage_prepass_workspace_bytes(4, 32, 4096, 128, 0, 0) == 0


def test_noalloc_prepass_rejects_before_touching_a_device(lib):
    """The fixed-scratch pre-pass checks its size limit (and a null V tile
    buffer) before any HIP call."""
    m = re.search(r"#define SAGE_SCRATCH_BYTES \((\d+)u << (\d+)\)", HEADER.read_text())
    limit = int(m.group(1)) << int(m.group(2))
    assert limit == 4 << 20
    a = _prepass_args(B=16, Hq=64, Hkv=64, Nq=4096, Nkv=4096, D=128, smooth=1, km=ctypes.c_void_p(16))
    assert lib.sage_prepass_workspace_bytes(16, 64, 4096, 128, 1, 0) > limit
    fn = lib.sage_prepass_vt_noalloc
    rc = fn(*a[:-3], 0, ctypes.c_void_p(16), ctypes.c_size_t(1 << 30), None)
    msg = lib.sage_last_error().decode()
    assert rc != 0 and "invalid argument" in msg and "scratch" in msg, msg
    rc = fn(*_prepass_args()[:-3], 0, None, ctypes.c_size_t(0), None)
    msg = lib.sage_last_error().decode()
    assert rc != 0 and "invalid argument" in msg and "vtiles" in msg, msg


def _prepass_args(**over):
    s3 = (ctypes.c_int64 * 3)(0, 0, 0)
    a = dict(q=ctypes.c_void_p(16), k=ctypes.c_void_p(16), v=None, in_dtype=2, B=1, Hq=2, Hkv=2, Nq=64, Nkv=64,
             D=64, qs=s3, ks=s3, vs=None, mul=0.18, blkq=128, blkk=64, q_sub=128, smooth=0, vmode=0,
             q8=ctypes.c_void_p(16), q8s=s3, qsc=ctypes.c_void_p(16), k8=ctypes.c_void_p(16), k8s=s3,
             ksc=ctypes.c_void_p(16), km=None, v8=None, v8s=None, vsc=None, ws=None, wsb=0, st=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,needle", [
    (dict(D=96), "head_dim"),
    (dict(Hq=3, Hkv=2), "multiple"),
    (dict(B=0), "empty shape"),
    (dict(blkq=100), "blkq"),
    (dict(q_sub=48), "q_sub"),
    (dict(q_sub=2), "q_sub"),
    (dict(q_sub=0), "q_sub"),
    (dict(in_dtype=7), "in_dtype"),
    (dict(smooth=1), "km is null"),
    (dict(q=None), "null pointer"),
    (dict(q=ctypes.c_void_p(8)), "aligned"),
    (dict(q=None, qs=None, q8s=None, qsc=None), "null pointer"),  # q8 given without q
])
def test_prepass_rejects_bad_arguments(lib, over, needle):
    rc = lib.sage_prepass(*_prepass_args(**over))
    msg = lib.sage_last_error().decode()
    assert rc != 0 and "invalid argument" in msg and needle in msg, msg


@pytest.mark.parametrize("over,vt_over,needle", [
    ({}, dict(pv=7), "pv_mode"),
    ({}, dict(pv=2), "FP8 V tiles need v_mode"),          # FP8 tiles without v_scale
    ({}, dict(vt=None), "null pointer"),
    (dict(v=None), {}, "null V pointer"),
    ({}, dict(vtb=1000), "vtiles"),                       # 1000 < 2*64*64*2 bytes
    ({}, dict(vt=ctypes.c_void_p(24)), "aligned"),
    (dict(q_sub=2), {}, "q_sub"),                         # the pre-pass's own checks still apply
])
def test_prepass_vt_rejects_bad_arguments(lib, over, vt_over, needle):
    s3 = (ctypes.c_int64 * 3)(0, 0, 0)
    base = dict(v=ctypes.c_void_p(16), vs=s3)
    base.update(over)
    tail = dict(pv=0, vt=ctypes.c_void_p(16), vtb=1 << 20, st=None)
    tail.update(vt_over)
    args = _prepass_args(**base)[:-1] + list(tail.values())
    rc = lib.sage_prepass_vt(*args)
    msg = lib.sage_last_error().decode()
    assert rc != 0 and "invalid argument" in msg and needle in msg and "sage_prepass_vt" in msg, msg


def test_attn_rejects_bad_arguments(lib):
    s3 = (ctypes.c_int64 * 3)(0, 0, 0)
    p = ctypes.c_void_p(16)
    rc = lib.sage_attn_fwd(p, s3, p, p, s3, p, p, 2, s3, None, p, 2, s3, 1, 2, 2, 64, 64, 64, 0, 128, 32, 128, 0,
                           None)
    assert rc != 0 and "blkk" in lib.sage_last_error().decode()
    rc = lib.sage_attn_fwd(p, s3, p, p, s3, p, p, 2, s3, None, p, 1, s3, 1, 2, 2, 64, 64, 64, 0, 128, 64, 128, 0,
                           None)
    assert rc != 0 and "v_dtype" in lib.sage_last_error().decode()


def test_vtile_bytes_and_rejections(lib):
    # tiles of 64 keys (ragged N rounded up), 2 bytes per element for fp16/bf16, 1 for e4m3
    assert lib.sage_vtile_bytes(4, 32, 4096, 128, 0) == 4 * 32 * 64 * 128 * 64 * 2
    assert lib.sage_vtile_bytes(2, 8, 17776, 64, 1) == 2 * 8 * 278 * 64 * 64 * 2
    assert lib.sage_vtile_bytes(1, 32, 32768, 128, 2) == 32 * 512 * 128 * 64
    assert lib.sage_prepass_workspace_bytes(4, 32, 4096, 128, 0, 2) == 4 * 32 * 16 * 128 * 4
    s3 = (ctypes.c_int64 * 3)(0, 0, 0)
    p = ctypes.c_void_p(16)
    big = ctypes.c_size_t(1 << 40)
    for args, needle in [
        ((p, 2, 1, 2, 64, 96, s3, 0, None, p, big, None), "head_dim"),
        ((p, 2, 1, 2, 64, 64, s3, 2, None, p, big, None), "null"),
        ((p, 2, 1, 2, 64, 64, s3, 5, None, p, big, None), "pv_mode"),
        ((p, 2, 1, 2, 64, 64, s3, 0, None, p, ctypes.c_size_t(64), None), "out"),
    ]:
        rc = lib.sage_vtiles(*args)
        msg = lib.sage_last_error().decode()
        assert rc != 0 and "invalid argument" in msg and needle in msg, msg


def test_library_override_must_exist(hip_impl, monkeypatch, tmp_path):
    """$TRIBENCH_SAGE_HIP_LIB naming no file is an error, not a silent fall
    back to the in-tree library; naming a file selects it."""
    missing = tmp_path / "no_such_lib.so"
    monkeypatch.setenv("TRIBENCH_SAGE_HIP_LIB", str(missing))
    with pytest.raises(RuntimeError, match="is not a file"):
        hip_impl.library_path()
    monkeypatch.delenv("TRIBENCH_SAGE_HIP_LIB")
    default = hip_impl.library_path()
    monkeypatch.setenv("TRIBENCH_SAGE_HIP_LIB", str(default))
    assert hip_impl.library_path() == default


def test_hip_variant_refuses_cpu_tensors(hip_impl):
    import torch

    q = torch.zeros(1, 2, 16, 64)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        hip_impl.run(q, q, q)


def test_flash_rejects_bad_arguments(lib):
    s3 = (ctypes.c_int64 * 3)(0, 0, 0)
    p = ctypes.c_void_p(16)
    for args, needle in [
        ((p, s3, p, s3, p, 4, None, p, s3, 1, 1, 2, 2, 64, 64, 96, 0.18, 0, None), "head_dim"),
        ((p, s3, p, s3, p, 4, None, p, s3, 0, 1, 2, 2, 64, 64, 64, 0.18, 0, None), "in_dtype"),
        ((p, s3, p, s3, p, 2, None, p, s3, 2, 1, 2, 2, 64, 64, 64, 0.18, 0, None), "v_dtype"),
        ((p, s3, p, s3, p, 4, None, p, s3, 2, 1, 3, 2, 64, 64, 64, 0.18, 0, None), "Hq"),
        ((p, s3, p, s3, p, 4, None, p, s3, 2, 1, 2, 2, 64, 64, 64, 0.0, 0, None), "qk_mul"),
        ((None, s3, p, s3, p, 4, None, p, s3, 2, 1, 2, 2, 64, 64, 64, 0.18, 0, None), "null"),
        ((ctypes.c_void_p(8), s3, p, s3, p, 4, None, p, s3, 2, 1, 2, 2, 64, 64, 64, 0.18, 0, None), "aligned"),
    ]:
        rc = lib.sage_flash_fwd(*args)
        msg = lib.sage_last_error().decode()
        assert rc != 0 and "invalid argument" in msg and needle in msg, msg


def test_attn_fwd_q_rejects_bad_arguments(lib):
    s3 = (ctypes.c_int64 * 3)(0, 0, 0)
    p = ctypes.c_void_p(16)
    base = dict(q=p, qs=s3, qdt=2, qmul=0.18, q8o=None, qso=None, k8=p, k8s=s3, ksc=p, v=p, vdt=4, vs=None,
                vsc=None, o=p, os=s3, B=1, Hq=2, Hkv=2, Nq=64, Nkv=64, D=64, causal=0, blkq=128, blkk=64,
                q_sub=128, pv=0, st=None)
    for over, needle in [
        (dict(blkq=64, q_sub=64), "blkq"),
        (dict(q_sub=48), "q_sub"),
        (dict(q_sub=2), "q_sub"),
        (dict(qdt=9), "q_dtype"),
        (dict(qmul=-1.0), "q_mul"),
        (dict(vdt=2), "v_dtype"),
        (dict(q=None), "null"),
        (dict(D=96), "head_dim"),
        (dict(q8o=ctypes.c_void_p(8)), "aligned"),
    ]:
        a = dict(base)
        a.update(over)
        rc = lib.sage_attn_fwd_q(*a.values())
        msg = lib.sage_last_error().decode()
        assert rc != 0 and "invalid argument" in msg and needle in msg, msg
