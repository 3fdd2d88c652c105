"""The harness around the hot path, on the CPU: schema, pack index, case
grid, inputs, reference, correctness gate, timers, metrics, CLI and outputs.

The schema cases cover what the reference's tests/test_meta_schema.py
(:12-134) checks of a meta.json; the CLI failure handling is forced from the
host with fake packs (an impl that raises, an impl that returns wrong
values), as the reference's CLI handles them (cli.py:313-339).
"""
from __future__ import annotations

import copy
import json
import math
import textwrap
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O
from tribench_amd.harness import bench as hb
from tribench_amd.harness import cli
from tribench_amd.harness import schema, stats
from tribench_amd.harness.cases import Case, case_grid, seeded_inputs
from tribench_amd.harness.correctness import _get_tolerance, check_correctness
from tribench_amd.harness.metrics import PEAKS_MI355X, compute_gbps, compute_tflops, roofline_fraction
from tribench_amd.harness.packs import PackIndex
from tribench_amd.harness.types import CorrectnessSpec

PACKS = Path(__file__).resolve().parents[1] / "tribench_amd" / "kernels"

VALID_META = {
    "schema_version": "1.0",
    "name": "test_kernel",
    "family": "test",
    "description": "A test kernel",
    "entrypoints": {"make_inputs": "reference.py:make_inputs", "reference": "reference.py:ref",
                    "triton": "impl.py:run", "variants": {"hip": "impl.py:run"}},
    "supported": {"dtypes": ["fp16", "bf16"], "layouts": ["contiguous"], "backends": ["hip"]},
    "cases": [{"name": "small", "N": 16}],
}


# ---------------------------------------------------------------------------
# schema
# ---------------------------------------------------------------------------

def test_valid_meta_passes():
    assert schema.check(VALID_META) == []


@pytest.mark.parametrize("field", ["schema_version", "name", "family", "description", "entrypoints", "supported",
                                   "cases"])
def test_missing_top_field(field):
    m = copy.deepcopy(VALID_META)
    del m[field]
    assert any(f"'{field}' is required" in e for e in schema.check(m))


@pytest.mark.parametrize("path,value,needle", [
    (("supported", "dtypes"), ["fp8"], "supported.dtypes: 'fp8'"),
    (("supported", "layouts"), ["strided"], "supported.layouts: 'strided'"),
    (("supported", "backends"), ["metal"], "supported.backends: 'metal'"),
    (("entrypoints", "variants"), ["x"], "variants must map"),
    (("entrypoints", "reference"), "reference.py", "not of the form"),
    (("entrypoints", "estimate"), "reference.py:1x", "not of the form"),
])
def test_bad_values(path, value, needle):
    m = copy.deepcopy(VALID_META)
    m[path[0]][path[1]] = value
    assert any(needle in e for e in schema.check(m))


def test_case_names_and_field_types():
    m = copy.deepcopy(VALID_META)
    m["cases"] = [{"N": 3}, {"name": "a"}, {"name": "a"}]
    m["schema_version"] = 1
    errs = schema.check(m)
    assert any("cases[0] needs a 'name'" in e for e in errs)
    assert any("'a' is used twice" in e for e in errs)
    assert any("'schema_version' must be a str" in e for e in errs)


def test_triton_entrypoint_is_required():
    """TriBench's validator requires make_inputs, reference and triton
    (tribench/meta.py:29); so does this one, so the packs pass both."""
    for role in ("make_inputs", "reference", "triton"):
        m = copy.deepcopy(VALID_META)
        m["entrypoints"].pop(role)
        assert any(f"'{role}' is required" in e for e in schema.check(m))


@pytest.mark.parametrize("pack", ["sage_attn", "flash_attn"])
def test_packs_satisfy_the_reference_required_fields(pack):
    """Each committed meta.json has every field TriBench's validate-meta
    requires (top level and entrypoints, tribench/meta.py:24-29), its
    entrypoint files exist, and its triton slot is the HIP variant."""
    raw = json.loads((PACKS / pack / "meta.json").read_text())
    assert {"schema_version", "name", "family", "description", "entrypoints", "supported", "cases"} <= set(raw)
    assert {"make_inputs", "reference", "triton"} <= set(raw["entrypoints"])
    assert raw["entrypoints"]["triton"] == raw["entrypoints"]["variants"]["hip"] == "hip_impl.py:run"
    assert schema.check(raw, PACKS / pack) == []


def test_sage_pack_meta_and_entrypoints():
    index = PackIndex()
    assert "sage_attn" in index.names()
    assert index.problems() == {}
    meta = index.pack("sage_attn").meta
    assert meta.entrypoints.variants == {"hip": "hip_impl.py:run"}
    names = [c.name for c in meta.cases]
    assert {"s4k_d64", "s8k_d64", "cfg1_b1h2n256d64", "cfg2_b4h32n4096d128"} <= set(names)


def test_index_reports_a_broken_pack_and_keeps_the_others(tmp_path):
    good = tmp_path / "good"
    good.mkdir()
    m = copy.deepcopy(VALID_META)
    m["name"] = "good"
    (good / "meta.json").write_text(json.dumps(m))
    for f in ("reference.py", "impl.py"):
        (good / f).write_text("")
    bad = tmp_path / "bad"
    bad.mkdir()
    (bad / "meta.json").write_text("{not json")
    index = PackIndex(tmp_path)
    assert index.names() == ["good"]
    assert list(index.problems()) == [str(bad / "meta.json")]
    with pytest.raises(KeyError, match="no kernel pack 'nope'"):
        index.pack("nope")


def test_flash_pack_meta_entrypoints_and_shared_reference():
    """The flash_attn pack (kernels/flash_attn/meta.json of the reference, plus a
    hip variant): valid meta, the reference's two cases, and make_inputs / ref /
    estimate that agree with the sage_attn pack and the oracle."""
    import numpy as np
    import torch

    from oracle import sage_oracle as O

    pack = PackIndex().pack("flash_attn")
    meta = pack.meta
    assert meta.entrypoints.variants == {"hip": "hip_impl.py:run"}
    assert {"s4k_d64", "s8k_d64"} <= {c.name for c in meta.cases}
    ref_mod = pack.resolve("reference.py:ref").__module__
    assert ref_mod == "tribench.kernels.flash_attn.reference"
    make = pack.entry("make_inputs")
    ref = pack.entry("reference")
    est = pack.entry("estimate")
    assert ref is pack.resolve("reference.py:ref")  # one import per file
    case = dict(batch_size=1, num_heads=2, seq_len=70, head_dim=64, causal=True)
    inp = make(case, "cpu", 0, torch.float16)
    assert inp["q"].dtype == torch.float16 and inp["q"].shape == (1, 2, 70, 64) and inp["causal"]
    out = ref(inp["q"], inp["k"], inp["v"], causal=True)
    want = O.sdpa(inp["q"].float().numpy(), inp["k"].float().numpy(), inp["v"].float().numpy(), causal=True)
    assert np.abs(out.numpy() - want).max() < 1e-5
    e = est(dict(batch_size=8, num_heads=16, seq_len=4096, head_dim=64))
    assert e["flops"] == 4 * 8 * 16 * 4096 * 4096 * 64 and e["bytes"] == 4 * 8 * 16 * 4096 * 64 * 2


# ---------------------------------------------------------------------------
# pack index / case grid / inputs / reference / estimate
# ---------------------------------------------------------------------------

def test_pack_loads_by_file_path_without_a_parent_package():
    import sys

    pack = PackIndex().pack("sage_attn")
    impls = pack.implementations()
    assert [n for n, _ in impls] == ["hip"]  # the triton slot names the same function: listed once
    fn = impls[0][1]
    assert fn.__module__ == "tribench.kernels.sage_attn.hip_impl"
    assert "tribench.kernels.sage_attn" not in sys.modules and "tribench" not in sys.modules
    assert pack.entry("triton") is pack.variant("hip")
    with pytest.raises(KeyError, match="no variant 'cuda'"):
        pack.variant("cuda")


def test_case_grid_and_filters():
    meta = PackIndex().pack("sage_attn").meta
    grid = case_grid(meta, cases=["cfg2_b4h32n4096d128"], dtypes=["bf16"])
    assert grid == [Case("cfg2_b4h32n4096d128", dict(meta.cases[3].params), "bf16", "contiguous")]
    assert grid[0].params["head_dim"] == 128
    assert len(case_grid(meta)) == len(meta.cases) * 3
    assert [c.dtype for c in case_grid(meta, cases=["s4k_d64"], dtypes=["fp32", "bf16", "fp32"])] == ["fp32", "bf16"]
    with pytest.raises(ValueError, match="no dtype 'fp64'"):
        case_grid(meta, dtypes=["fp64"])
    # case names a pack does not offer are passed over (tribench/gen.py:19-20)
    assert case_grid(meta, cases=["nope"]) == []
    assert [c.name for c in case_grid(meta, cases=["nope", "s4k_d64"], dtypes=["bf16"])] == ["s4k_d64"]


def test_seeded_inputs(pack_ref):
    case = Case("c", dict(batch_size=1, num_heads=2, num_kv_heads=1, seq_len=40, head_dim=64, k_offset_std=2.0),
                "bf16", "contiguous")
    a = seeded_inputs(pack_ref.make_inputs, case, "cpu", 0)
    b = seeded_inputs(pack_ref.make_inputs, case, "cpu", 0)
    c = seeded_inputs(pack_ref.make_inputs, case, "cpu", 1)
    # the global generator is seeded before make_inputs (a pack drawing from it is reproducible)
    draw = lambda params, device, seed, dtype: {"x": torch.rand(3, dtype=dtype)}  # noqa: E731
    x1 = seeded_inputs(draw, Case("d", {}, "fp32", "contiguous"), "cpu", 5)["x"]
    x2 = seeded_inputs(draw, Case("d", {}, "fp32", "contiguous"), "cpu", 5)["x"]
    assert torch.equal(x1, x2)
    assert all(torch.equal(a[x], b[x]) for x in "qkv") and not torch.equal(a["q"], c["q"])
    assert a["q"].shape == (1, 2, 40, 64) and a["k"].shape == (1, 1, 40, 64) and a["q"].dtype == torch.bfloat16


def test_make_inputs_distributions(pack_ref):
    base = dict(batch_size=2, num_heads=2, seq_len=4000, head_dim=64)
    plain = pack_ref.make_inputs(base, "cpu", 0, torch.float32)
    off = pack_ref.make_inputs(dict(base, k_offset_std=2.0), "cpu", 0, torch.float32)
    d = off["k"] - plain["k"]  # the offset is constant over tokens
    assert torch.allclose(d, d[:, :, :1].expand_as(d), atol=1e-5) and 0.5 < d[:, :, 0].std() < 4
    assert torch.equal(off["q"], plain["q"]) and torch.equal(off["v"], plain["v"])
    st = pack_ref.make_inputs(dict(base, v_dist="student_t", v_df=3), "cpu", 0, torch.float32)
    kurt = lambda x: float(((x - x.mean()) ** 4).mean() / x.var() ** 2)  # noqa: E731
    assert kurt(st["v"]) > 6 > kurt(plain["v"])


@pytest.mark.parametrize("causal", [False, True])
def test_pack_reference_matches_oracle(pack_ref, causal):
    inp = pack_ref.make_inputs(dict(batch_size=1, num_heads=4, num_kv_heads=2, seq_len=70, head_dim=64),
                               "cpu", 3, torch.float32)
    got = pack_ref.ref(inp["q"], inp["k"], inp["v"], causal=causal, q_chunk=32)
    want = O.sdpa(inp["q"].numpy(), inp["k"].numpy(), inp["v"].numpy(), causal=causal)
    assert got.dtype == torch.float32 and np.abs(got.numpy() - want).max() < 1e-5


def test_estimate(pack_ref):
    e = pack_ref.estimate(dict(batch_size=4, num_heads=32, seq_len=4096, head_dim=128))
    assert e["flops"] == e["algo_flops"] == 2 ** 40 and e["bytes"] == 4 * 4 * 32 * 4096 * 128 * 2
    assert abs(e["prepass_bytes"] / 402.8e6 - 1) < 1e-3
    c = pack_ref.estimate(dict(batch_size=2, num_heads=32, seq_len=16384, head_dim=128, causal=True))
    assert c["flops"] == 2 ** 43 and c["algo_flops"] == O.attention_flops(2, 32, 16384, 16384, 128, True)[1]


# ---------------------------------------------------------------------------
# correctness gate / metrics
# ---------------------------------------------------------------------------

def test_tolerance_precedence():
    assert _get_tolerance("bf16", CorrectnessSpec()) == (1e-2, 1e-2)
    assert _get_tolerance("fp32", CorrectnessSpec()) == (1e-5, 1e-4)
    assert _get_tolerance("bf16", CorrectnessSpec(atol=5e-2, rtol=5e-2)) == (5e-2, 5e-2)
    spec = CorrectnessSpec(atol=5e-2, rtol=5e-2, per_dtype={"fp16": {"atol": 1e-3}})
    assert _get_tolerance("fp16", spec) == (1e-3, 5e-2)


def test_per_case_tolerance_overrides():
    spec = CorrectnessSpec(atol=5e-2, rtol=5e-2, per_dtype={"fp16": {"atol": 1e-3}},
                           per_case={"wide": {"atol": 2.0, "min_cos": 0.999}})
    assert spec.for_case("other") is spec and spec.for_case(None) is spec
    wide = spec.for_case("wide")
    assert (wide.atol, wide.rtol, wide.min_cos) == (2.0, 5e-2, 0.999)
    assert _get_tolerance("fp16", wide) == (2.0, 5e-2)  # the case's atol beats the per-dtype one
    ref = torch.randn(1000, generator=torch.Generator().manual_seed(1))
    assert not check_correctness(ref, ref + 1.0, "bf16", spec).passed
    assert check_correctness(ref, ref + 1.0 * (ref > 0), "bf16", spec.for_case("wide")).passed is False  # cosine
    one_big = ref + 0.5 * (torch.arange(1000) == 7)  # one error of 0.5: inside atol 2, cosine ~ 1
    assert check_correctness(ref, one_big, "bf16", spec.for_case("wide")).passed
    assert not check_correctness(ref, one_big, "bf16", spec).passed
    m = copy.deepcopy(VALID_META)
    m["correctness"] = {"atol": 5e-2, "per_case": {"small": {"atol": 1.0}}}
    assert schema.check(m) == []
    m["correctness"]["per_case"] = {"nope": {"atol": 1.0}}
    assert any("no case named 'nope'" in e for e in schema.check(m))
    m["correctness"]["per_case"] = {"small": {"tol": 1.0}}
    assert any("allowed keys are" in e for e in schema.check(m))
    m["correctness"] = {"atol": "big"}
    assert any("correctness.atol must be a number" in e for e in schema.check(m))


def test_sage_pack_fp8_case_gate():
    meta = schema.read(PACKS / "sage_attn" / "meta.json")
    c5 = meta.correctness.for_case("cfg5_fp8pv_b1h32n32768d128")
    assert (c5.atol, c5.rtol, c5.min_cos) == (2.0, 5e-2, 0.999)
    assert meta.correctness.for_case("cfg2_b4h32n4096d128").atol == 5e-2


def test_check_correctness_reports_cosine_and_bounds():
    ref = torch.randn(1000, generator=torch.Generator().manual_seed(0))
    res = check_correctness(ref, ref + 1e-3, "bf16", CorrectnessSpec(atol=5e-2, rtol=5e-2, max_abs=2e-2,
                                                                   min_cos=0.999))
    assert res.passed and abs(res.max_abs_err - 1e-3) < 1e-6 and res.cosine > 0.9999
    bad = check_correctness(ref, ref + 3e-2, "bf16", CorrectnessSpec(atol=5e-2, rtol=5e-2, max_abs=2e-2))
    assert not bad.passed and "max_abs" in bad.error_msg
    neg = check_correctness(ref, -ref, "bf16", CorrectnessSpec(atol=10, rtol=0, min_cos=0.999))
    assert not neg.passed and neg.cosine < -0.99
    assert not check_correctness(ref, ref[:10], "bf16", CorrectnessSpec()).passed
    assert check_correctness([ref, ref], [ref, ref], "bf16", CorrectnessSpec()).passed


def test_metrics():
    assert compute_tflops(1e12, 1.0) == 1000.0 and compute_gbps(8e9, 1.0) == 8000.0
    assert compute_tflops(1.0, 0.0) == 0.0
    assert roofline_fraction(2500.0, "int8") == pytest.approx(2500 / PEAKS_MI355X["int8"])
    assert PEAKS_MI355X["hbm_gbps"] == 8000.0


# ---------------------------------------------------------------------------
# timers, fake packs, CLI
# ---------------------------------------------------------------------------

def _fake_pack(root: Path, impl_body: str) -> Path:
    d = root / "kernels" / "fake"
    d.mkdir(parents=True)
    meta = copy.deepcopy(VALID_META)
    meta["name"] = "fake"
    meta["supported"]["dtypes"] = ["fp32"]
    meta["entrypoints"]["estimate"] = "reference.py:estimate"
    meta["correctness"] = {"atol": 1e-5, "rtol": 1e-5}
    (d / "meta.json").write_text(json.dumps(meta))
    (d / "reference.py").write_text(textwrap.dedent("""
        import torch
        def make_inputs(case, device, seed, dtype, **kw):
            g = torch.Generator().manual_seed(seed)
            return {"x": torch.randn(case["N"], generator=g).to(dtype).to(device)}
        def ref(x):
            return x * 2
        def estimate(case):
            return {"flops": 2 * case["N"], "bytes": 8 * case["N"]}
    """))
    (d / "impl.py").write_text(textwrap.dedent(impl_body))
    return root / "kernels"


@pytest.mark.parametrize("body,code,needle", [
    ("def run(x):\n    return x * 2\n", 0, "PASS"),
    ("def run(x):\n    return x * 3\n", 1, "FAIL"),
    ("def run(x):\n    raise RuntimeError('sage_attn hip: invalid argument: shape')\n", 1, "Shape mismatch"),
])
def test_cli_test_on_fake_packs(tmp_path, monkeypatch, capsys, body, code, needle):
    kdir = _fake_pack(tmp_path, body)
    monkeypatch.setattr("tribench_amd.harness.packs.KERNELS_DIR", kdir)
    with pytest.raises(SystemExit) as e:
        cli.main(["test", "--kernel", "fake", "--device", "cpu"])
    out = capsys.readouterr().out
    assert e.value.code == code and needle in out


def test_cli_test_all_packs_with_a_case_of_one_pack(tmp_path, monkeypatch, capsys):
    """--kernel all with a case name only one pack offers: the other pack
    runs no case and the command passes."""
    kdir = _fake_pack(tmp_path, "def run(x):\n    return x * 2\n")
    other = kdir / "other"
    other.mkdir()
    for f in ("reference.py", "impl.py"):
        (other / f).write_text((kdir / "fake" / f).read_text())
    meta = json.loads((kdir / "fake" / "meta.json").read_text())
    meta["name"] = "other"
    meta["cases"] = [{"name": "big", "N": 64}]
    (other / "meta.json").write_text(json.dumps(meta))
    monkeypatch.setattr("tribench_amd.harness.packs.KERNELS_DIR", kdir)
    with pytest.raises(SystemExit) as e:
        cli.main(["test", "--kernel", "all", "--cases", "small", "--device", "cpu"])
    out = capsys.readouterr().out
    assert e.value.code == 0, out
    assert "--- other (0 case(s)) ---" in out and "PASS  small" in out and "SKIP" not in out


def test_cli_test_hip_variant_without_gpu_fails_loudly(capsys):
    with pytest.raises(SystemExit) as e:
        cli.main(["test", "--kernel", "sage_attn", "--cases", "cfg1_b1h2n256d64", "--dtype", "fp32",
                  "--device", "cpu"])
    out = capsys.readouterr().out
    assert e.value.code == 1 and "FAIL" in out and "ROCm GPU device" in out


def test_cli_run_writes_results(tmp_path, monkeypatch, capsys):
    kdir = _fake_pack(tmp_path, "def run(x):\n    return x * 2\n")
    monkeypatch.setattr("tribench_amd.harness.packs.KERNELS_DIR", kdir)
    with pytest.raises(SystemExit) as e:
        cli.main(["run", "--kernel", "fake", "--device", "cpu", "--timer", "cpu_wall", "--warmup-ms", "1",
                  "--rep-ms", "5", "--output-dir", str(tmp_path / "res"), "--cpu-ref"])
    assert e.value.code == 0
    runs = list((tmp_path / "res").glob("*/run.json"))
    assert len(runs) == 1
    rec = json.loads(runs[0].read_text())
    rows = rec["results"]
    assert rows[0]["variant"] == "hip" and rows[0]["correctness"]["passed"] and rows[0]["effective_tops"] > 0
    assert rows[1]["variant"] == "cpu_ref" and rows[1]["cpu_threads"] >= 1
    assert (runs[0].parent / "summary.md").exists()
    report = (runs[0].parent / "report.html").read_text()
    assert "fake" in report and "cpu_ref" in report and "<svg" in report
    with pytest.raises(SystemExit):
        cli.main(["run", "--kernel", "fake", "--device", "cpu", "--timer", "cpu_wall", "--warmup-ms", "1",
                  "--rep-ms", "5", "--output-dir", str(tmp_path / "res2"), "--no-plots"])
    assert not list((tmp_path / "res2").glob("*/report.html"))


def test_report_html_columns_escaping_and_no_external_resources(tmp_path):
    from tribench_amd.harness.types import BenchResult, CorrectnessResult, EnvInfo, RunRecord
    from tribench_amd.harness.viz import generate_run_plots, render_html

    lat = dict(latency_ms_p50=1.0, latency_ms_p90=1.1, latency_ms_p95=1.2, latency_ms_p99=1.3,
               latency_ms_min=0.9, latency_ms_max=1.4, latency_ms_mean=1.05, latency_ms_std=0.1)
    ok = BenchResult("sage_attn", "cfg2<b>", "bf16", "contiguous", variant="hip", effective_tops=1117.4,
                     algo_tops=1117.4, roofline_peak=5000.0, roofline_unit="int8", roofline_fraction=0.2235,
                     prepass_ms_p50=0.12, prepass_gbps=3300.0, prepass_hbm_fraction=0.4125,
                     correctness=CorrectnessResult(True, 5e-2, 5e-2, max_abs_err=1.2e-2, cosine=0.99995), **lat)
    bad = BenchResult("sage_attn", "cfg3", "bf16", "contiguous", variant="hip",
                      correctness=CorrectnessResult(False, 5e-2, 5e-2, max_abs_err=0.5), **lat)
    cpu = BenchResult("sage_attn", "cfg2<b>", "bf16", "contiguous", variant="cpu_ref", cpu_threads=16,
                      effective_tops=0.05, **lat)
    rec = RunRecord(run_id="r1", env=EnvInfo(gpu_name="AMD Instinct MI355X", rocm_arch="gfx950:sramecc+:xnack-",
                                             hip_version="7.0.1"), results=[ok, bad, cpu])
    page = render_html(rec)
    assert "gfx950:sramecc+:xnack-" in page and "7.0.1" in page
    assert "cfg2&lt;b&gt;" in page and "cfg2<b>" not in page
    assert "22.4% of 5000 int8" in page and "41.2%" in page and "0.999950" in page
    assert page.count('<tr class="fail">') == 1 and "FAIL" in page and "cpu_ref (16 threads)" in page
    assert "http" not in page.replace('xmlns="http://www.w3.org/2000/svg"', "") and "<script" not in page
    # the failed row is in the table but not in the charts
    assert page.count("cfg3") == 1
    assert generate_run_plots(RunRecord(run_id="empty"), tmp_path) == []
    (path,) = generate_run_plots(rec, tmp_path / "run")
    assert path.name == "report.html" and path.read_text(encoding="utf-8") == page


def test_cli_list_and_validate(capsys):
    with pytest.raises(SystemExit) as e:
        cli.main(["validate-meta"])
    assert e.value.code == 0
    with pytest.raises(SystemExit) as e:
        cli.main(["list"])
    assert e.value.code == 0 and "sage_attn" in capsys.readouterr().out


def test_cpu_timer_and_stats():
    lats = hb._bench_cpu_wall(lambda: math.sqrt(2.0), 1.0, 2.0)
    st = stats.summarize(lats)
    assert len(lats) >= 1 and st.p50 >= 0 and st.p99 >= st.p50
    threads, model = hb.cpu_info()
    assert threads >= 1 and isinstance(model, str)
    s = stats.summarize([1.0, 1.0, 1.0, 5.0])
    assert s.p50 == 1.0 and s.tail == pytest.approx(s.p99) and s.jitter == pytest.approx(s.std / 2.0)
    assert stats.summarize([0.0]).tail is None
    with pytest.raises(ValueError):
        stats.summarize([])


def test_workload_and_rates():
    attn = stats.workload(dict(batch_size=4, num_heads=32, num_kv_heads=8, seq_len=4096, head_dim=128))
    assert attn == stats.Workload(tokens=4 * 4096, elements=4 * 32 * 4096 * 128, sequences=4)
    assert stats.workload(dict(M=64, N=32)) == stats.Workload(elements=64 * 32)
    assert stats.workload(dict(seq_len=10)) == stats.Workload(tokens=10, elements=10)
    assert stats.workload(dict(flag=True, name="x")) == stats.Workload()
    r = stats.rates(attn, 2.0)
    assert r["tokens_per_s"] == 4 * 4096 * 500 and r["sequences_per_s"] == 2000
    assert stats.rates(attn, 0.0)["elements_per_s"] is None
    with stats.PeakMemory("cpu") as mem:
        pass
    assert mem.allocated_mib is None and mem.reserved_mib is None


def test_load_meta_keeps_case_params():
    meta = schema.read(PACKS / "sage_attn" / "meta.json")
    c = {x.name: x.params for x in meta.cases}["cfg5_fp8pv_b1h32n32768d128"]
    assert c["pv_dtype"] == "fp8" and c["q_gran"] == "wave" and "name" not in c


def test_roofline_unit_per_pack():
    from tribench_amd.harness.cli import roofline_unit_for

    index = PackIndex()
    case = lambda dt: Case("c", {}, dt, "contiguous")  # noqa: E731
    assert roofline_unit_for(index.pack("sage_attn").meta, case("bf16")) == "int8"
    assert roofline_unit_for(index.pack("flash_attn").meta, case("fp16")) == "fp16"
    assert roofline_unit_for(index.pack("flash_attn").meta, case("bf16")) == "bf16"
