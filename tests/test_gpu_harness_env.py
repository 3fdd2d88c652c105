"""The harness's `run` command on the GPU, in-process: the ROCm environment of
the run record (the reference records only CUDA fields, tribench/env.py:12-52)
and the roofline columns of run.json, summary.md and report.html
(tribench/io.py:53-115, viz.py:495-533 carry the reference's own columns)."""
from __future__ import annotations

import json

import pytest

from tribench_amd.harness import cli

pytestmark = pytest.mark.gpu


def test_cli_run_records_rocm_env_and_roofline_columns(tmp_path, gpu_device, capsys):
    out_dir = tmp_path / "res"
    print("[harness-env] cli run sage_attn cfg1_b1h2n256d64 fp32 --cpu-ref", flush=True)
    with pytest.raises(SystemExit) as e:
        cli.main(["run", "--kernel", "sage_attn", "--cases", "cfg1_b1h2n256d64", "--dtype", "fp32",
                  "--device", "cuda:0", "--warmup-ms", "5", "--rep-ms", "20", "--cpu-ref",
                  "--output-dir", str(out_dir)])
    printed = capsys.readouterr().out
    assert e.value.code == 0, printed
    (run_json,) = out_dir.glob("*/run.json")
    rec = json.loads(run_json.read_text())
    env = rec["env"]
    assert env["rocm_arch"].startswith("gfx950"), env
    assert env["hip_version"] and env["gpu_count"] >= 1 and env["torch_version"]
    rows = rec["results"]
    hip = [r for r in rows if r["variant"] == "hip"]
    cpu = [r for r in rows if r["variant"] == "cpu_ref"]
    assert len(hip) == 1 and len(cpu) == 1, [r["variant"] for r in rows]  # the triton slot runs once, as hip
    h = hip[0]
    assert h["correctness"]["passed"] and h["correctness"]["cosine"] >= 0.999
    assert h["effective_tops"] > 0 and h["roofline_unit"] == "int8" and h["roofline_peak"] == 5000.0
    assert 0 < h["roofline_fraction"] < 1 and h["prepass_gbps"] > 0 and 0 < h["prepass_hbm_fraction"] < 1
    assert cpu[0]["cpu_threads"] >= 1 and cpu[0]["cpu_model"]
    summary = (run_json.parent / "summary.md").read_text()
    assert "roofline" in summary and "prepass GB/s" in summary and "% int8" in summary
    report = (run_json.parent / "report.html").read_text()
    assert "gfx950" in report and "cpu_ref" in report and "<svg" in report
    assert "<th>roofline</th>" in report and "<th>pre-pass GB/s</th>" in report and "<th>eff. TOPS</th>" in report


def test_cli_test_command_on_both_packs(gpu_device, capsys):
    """`test` (tribench/cli.py's correctness command) on the GPU: every case of
    a small selection passes the pack's gate, for the INT8 and the flash pack."""
    for kernel, cases, dtype in (("sage_attn", "cfg1_b1h2n256d64", "bf16"), ("flash_attn", "s4k_d64", "fp16")):
        print(f"[harness-test] cli test {kernel} {cases} {dtype}", flush=True)
        with pytest.raises(SystemExit) as e:
            cli.main(["test", "--kernel", kernel, "--cases", cases, "--dtype", dtype, "--device", "cuda:0"])
        printed = capsys.readouterr().out
        assert e.value.code == 0 and "FAIL" not in printed, printed


def test_cli_run_with_the_hip_graph_timer(tmp_path, gpu_device, capsys):
    """`run --timer hip_graph`: the call captured into a HIP graph and its
    replays timed (harness/bench.py); the row still passes its correctness
    check, which runs the call eagerly."""
    out_dir = tmp_path / "res"
    print("[harness-graph] cli run sage_attn cfg1_b1h2n256d64 bf16 --timer hip_graph", flush=True)
    with pytest.raises(SystemExit) as e:
        cli.main(["run", "--kernel", "sage_attn", "--cases", "cfg1_b1h2n256d64", "--dtype", "bf16",
                  "--device", "cuda:0", "--warmup-ms", "5", "--rep-ms", "20", "--timer", "hip_graph",
                  "--no-plots", "--output-dir", str(out_dir)])
    printed = capsys.readouterr().out
    assert e.value.code == 0, printed
    (run_json,) = out_dir.glob("*/run.json")
    (h,) = [r for r in json.loads(run_json.read_text())["results"] if r["variant"] == "hip"]
    assert h["correctness"]["passed"] and h["timer_backend"] == "hip_graph", h
    assert h["latency_ms_p50"] > 0, h
