"""Command line of the harness (counterpart of tribench/cli.py).

    python -m tribench_amd list
    python -m tribench_amd validate-meta
    python -m tribench_amd test --kernel sage_attn [--cases c1,c2] [--dtype bf16]
    python -m tribench_amd run  --kernel sage_attn [--cases ...] [--timer hip_event|hip_graph]
                                [--cpu-ref] [--no-plots] [--output-dir results]

Subcommands, options and exit codes follow cli.py:11-61, 205-582 of the
reference: every implementation of a pack (its ``triton`` entrypoint when
present, then each variant) is checked against the pack's reference on the
same seeded inputs; ``run`` times them and writes run.json, summary.md and
report.html (``viz.py``; ``--no-plots`` leaves it out).
``run`` adds effective TOPS, the roofline fraction and, with ``--cpu-ref``, a
``cpu_ref`` row timing the pack's reference on this host's cores.
"""
from __future__ import annotations

import argparse
import sys
from typing import Sequence

from .. import __version__


def _build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="tribench_amd", description="Kernel-pack benchmark harness (MI355X)")
    p.add_argument("--version", action="version", version=f"%(prog)s {__version__}")
    sub = p.add_subparsers(dest="command", required=True)
    sub.add_parser("list", help="List registered kernels with dtypes and cases")
    sub.add_parser("validate-meta", help="Validate every kernel's meta.json")
    t = sub.add_parser("test", help="Run correctness tests")
    t.add_argument("--kernel", default="all")
    t.add_argument("--cases", default=None)
    t.add_argument("--dtype", default=None)
    t.add_argument("--device", default="cuda:0")
    t.add_argument("--seed", type=int, default=0)
    r = sub.add_parser("run", help="Run benchmarks and save results")
    r.add_argument("--kernel", default="all")
    r.add_argument("--cases", default=None)
    r.add_argument("--dtype", default=None)
    r.add_argument("--layout", default=None)
    r.add_argument("--device", default="cuda:0")
    r.add_argument("--seed", type=int, default=0)
    r.add_argument("--warmup-ms", type=float, default=200.0)
    r.add_argument("--rep-ms", type=float, default=2000.0)
    r.add_argument("--quantiles", default="0.5,0.9,0.95,0.99")
    r.add_argument("--timer", default="hip_event", choices=["hip_event", "hip_graph", "cpu_wall"])
    r.add_argument("--output-dir", default="results")
    r.add_argument("--no-correctness", action="store_true")
    r.add_argument("--cpu-ref", action="store_true", help="also time the reference on the host CPU")
    r.add_argument("--no-plots", action="store_true", help="do not write report.html")
    return p


def _first_line(e: Exception) -> str:
    s = str(e)
    return s.splitlines()[0] if s else ""


def roofline_unit_for(meta, case) -> str:
    """MFMA peak a case is priced against: INT8 for packs tagged "int8" (the
    quantized QK product dominates), else the case's dtype."""
    if "int8" in (getattr(meta, "tags", None) or []):
        return "int8"
    return case.dtype if case.dtype in ("fp16", "bf16", "fp32") else "bf16"


def _print_error(prefix: str, e: Exception) -> None:
    from .errors import get_hint

    print(f"{prefix}Error: {e.__class__.__name__}: {_first_line(e)}")
    hint = get_hint(e)
    if hint:
        print(f"{prefix}Hint: {hint}")


def _clear_device_cache() -> None:
    try:
        import torch

        if torch.cuda.is_available():
            try:
                torch.cuda.synchronize()
            except Exception:
                pass
            torch.cuda.empty_cache()
    except Exception:
        pass


def _sync(device: str) -> None:
    import torch

    if device.startswith("cuda") and torch.cuda.is_available():
        torch.cuda.synchronize()


def _cmd_list(args) -> int:
    from .packs import PackIndex

    index = PackIndex()
    for name in index.names():
        pack = index.pack(name)
        m = pack.meta
        impls = [label for label, spec in [("triton", m.entrypoints.triton), *m.entrypoints.variants.items()]
                 if spec]
        print(f"{m.name:20s} {m.family:12s} dtypes={','.join(m.supported.dtypes)} impls={','.join(impls)} "
              f"cases={','.join(c.name for c in m.cases)}")
    for path, msg in index.broken.items():
        print(f"(not loaded) {path}: {msg}")
    return 0


def _cmd_validate_meta(args) -> int:
    from .packs import PackIndex

    index = PackIndex()
    problems = index.problems()
    if not problems:
        print(f"All meta.json files are valid ({len(index.names())} pack(s)).")
        return 0
    for path, errors in problems.items():
        print(f"{path}:")
        for e in errors:
            print(f"   - {e}")
    return 1


def _cmd_test(args) -> int:
    from .cases import case_grid, seeded_inputs
    from .correctness import check_correctness
    from .packs import PackIndex

    index = PackIndex()
    names = index.names() if args.kernel == "all" else [n.strip() for n in args.kernel.split(",")]
    dtype_filter = args.dtype.split(",") if args.dtype else None
    case_filter = args.cases.split(",") if args.cases else None
    all_passed = True
    for name in names:
        try:
            pack = index.pack(name)
            meta = pack.meta
            cases = case_grid(meta, cases=case_filter, dtypes=dtype_filter)
            make_inputs = pack.entry("make_inputs")
            reference = pack.entry("reference")
            impls = pack.implementations()
        except Exception as e:
            all_passed = False
            print(f"\n--- {name} ---\n  SKIP  kernel initialization failed")
            _print_error("   ", e)
            continue
        print(f"\n--- {name} ({len(cases)} case(s)) ---")
        for case in cases:
            try:
                inputs = seeded_inputs(make_inputs, case, args.device, args.seed)
                ref_out = reference(**inputs)
            except Exception as e:
                all_passed = False
                print(f"    SKIP  {case.label()}  (setup/reference exception)")
                _print_error("     ", e)
                _clear_device_cache()
                continue
            for impl_name, fn in impls:
                label = impl_name if impl_name == "triton" else f"variant:{impl_name}"
                try:
                    out = fn(**inputs)
                    _sync(args.device)
                    res = check_correctness(ref_out, out, case.dtype, meta.correctness.for_case(case.name))
                    status = "PASS" if res.passed else "FAIL"
                    cos = "" if res.cosine is None else f"  cos={res.cosine:.6f}"
                    print(f"    {status}  {case.name} [{label}] dtype={case.dtype}  "
                          f"max_abs={res.max_abs_err:.2e}  max_rel={res.max_rel_err:.2e}{cos}")
                    if not res.passed:
                        all_passed = False
                        if res.error_msg:
                            print(f"     {res.error_msg}")
                except Exception as e:
                    all_passed = False
                    print(f"    FAIL  {case.name} [{label}] dtype={case.dtype}  (Exception)")
                    _print_error("     ", e)
                    _clear_device_cache()
            del inputs, ref_out
            _clear_device_cache()
    return 0 if all_passed else 1


def _cmd_run(args) -> int:
    from .bench import run_benchmark, run_cpu_reference
    from .cases import case_grid
    from .env import capture_env
    from .io import make_run_id, write_json, write_summary_md
    from .packs import PackIndex
    from .types import RunRecord

    index = PackIndex()
    names = index.names() if args.kernel == "all" else [n.strip() for n in args.kernel.split(",")]
    dtype_filter = args.dtype.split(",") if args.dtype else None
    case_filter = args.cases.split(",") if args.cases else None
    layout_filter = args.layout.split(",") if args.layout else None
    quantiles = [float(x) for x in args.quantiles.split(",")]
    record = RunRecord(run_id=make_run_id(args.kernel, args.device), env=capture_env(" ".join(sys.argv)),
                       seed=args.seed, timer_backend=args.timer, warmup_ms=args.warmup_ms, rep_ms=args.rep_ms,
                       quantiles=quantiles)
    failed = False
    for name in names:
        try:
            pack = index.pack(name)
            meta = pack.meta
            cases = case_grid(meta, cases=case_filter, dtypes=dtype_filter, layouts=layout_filter)
            make_inputs = pack.entry("make_inputs")
            reference = pack.entry("reference")
            estimate = pack.entry("estimate")
            impls = pack.implementations()
            stage_mod = sys.modules.get(f"tribench.kernels.{name}.hip_impl")
        except Exception as e:
            failed = True
            print(f"\n--- Benchmarking {name} ---\n  SKIP  kernel initialization failed")
            _print_error("   ", e)
            continue
        print(f"\n--- Benchmarking {name} ({len(cases)} case(s)) ---")
        for case in cases:
            main_p50 = None
            for impl_name, fn in impls:
                stages = None
                if stage_mod is not None and hasattr(stage_mod, "prepass_stage"):
                    stages = {"prepass": stage_mod.prepass_stage}
                try:
                    res = run_benchmark(kernel_name=name, meta=meta, make_inputs_fn=make_inputs,
                                        reference_fn=reference, triton_fn=fn, estimate_fn=estimate, case=case,
                                        device=args.device, seed=args.seed, warmup_ms=args.warmup_ms,
                                        rep_ms=args.rep_ms, quantiles=quantiles, timer_backend=args.timer,
                                        run_correctness=not args.no_correctness, stage_fns=stages,
                                        roofline_unit=roofline_unit_for(meta, case))
                except Exception as e:
                    failed = True
                    print(f"    SKIP  {case.name} [{impl_name}] dtype={case.dtype}  (benchmark exception)")
                    _print_error("     ", e)
                    _clear_device_cache()
                    if args.kernel != "all":
                        raise
                    continue
                if impl_name != "triton":
                    res.variant = impl_name
                if main_p50 is None:
                    main_p50 = res.latency_ms_p50
                    res.triton_vs_variant_p50_ratio = 1.0
                elif res.latency_ms_p50 > 0:
                    res.triton_vs_variant_p50_ratio = main_p50 / res.latency_ms_p50
                record.results.append(res)
                corr = ""
                if res.correctness:
                    corr = " PASS" if res.correctness.passed else " FAIL"
                    failed |= not res.correctness.passed
                tops = f"  {res.effective_tops:.1f} TOPS" if res.effective_tops else ""
                roof = f" ({100 * res.roofline_fraction:.1f}% {res.roofline_unit} peak)" if res.roofline_fraction else ""
                pre = f"  prepass {res.prepass_ms_p50:.4f}ms {res.prepass_gbps:.0f} GB/s" if res.prepass_gbps else ""
                print(f"    {res.case_name} [{impl_name}]  {res.dtype}  p50={res.latency_ms_p50:.4f}ms  "
                      f"p95={res.latency_ms_p95:.4f}ms{tops}{roof}{pre}{corr}")
            if args.cpu_ref:
                cres = run_cpu_reference(kernel_name=name, make_inputs_fn=make_inputs, reference_fn=reference,
                                         estimate_fn=estimate, case=case, seed=args.seed)
                record.results.append(cres)
                print(f"    {cres.case_name} [cpu_ref]  p50={cres.latency_ms_p50:.1f}ms  "
                      f"{cres.effective_tops or 0:.3f} TOPS on {cres.cpu_threads} threads ({cres.cpu_model})")
    json_path = write_json(record, args.output_dir)
    md_path = write_summary_md(record, args.output_dir)
    print(f"\nResults saved to: {json_path.parent}\n   JSON:     {json_path}\n   Summary:  {md_path}")
    if not args.no_plots:
        from .viz import generate_run_plots
        for p in generate_run_plots(record, json_path.parent):
            print(f"   Report:   {p}")
    return 1 if failed else 0


def main(argv: Sequence[str] | None = None) -> None:
    args = _build_parser().parse_args(argv)
    handlers = {"list": _cmd_list, "validate-meta": _cmd_validate_meta, "test": _cmd_test, "run": _cmd_run}
    sys.exit(handlers[args.command](args))


if __name__ == "__main__":
    main()
