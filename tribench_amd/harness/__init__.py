"""Benchmark harness for kernel packs: the counterpart of TriBench's
``tribench`` package (registry, schema, case grid, correctness gate, timers,
metrics, CLI), without Triton and with MI355X roofline reporting."""
