"""CPU oracle of the sage_attn hot path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product path never does.
"""
