"""tribench_amd — MI355X-native SageAttention hot path for TriBench.

``csrc/``     hand-written gfx950 HIP kernels and the C ABI (include/sage_attn.h)
``kernels/``  the sage_attn kernel pack (meta.json, reference.py, hip_impl.py)
``harness/``  the harness that drives kernel packs (test / run)
``build.py``  builds ``lib/libsage_attn.so``
"""
__version__ = "0.1.0"
