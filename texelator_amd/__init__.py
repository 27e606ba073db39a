"""gfx950 (MI355X) BC4 weight path: decode GEMV and bf16 prefill GEMM over 8-byte BC4 blocks.

Mirrors the reference package's module API for this path: ``runtime``, ``tuning``,
``autotune``, ``prefill``, ``hardware`` and ``encoder``. Kernels live in
``libtexelator_hip.so`` (built from ``csrc/`` by ``texelator_amd.build``).
"""

__version__ = "0.1.0"
