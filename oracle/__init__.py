"""CPU oracle for the BC4 weight path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import, call or link anything in this package, and only as the
checker. The product (``texelator_amd``) never imports it; the product path fails
loudly when its HIP library is missing instead of falling back to this code.

Two independent restatements live here:

* ``oracle.bc4`` -- numpy: palette, block codec, LUT decoder, float64 matvec/GEMM,
  and the reference's error metrics.
* ``oracle/bc4_oracle.c`` -- plain C (built to ``oracle/liboracle.so`` by
  ``oracle/Makefile``): palette, decoder, matvec/GEMM. Tests check the two
  against each other and against closed forms.

Parity pins (what each function is checked against) are listed in the
docstring of each function. Functions with no independent pin say
"parity unpinned".
"""
