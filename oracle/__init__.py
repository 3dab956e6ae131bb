"""CPU oracle for the eas hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
(``easy_as_amd``) never imports, links or runs anything here; its GPU path has
no CPU fallback.

* ``ops``    — closed-form arithmetic (f32 add, correctly rounded fmaf via the C
               restatement in ``fmaf.c``, an independent round-to-odd fmaf that
               pins it, f64 matmul references).
* ``interp`` — numpy interpreter of eas kernels with the reference's execution
               semantics (SPMD lanes, Metal threadgroups, dot, simdgroup MMA).
"""
