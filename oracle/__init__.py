"""CPU oracle for the algebraic-extra kernel hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in float64 NumPy (plus torch-CPU only for bfloat16
rounding and float64 autograd checks), the numerics of the reference's
attention, fused LM-head and QK RMS-norm kernels:

* ``oracle.attention`` -- ``src/algebraic/kernels/flash.py`` (variants, rho,
  forward statistics, tile VJP, sink gradient, range guard) and the dense
  ``algebraic.asinh_attention`` / ``standard.softmax_attention``.
* ``oracle.head``      -- ``src/algebraic/kernels/fused_head.py`` and the dense
  heads in ``algebraic.py`` / ``standard.py`` / ``evaluation.py``.
* ``oracle.qknorm``    -- ``src/algebraic/kernels/qk_norm.py`` and
  ``algebraic.rms_norm``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker (or the timed CPU
baseline); the shipped HIP path never calls into it.

Every function cites the reference file:line it follows. Each is pinned by
checks in ``tests/test_oracle.py`` against closed forms and independent
textbook formulations (softmax of ``n*asinh(s/c)`` logits, float64 autograd,
finite differences, known-answer constants from the reference's own tests).
"""
