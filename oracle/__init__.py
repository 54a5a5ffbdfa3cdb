"""CPU oracle for the Cheby-RKV hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
CPU baseline, as the thing timed on the host cores).  The product path in
``orthossm_amd`` never imports it and has no CPU fallback.

Modules
-------
``cheby_ema``       float64 restatement of the operator (forward, carry,
                    dynamic lambda, TTT coefficient gradient by a closed-form
                    adjoint and by torch autograd).
``reference_form``  float32 torch restatement of the reference's own PyTorch
                    formulation (basis + einsum + per-head EMA loop); it is
                    the CPU baseline and an independent cross-check.
"""
