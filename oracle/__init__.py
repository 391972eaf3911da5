"""CPU oracle for the AttnRes read: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
CPU baseline, as the thing timed on the host cores).  The product path in
``lr-attnres_amd/`` never imports it and has no CPU fallback.

Modules
-------
``attnres_oracle``  eager PyTorch restatement of the reference's eager op
                    (same cast / rounding / eps sequence), fp32/bf16/fp16.
``fp64``            independent float64 numpy formulation from the math,
                    including closed-form gradients; used to pin the eager
                    restatement (and, through it, the HIP kernels).

Pinning status per function is listed in the header of each module.
"""
