"""CPU oracle for the coded-projection hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything under ``oracle/``, and only as the checker or
as the timed CPU baseline.  The product package (``escha_mlx_amd``) never
imports it and fails loudly when its HIP library is missing.

``ref_np`` restates the reference's NumPy contract (escha_mlx/ref.py) plus the
GPU kernels' fixed accumulation order (escha_mlx/msl.py:205-308), so that the
HIP results can be checked bit-for-bit where the order is reproduced and under
a stated tolerance where it is not.  Each function cites the reference
file:line it follows and names the check that pins it (golden vectors, closed
forms, brute force); a function with no such check says "parity unpinned".
"""
