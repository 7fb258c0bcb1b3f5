"""CPU oracle of the quantized-matmul hot path.  TEST INFRASTRUCTURE ONLY.

Used by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` as the checker; the ``mlxturbo_amd`` package never imports it.
"""
