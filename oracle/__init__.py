"""CPU oracle for the MoE forward path (test infrastructure, never shipped).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker: the product
path in ``llm_gpu_kernels_amd`` never calls it.
"""
