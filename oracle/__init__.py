"""CPU oracle for the KV-reuse path — TEST INFRASTRUCTURE ONLY.

Restatements of the reference's CPU semantics used as the checker for the HIP kernels and as
the CPU baseline in ``bench.py``. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this package; the product package
``semblend_amd`` never does.
"""
