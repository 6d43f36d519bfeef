"""CPU oracle for the KV-reuse path — TEST INFRASTRUCTURE ONLY.

Restatements of the reference's CPU semantics that the HIP kernels are tested against, and
the CPU baseline in ``bench.py``. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this package; the product package
``semblend_amd`` never does.
"""
