"""CPU oracle for the fused GGML dequantize x matvec path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only to compare against.  The product package
``pyrite_amd`` never imports it.
"""
