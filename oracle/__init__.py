"""CPU oracle for the GDN decode / prefill paths (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline.  The product path (``kachua_mlsys_amd``) never imports it.
"""
