"""CPU oracle for the quantized-linear path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the timed
CPU baseline.  The product package ``mindpipe_amd`` never imports it.
"""
