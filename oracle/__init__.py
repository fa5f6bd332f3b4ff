"""CPU oracle for the Qwen3.6-35B-A3B attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or, for ``cpu_baseline``, as the timed CPU restatement).  The product
path (the HIP library and its Python host layer) never imports it.
"""
