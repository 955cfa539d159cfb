"""CPU oracle for the sparse-prefill path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker or the timed CPU baseline.
"""
