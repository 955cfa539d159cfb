"""Measurement harnesses beside ``bench.py``: layer / model sweeps over the
BASELINE configs and rocprofv3 workloads with the HBM-traffic reduction. Not part
of the ``exp3_amd`` package that callers import."""
