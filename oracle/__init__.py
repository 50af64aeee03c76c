"""CPU oracle for the INT8 weight-only linear path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only to
check results against it (or, in the baseline leg, to time the reference's CPU
path beside them).  The product (``pageserve_amd``) never imports it and has
no CPU fallback: without its HIP library it raises.
"""
