"""Test oracle for frame_analytics_amd -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

* ``oracle.reference`` -- float64 NumPy restatement of the reference's metric
  definitions (NevermindNilas/frame_analytics reference.py / functional.py).
* ``oracle.ref_cpu``   -- ctypes binding of the reference's own CPU C++ kernels,
  compiled by ``oracle/Makefile`` from the reference sources into ``oracle/_ref``.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this package, and only as the checker / the CPU baseline.
The product package ``frame_analytics_amd`` never imports it.
"""
