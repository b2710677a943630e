"""CPU oracle for the VoroTracing traversal hot path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this package, and only as the checker.  The product
package ``vorotracing_amd`` never imports it and has no CPU fallback.

``oracle.core`` binds ``liboracle.so`` (the C restatement of the reference
kernels, ``oracle.c``); ``oracle.host_ops`` restates the reference's
host-side preparation steps (Morton reorder, tile permutation, q8
quantisation, fp16 padding, nearest-site start cell) in numpy.
"""
