"""TEST INFRASTRUCTURE ONLY — CPU oracle for the dot_amd hot path.

``oracle.sinkhorn`` and ``oracle.bidirectional_softmax`` restate the
reference's algorithms in numpy (float64 by default); ``oracle.ref`` calls the
reference's own CPU kernels compiled into ``oracle/_ref/`` by
``oracle/Makefile``.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker or the timed CPU baseline: the ``dot_amd`` product never imports it
and has no CPU fallback for GPU tensors.
"""
