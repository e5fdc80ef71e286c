"""CPU oracle for kernelforge_amd -- TEST INFRASTRUCTURE ONLY.

Plain-torch (CPU) restatements of the reference algorithms, each citing the
KernelForge file:line it follows.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only
as the checker or the timed CPU baseline.  The shipped package
(``kernelforge_amd``) never imports it and has no CPU fallback.

How each function is pinned (beyond restating the reference):

- ``rmsnorm``: fp64 brute-force golden vectors (tests/golden), the closed form
  with weight = 1 (unit RMS per row), scale equivariance.
- ``sana``: golden vectors from the O(N^2) quadratic form in pure-Python fp64
  (a different algorithm from the linear form restated here), linearity in v,
  relu(q) = 0 -> 0, split-count invariance.
- ``fa``: golden vectors from explicit pure-Python softmax/JVP formulas,
  central finite differences, JVP/VJP duality, uniform score shift -> tO = 0,
  value-only tangents -> tO = P tV, probability-mass preservation, and the
  tiled online recurrence (``fa.fused_forward_jvp_tiled``) against the dense
  jvp at several tile sizes.
"""
