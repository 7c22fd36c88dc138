"""CPU oracle for the MedNeXt operator path — TEST INFRASTRUCTURE ONLY.

Plain numpy (float64) restatements of what the reference computes on this path,
each function citing the reference file:line it follows. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
anything here, and only as the checker (or, for the CPU baseline, as the timed
reference CPU path) — never as the product path. The product
(``mednext-accel_amd/``) must not import this package.

Pinning (how each oracle function is itself checked, see tests/test_oracle.py):
  depthwise.*   torch float64 F.conv3d + autograd (the reference's own library
                routine), closed forms (k=1 scale, impulse -> kernel, all-ones
                interior -> sum(w)+b), brute-force loops on tiny shapes, and the
                committed golden fixtures in tests/golden/.
  groupnorm.*   torch float64 F.group_norm + autograd, closed-form invariants
                (zero mean / unit variance per (n, c), dx orthogonal to 1 and x̂).
  pointwise.*   torch float64 F.conv3d(1x1x1) / addmm, F.gelu(approximate="none"),
                GELU special values (gelu(0)=0, odd part, large-|x| limits).
  block.*       composition of the above checked against a torch float64
                MedNeXt block (reference models/blocks.py:82-91) + autograd.
  policy.*      the reference's integer launch recipe, pinned by the
                reference's own 209-row launch fixture (tests/golden/).
"""
