"""CPU oracle for the MedNeXt operator path — TEST INFRASTRUCTURE ONLY.

Plain numpy (float64) restatements of what the reference computes on this path,
each function citing the reference file:line it follows. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
anything here, and only as the checker (or, for the CPU baseline, as the timed
reference CPU path) — never as the product path. The product
(``mednext-accel_amd/``) must not import this package.

Pinning (how each oracle function is itself checked, see tests/test_oracle.py):
  depthwise.*      torch float64 F.conv3d + autograd (the reference's own library
                   routine), closed forms (k=1 scale, impulse -> kernel, all-ones
                   interior -> sum(w)+b), brute-force loops on tiny shapes, a
                   planted mistake (flipped kernel) that the checks must catch,
                   and the committed golden fixtures in tests/golden/.
  groupnorm.*      torch float64 F.group_norm + autograd, the golden fixtures,
                   and closed-form invariants (per-(n, c) zero mean and variance
                   var/(var+eps); the backward's projection identities with eps).
  pointwise.*      torch float64 F.conv3d(1x1x1) / addmm, the golden fixtures, an
                   asymmetric shape that fails a transposed weight, and GELU
                   special values (gelu(0)=0, odd part, large-|x| limits).
  grn.*            torch float64 autograd of the reference's GRN formula (a
                   check of the hand-derived backward), central finite
                   differences, the reference tests' closed-form coupling case
                   (x = (1, 2, 4), gamma = (2, 3, -4), dy only in channel 0 ->
                   -2 / (7 + eps)^2 in the others) and the all-zero input
                   (dx = dy exactly, dgamma = 0).
  reference_cpu.*  not a restatement: the reference's own CPU path (PyTorch's
                   F.conv3d + aten.convolution_backward), timed by bench.py as
                   the CPU baseline.
"""
