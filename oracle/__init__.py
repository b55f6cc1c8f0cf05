"""Test oracle for the mL1-ACE hot path.  TEST INFRASTRUCTURE ONLY.

This package is a CPU restatement of the reference's algorithm, used as the
checker for the HIP implementation.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import it.
The product (``ace-kernels_amd/ace_kernels``) never imports, calls or falls
back to anything in here.

Modules:

- ``oracle.reference``: the reference loss itself (``HardL1ACELoss`` /
  ``SoftL1ACELoss`` forward with their ``hard_binned_calibration`` /
  ``soft_binned_calibration`` B x C loop of ``bucketize`` + ``scatter_add`` +
  ``scatter_reduce``), differentiated by autograd, on torch CPU tensors.  It is
  the golden-vector reproducer and the timed CPU baseline.
- ``oracle.v2``: the reference's vectorised per-bin statistics and its
  handwritten ("v2") backward, float32 or float64; pinned by float64
  ``gradcheck`` and by autograd through ``oracle.reference``.
- ``oracle.f64``: an independent float64 NumPy restatement written from the
  mathematics (per-bin weights W, P, G), including per-bin statistics used to
  judge the accuracy of the GPU sums at full size.

Pinning (each function is checked by something other than a retyping of its
own formula):

- ``reference``: the 43 golden cases of ``tests/golden`` (loss and gradient,
  written by the reference on its own platform), loss in [0, 1], voxel-order
  invariance, and agreement with ``f64`` on every case.
- ``v2``: float64 ``gradcheck`` (finite differences) and float64 agreement
  with autograd through ``reference``; golden cases.
- ``f64``: golden losses; closed forms (constant probabilities -> 0.25,
  one bin hard == one bin soft); hard counts sum to N; soft weights sum to 1.
"""
