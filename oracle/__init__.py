"""CPU oracle for the GMDN fast-weight state scan.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the reference the
kernels are compared with (or, in the bench, as the timed CPU baseline),
never as a product path.

The oracle restates the reference algorithm in PyTorch on the CPU (any float
dtype; tests use float64 for tight checks and float32 for the reference's own
CPU precision).  Each function cites the reference file:line it follows.

Pinning (how the oracle itself is checked, see tests/test_oracle_*.py):

* ``scan.scan_forward``     -- closed forms (K=0 prefix sums, linearity in U,
                               adam sign descent, muon m=0, constant-G EMAs),
                               msign against an SVD restatement.
* ``scan.msign_sq``         -- SVD closed form ``P diag(p^ns(s/(|M|_F+eps))) R^T``
                               and the scalar recurrence for ``c*I``.
* ``scan.scan_backward``    -- two derivations: torch autograd of
                               ``scan_forward`` and the hand VJP; plus
                               ``torch.autograd.gradcheck`` in float64.
* ``chunk.mixer_core``      -- matrix form vs. E-form vs. token loop; the C=1,
                               alpha=1 case equals textbook DeltaNet.
* ``chunk`` gradients       -- autograd of the matrix form vs. gradcheck.

No golden vectors exist in the reference (its only test is differential,
Triton vs. eager, ``test.py:41-62``), so parity against absolute reference
values is pinned only through the checks above.
"""
