"""Pins of the outer-Muon oracle (oracle/muon.py) on the CPU.

* ``msign`` against its thin-SVD closed form (an independent derivation) for
  square, wide, tall and single-row/column matrices and step counts 0..5, and
  against the scalar closed form for scaled orthonormal rows.
* The same check rejects a planted mistake (a flipped coefficient sign).
* ``muon_step`` against hand-derived closed forms of two optimizer steps on
  rank-one gradients with orthogonal singular vectors, which pin the
  momentum recurrence, the Nesterov form, the max(1, rows/cols)^0.5 scale and
  the weight-decay order.
"""
import numpy as np
import pytest
import torch

from oracle import muon as om

SHAPES = [(5, 5), (3, 7), (7, 3), (1, 4), (4, 1), (24, 64), (64, 24)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("steps", [0, 1, 3, 5])
def test_msign_matches_svd_closed_form(shape, steps):
    g = torch.Generator().manual_seed(hash((shape, steps)) % 2**31)
    M = torch.randn(*shape, generator=g, dtype=torch.float64)
    got = om.msign(M, steps, compute_dtype=torch.float64).numpy()
    ref = om.msign_svd(M.numpy(), steps)
    assert np.abs(got - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())


def test_msign_batched_matches_per_matrix():
    M = torch.randn(3, 6, 10, dtype=torch.float64)
    got = om.msign(M, 5, compute_dtype=torch.float64)
    for i in range(3):
        torch.testing.assert_close(got[i], om.msign(M[i], 5, compute_dtype=torch.float64), rtol=0, atol=1e-14)


def test_msign_transpose_symmetry():
    M = torch.randn(9, 4, dtype=torch.float64)
    torch.testing.assert_close(om.msign(M, 5, compute_dtype=torch.float64),
                               om.msign(M.T, 5, compute_dtype=torch.float64).T, rtol=0, atol=1e-13)


def test_msign_scaled_orthonormal_rows():
    # M = c Q with orthonormal rows: every singular value is c, |M|_F = c sqrt(m)
    m, n, c = 6, 11, 2.5
    Q, _ = np.linalg.qr(np.random.default_rng(0).standard_normal((n, m)))
    M = c * Q.T
    x = om.ns_poly(c / (c * np.sqrt(m) + om.EPS), 5)
    got = om.msign(torch.from_numpy(M), 5, compute_dtype=torch.float64).numpy()
    assert np.abs(got - x * Q.T).max() < 1e-12


def test_svd_check_rejects_flipped_coefficient():
    M = torch.randn(8, 12, dtype=torch.float64)
    a, b, c = om.NS_COEFFS
    X = M / M.norm()
    for _ in range(5):  # planted mistake: +b instead of b
        A = X @ X.T
        X = a * X + (-b * A + c * A @ A) @ X
    ref = om.msign_svd(M.numpy(), 5)
    assert np.abs(X.numpy() - ref).max() > 1e-2


def _unit(shape, i, j):
    E = torch.zeros(shape, dtype=torch.float64)
    E[i, j] = 1.0
    return E


@pytest.mark.parametrize("shape", [(3, 5), (5, 3)])
@pytest.mark.parametrize("nesterov", [True, False])
@pytest.mark.parametrize("wd", [0.0, 0.1])
def test_muon_step_closed_form(shape, nesterov, wd):
    lr, mom, steps = 0.05, 0.9, 5
    a1, a2 = 0.7, 1.3
    E00, E11 = _unit(shape, 0, 0), _unit(shape, 1, 1)
    p0 = torch.randn(shape, dtype=torch.float64)
    p = p0.clone()
    scale = max(1.0, shape[0] / shape[1]) ** 0.5
    kw = dict(lr=lr, momentum=mom, nesterov=nesterov, weight_decay=wd, ns_steps=steps,
              compute_dtype=torch.float64)
    bufs = om.muon_step([p], [a1 * E00], [None], **kw)
    # step 1: buf = g1; u = g1 + mom buf (Nesterov) or buf -- rank one
    s1 = (1 + mom) * a1 if nesterov else a1
    exp = p0 * (1 - lr * wd) - lr * scale * om.ns_poly(s1 / (s1 + om.EPS), steps) * E00
    torch.testing.assert_close(p, exp, rtol=0, atol=1e-13)
    bufs = om.muon_step([p], [a2 * E11], bufs, **kw)
    # step 2: buf = mom a1 E00 + a2 E11; u = g2 + mom buf or buf
    sa, sb = (mom * mom * a1, (1 + mom) * a2) if nesterov else (mom * a1, a2)
    nrm = np.hypot(sa, sb) + om.EPS
    exp = exp * (1 - lr * wd) - lr * scale * (om.ns_poly(sa / nrm, steps) * E00 + om.ns_poly(sb / nrm, steps) * E11)
    torch.testing.assert_close(p, exp, rtol=0, atol=1e-13)
    torch.testing.assert_close(bufs[0], mom * a1 * E00 + a2 * E11, rtol=0, atol=1e-15)
