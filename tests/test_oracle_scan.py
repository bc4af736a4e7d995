"""Pins of the scan oracle (oracle/scan.py) by checks that do not retype it.

Each check is a closed form, a brute-force small case, an independent
derivation or an invariant, chosen so that a plausible mistake (transposed
product, dropped term, wrong constant) fails at least one of them; the last
tests plant such mistakes in the oracle and confirm the pins catch them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import scan as osc

D64 = torch.float64


def _gates(B, H, N, gen, lo=0.2, hi=0.9):
    return [lo + (hi - lo) * torch.rand(B, H, N, generator=gen, dtype=D64) for _ in range(4)]


def test_delta_no_decay_brute_force():
    """a = 0: S_1 = U_0, S_2 = U_1 - U_0 K_1, S_3 = U_2 - S_2 K_2 -- pins the
    orientation of the S K product on non-symmetric K."""
    gen = torch.Generator().manual_seed(0)
    U = torch.randn(1, 1, 4, 5, 5, generator=gen, dtype=D64)
    K = torch.randn(1, 1, 4, 5, 5, generator=gen, dtype=D64)
    z = torch.zeros(1, 1, 4, dtype=D64)
    S = osc.scan_forward(U, K, z, z, z, z, 0, 0)[0, 0].numpy()
    u, k = U[0, 0].numpy(), K[0, 0].numpy()
    s2 = u[1] - u[0] @ k[1]
    assert np.allclose(S[0], 0)
    assert np.allclose(S[1], u[0])
    assert np.allclose(S[2], s2)
    assert np.allclose(S[3], u[2] - s2 @ k[2])


def test_delta_k_zero_closed_form():
    """K = 0: S_i = sum_{j<i} (prod_{l=j+1}^{i-1} a_l) U_j; a = 1 is a prefix sum."""
    gen = torch.Generator().manual_seed(1)
    B, H, N, d = 2, 3, 7, 4
    U = torch.randn(B, H, N, d, d, generator=gen, dtype=D64)
    K = torch.zeros_like(U)
    a, b, m, n = _gates(B, H, N, gen)
    S = osc.scan_forward(U, K, a, b, m, n, 0, 3)
    for i in range(N):
        exp = torch.zeros(B, H, d, d, dtype=D64)
        for j in range(i):
            w = torch.prod(a[:, :, j + 1:i], dim=-1) if j + 1 < i else torch.ones(B, H, dtype=D64)
            exp = exp + w[..., None, None] * U[:, :, j]
        assert torch.allclose(S[:, :, i], exp, atol=1e-12)
    S1 = osc.scan_forward(U, K, torch.ones_like(a), b, m, n, 0, 3)
    assert torch.allclose(S1[:, :, 1:], torch.cumsum(U, dim=2)[:, :, :-1], atol=1e-12)


def test_delta_linear_in_U():
    gen = torch.Generator().manual_seed(2)
    U1, U2, K = (torch.randn(1, 2, 5, 6, 6, generator=gen, dtype=D64) * 0.3 for _ in range(3))
    a, b, m, n = _gates(1, 2, 5, gen)
    f = lambda U: osc.scan_forward(U, K, a, b, m, n, 0, 0)
    assert torch.allclose(f(2.0 * U1 - 3.0 * U2), 2.0 * f(U1) - 3.0 * f(U2), atol=1e-10)


@pytest.mark.parametrize("ns", [0, 1, 3, 5])
def test_msign_matches_svd_closed_form(ns):
    gen = torch.Generator().manual_seed(3 + ns)
    for d in (4, 16):
        M = torch.randn(d, d, generator=gen, dtype=D64)
        X = osc.msign_sq(M, ns).numpy()
        assert np.allclose(X, osc.msign_svd(M.numpy(), ns), atol=1e-10)


def test_msign_scaled_identity_scalar_recurrence():
    d, c = 8, 2.5
    x = c / (c * math.sqrt(d) + osc.EPS_NORM)
    for _ in range(5):
        x = 3.4445 * x - 4.7750 * x ** 3 + 2.0315 * x ** 5
    X = osc.msign_sq(c * torch.eye(d, dtype=D64), 5)
    assert torch.allclose(X, x * torch.eye(d, dtype=D64), atol=1e-12)


def test_msign_polar_factor_limit():
    """NS drives singular values into the quintic's band around 1 (the
    coefficients oscillate in roughly [0.7, 1.2] instead of converging), so
    the result is close to the orthogonal polar factor P R^T."""
    gen = torch.Generator().manual_seed(4)
    M = torch.randn(16, 16, generator=gen, dtype=D64)
    s = np.linalg.svd(osc.msign_sq(M, 8).numpy(), compute_uv=False)
    assert s.min() > 0.6 and s.max() < 1.25


def test_adam_zero_moments_sign_descent():
    """m = n = 0: M = G, V = G^2, so S_1 = b_0 U_0 / (|U_0| + 1e-6)."""
    gen = torch.Generator().manual_seed(5)
    U = torch.randn(1, 1, 2, 4, 4, generator=gen, dtype=D64)
    K = torch.randn_like(U)
    a = torch.full((1, 1, 2), 0.7, dtype=D64)
    b = torch.full((1, 1, 2), 0.4, dtype=D64)
    z = torch.zeros(1, 1, 2, dtype=D64)
    S = osc.scan_forward(U, K, a, b, z, z, 2, 0)
    assert torch.allclose(S[0, 0, 1], 0.4 * U[0, 0, 0] / (U[0, 0, 0].abs() + 1e-6), atol=1e-12)


def test_adam_constant_gradient_closed_form_emas():
    """K = 0 and constant U make G constant: M_i = (1 - m^i) G, V_i = (1 - n^i) G^2.
    With a = 0: S_{i+1} = b (1 - m^{i+1}) G / (sqrt(1 - n^{i+1}) |G| + eps)."""
    gen = torch.Generator().manual_seed(6)
    N = 6
    G = torch.randn(4, 4, generator=gen, dtype=D64)
    U = G.expand(1, 1, N, 4, 4).clone()
    K = torch.zeros_like(U)
    m, n, bb = 0.8, 0.95, 0.3
    full = lambda v: torch.full((1, 1, N), v, dtype=D64)
    S, M_all, V_all = osc.scan_forward(U, K, full(0.0), full(bb), full(m), full(n), 2, 0, return_moments=True)
    for i in range(N - 1):
        Mi = (1 - m ** (i + 1)) * G
        Vi = (1 - n ** (i + 1)) * G * G
        assert torch.allclose(M_all[0, 0, i + 1], Mi, atol=1e-12)
        assert torch.allclose(V_all[0, 0, i + 1], Vi, atol=1e-12)
        assert torch.allclose(S[0, 0, i + 1], bb * Mi / (Vi.sqrt() + osc.EPS_ADAM), atol=1e-12)


def test_muon_zero_momentum_is_msign_of_chunk_gradient():
    gen = torch.Generator().manual_seed(7)
    U = torch.randn(1, 1, 2, 6, 6, generator=gen, dtype=D64)
    K = torch.randn_like(U)
    z = torch.zeros(1, 1, 2, dtype=D64)
    b = torch.full((1, 1, 2), 0.5, dtype=D64)
    S = osc.scan_forward(U, K, z, b, z, z, 1, 5)
    assert np.allclose(S[0, 0, 1].numpy(), 0.5 * osc.msign_svd(U[0, 0, 0].numpy(), 5), atol=1e-10)


def _diag_scalar_scan(u, k, a, b, m, n, rule, ns):
    """Closed form of the scan on diagonal U_i, K_i: every matrix stays
    diagonal, so each diagonal entry follows its own scalar recurrence, and
    msign of a diagonal matrix D is diag(sign(d) p^ns(|d| / (|d|_2 + eps)))
    (its SVD is the entries' magnitudes).  u, k: (N, dh) numpy; a..n: (N,)."""
    ca, cb, cc = osc.NS_COEFFS
    N, dh = u.shape
    s, mm, vv = np.zeros(dh), np.zeros(dh), np.zeros(dh)
    out = []
    for i in range(N):
        out.append(s.copy())
        g = u[i] - s * k[i]
        if rule == 0:
            s = a[i] * s + g
        elif rule == 1:
            mm = m[i] * mm + g
            x = np.abs(mm) / (np.sqrt((mm ** 2).sum()) + osc.EPS_NORM)
            for _ in range(ns):
                x = ca * x + cb * x ** 3 + cc * x ** 5
            s = a[i] * s + b[i] * np.sign(mm) * x
        else:
            mm = m[i] * mm + (1 - m[i]) * g
            vv = n[i] * vv + (1 - n[i]) * g * g
            s = a[i] * s + b[i] * mm / (np.sqrt(vv) + osc.EPS_ADAM)
    return np.stack(out)


@pytest.mark.parametrize("rule,ns", [(0, 0), (1, 1), (1, 3), (1, 5), (2, 0)])
def test_diagonal_inputs_reduce_to_scalar_recurrences(rule, ns):
    """Diagonal U_i, K_i with momentum gates m far from 0 (0.3 .. 0.95) and
    signs of U mixed, so the momentum and moment recurrences change both the
    relative sizes and the signs of the entries that msign / the adam ratio
    see: pins the m != 0 recurrences of muon and adam in closed form."""
    gen = torch.Generator().manual_seed(11)
    N, dh = 7, 6
    u = torch.randn(N, dh, generator=gen, dtype=D64).numpy()
    k = (0.5 * torch.rand(N, dh, generator=gen, dtype=D64)).numpy()
    a, b, m, n = (0.3 + 0.65 * torch.rand(N, generator=gen, dtype=D64) for _ in range(4))
    U = torch.diag_embed(torch.from_numpy(u))[None, None]
    K = torch.diag_embed(torch.from_numpy(k))[None, None]
    S = osc.scan_forward(U, K, a[None, None], b[None, None], m[None, None], n[None, None], rule, ns)[0, 0]
    want = _diag_scalar_scan(u, k, a.numpy(), b.numpy(), m.numpy(), n.numpy(), rule, ns)
    assert np.allclose(torch.diagonal(S, dim1=-2, dim2=-1).numpy(), want, atol=1e-12)
    off = S - torch.diag_embed(torch.diagonal(S, dim1=-2, dim2=-1))
    assert off.abs().max().item() == 0.0


def test_diagonal_pin_catches_dropped_muon_momentum(monkeypatch):
    """Plant m = 0 in the oracle's muon update: the diagonal closed form must
    reject it."""
    gen = torch.Generator().manual_seed(12)
    N, dh = 6, 5
    u = torch.randn(N, dh, generator=gen, dtype=D64).numpy()
    k = np.zeros((N, dh))
    a, b, m, n = (0.5 + 0.4 * torch.rand(N, generator=gen, dtype=D64) for _ in range(4))
    U = torch.diag_embed(torch.from_numpy(u))[None, None]
    K = torch.zeros_like(U)
    want = _diag_scalar_scan(u, k, a.numpy(), b.numpy(), m.numpy(), n.numpy(), 1, 3)
    S = osc.scan_forward(U, K, a[None, None], b[None, None], torch.zeros_like(m)[None, None], n[None, None], 1, 3)
    assert not np.allclose(torch.diagonal(S[0, 0], dim1=-2, dim2=-1).numpy(), want, atol=1e-6)


@pytest.mark.parametrize("rule,ns", [(0, 0), (1, 0), (1, 2), (1, 3), (2, 0)])
def test_manual_backward_equals_autograd(rule, ns):
    """Two derivations of the VJP: the hand reverse scan (fast_scan.py:134-186)
    and torch autograd of the forward."""
    gen = torch.Generator().manual_seed(10 + rule)
    ins = [t.double() for t in osc.make_scan_inputs(2, 2, 5, 16, 8, generator=gen)]
    xs = [t.clone().requires_grad_(True) for t in ins]
    S = osc.scan_forward(*xs, rule, ns)
    gS = torch.randn(S.shape, generator=gen, dtype=D64)
    auto = torch.autograd.grad(S, xs, gS, allow_unused=True)
    S_all, M_all, V_all = osc.scan_forward(*ins, rule, ns, return_moments=True)
    man = osc.scan_backward(*ins, S_all, M_all, V_all, gS, rule, ns)
    for g_a, g_m, t in zip(auto, man, ins):
        g_a = torch.zeros_like(t) if g_a is None else g_a
        assert torch.allclose(g_a, g_m, atol=1e-10, rtol=1e-8)


@pytest.mark.parametrize("rule,ns", [(0, 0), (1, 2), (2, 0)])
def test_scan_gradcheck(rule, ns):
    gen = torch.Generator().manual_seed(20 + rule)
    ins = [t.double().requires_grad_(True) for t in osc.make_scan_inputs(1, 1, 3, 8, 4, generator=gen)]
    assert torch.autograd.gradcheck(lambda *x: osc.scan_forward(*x, rule, ns), ins, eps=1e-6, atol=1e-5)


def test_msign_vjp_gradcheck():
    gen = torch.Generator().manual_seed(30)
    M = torch.randn(5, 5, generator=gen, dtype=D64, requires_grad=True)
    Yb = torch.randn(5, 5, generator=gen, dtype=D64)
    auto = torch.autograd.grad(osc.msign_sq(M, 3), M, Yb)[0]
    assert torch.allclose(osc.msign_vjp(M.detach(), Yb, 3), auto, atol=1e-10)
    assert torch.autograd.gradcheck(lambda x: osc.msign_sq(x, 3), (M,))


def test_make_scan_inputs_are_psd_and_bounded():
    gen = torch.Generator().manual_seed(40)
    U, K, a, b, m, n = osc.make_scan_inputs(2, 3, 4, 64, 32, generator=gen, dtype=D64)
    assert torch.allclose(K, K.transpose(-1, -2), atol=1e-6)  # built in fp32
    ev = torch.linalg.eigvalsh(K)
    assert ev.min() > -1e-6 and ev.max() < 1.5
    assert (a >= 0.75).all() and (a < 0.95).all() and (b >= 0.2).all() and (b < 0.7).all()


def test_rel_err_metric():
    y = torch.tensor([1.0, -4.0, 2.0])
    x = torch.tensor([1.5, -4.0, 2.0])
    assert osc.rel_err(x, y) == pytest.approx(0.5 / 4.0)


# ------------------------------------------------------------ planted mistakes
def test_pins_catch_transposed_state_product(monkeypatch):
    """An oracle computing S K^T instead of S K fails the brute-force case."""
    orig = osc.scan_forward

    def bad(U, K, a, b, m, n, rule, ns, return_moments=False):
        return orig(U, K.transpose(-1, -2), a, b, m, n, rule, ns, return_moments)

    monkeypatch.setattr(osc, "scan_forward", bad)
    with pytest.raises(AssertionError):
        test_delta_no_decay_brute_force()


def test_pins_catch_wrong_ns_coefficient(monkeypatch):
    """A quintic with c = 2.0 instead of 2.0315 fails the SVD closed form."""
    def bad(X):
        P = torch.matmul(X, X.transpose(-1, -2))
        return 3.4445 * X + torch.matmul(-4.7750 * P + 2.0 * torch.matmul(P, P), X)

    monkeypatch.setattr(osc, "ns_iterate", bad)
    with pytest.raises(AssertionError):
        test_msign_matches_svd_closed_form(3)


def test_pins_catch_wrong_adam_momentum(monkeypatch):
    """An adam EMA with the wrong momentum fails the closed-form EMAs."""
    orig = osc.scan_forward

    def bad(U, K, a, b, m, n, rule, ns, return_moments=False):
        return orig(U, K, a, b, m * 0.5 if rule == 2 else m, n, rule, ns, return_moments)

    monkeypatch.setattr(osc, "scan_forward", bad)
    with pytest.raises(AssertionError):
        test_adam_constant_gradient_closed_form_emas()
