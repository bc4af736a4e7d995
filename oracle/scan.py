"""Oracle: the chunk-level fast-weight state scan (reference ``fast_scan.py``).

TEST INFRASTRUCTURE ONLY -- imported by tests/, smoke() and the bench's CPU
baseline, never by the shipped package.

State convention (reference ``fast_scan.py:5-15``): per (batch, head) the
state ``S`` is a ``dh x dh`` matrix whose rows index d_v and columns d_k.
For chunk ``i`` with inputs ``U_i, K_i`` (dh x dh) and scalars
``a_i, b_i, m_i, n_i``:

    G_i = U_i - S_i K_i
    delta: S_{i+1} = a_i S_i + G_i
    muon : M_{i+1} = m_i M_i + G_i ;        S_{i+1} = a_i S_i + b_i msign(M_{i+1})
    adam : M_{i+1} = m_i M_i + (1-m_i) G_i ; V_{i+1} = n_i V_i + (1-n_i) G_i^2
           S_{i+1} = a_i S_i + b_i M_{i+1} / (sqrt(V_{i+1}) + 1e-6)

and the scan returns the PRE-update states ``S_0 .. S_{N-1}`` with
``S_0 = M_0 = V_0 = 0``.
"""
from __future__ import annotations

import numpy as np
import torch

# fast_scan.py:32-34
NS_COEFFS = (3.4445, -4.7750, 2.0315)
EPS_NORM = 1e-7
EPS_ADAM = 1e-6

RULES = {"delta": 0, "muon": 1, "adam": 2}


def _frob(X: torch.Tensor) -> torch.Tensor:
    return torch.sqrt((X * X).sum(dim=(-2, -1), keepdim=True))


def ns_iterate(X: torch.Tensor) -> torch.Tensor:
    """One quintic Newton-Schulz step ``X <- a X + (b XX^T + c (XX^T)^2) X``
    (fast_scan.py:67-68, :102-104)."""
    ca, cb, cc = NS_COEFFS
    P = torch.matmul(X, X.transpose(-1, -2))
    return ca * X + torch.matmul(cb * P + cc * torch.matmul(P, P), X)


def msign_sq(M: torch.Tensor, ns: int) -> torch.Tensor:
    """Square-matrix msign by ``ns`` quintic NS steps after Frobenius
    normalisation ``X0 = M / (|M|_F + 1e-7)`` (fast_scan.py:63-69)."""
    X = M / (_frob(M) + EPS_NORM)
    for _ in range(ns):
        X = ns_iterate(X)
    return X


def msign_svd(M: np.ndarray, ns: int) -> np.ndarray:
    """Closed form of ``msign_sq`` for one square matrix, from the SVD.

    Every NS step maps singular values through ``p(x) = a x + b x^3 + c x^5``
    and keeps the singular vectors, so with ``M = P diag(s) R^T``:
    ``msign_sq(M) = P diag(p^ns(s / (|M|_F + 1e-7))) R^T``.  Used only to pin
    ``msign_sq`` (a derivation independent of the matmul chain)."""
    ca, cb, cc = NS_COEFFS
    P, s, Rt = np.linalg.svd(np.asarray(M, dtype=np.float64))
    x = s / (np.sqrt((np.asarray(M, dtype=np.float64) ** 2).sum()) + EPS_NORM)
    for _ in range(ns):
        x = ca * x + cb * x ** 3 + cc * x ** 5
    return (P * x) @ Rt


def scan_forward(U, K, a, b, m, n, rule: int, ns: int, return_moments: bool = False):
    """Pre-update state stack (fast_scan.py:72-95).

    U, K: (B, H, N, dh, dh); a, b, m, n: (B, H, N).  Returns ``S_all`` of
    shape (B, H, N, dh, dh), or ``(S_all, M_all, V_all)`` with the
    pre-update moment stacks when ``return_moments`` (fast_scan.py:366-368
    keeps those for the backward).  Differentiable by torch autograd.
    """
    B, H, N, dh, _ = U.shape
    S = U.new_zeros(B, H, dh, dh)
    M = U.new_zeros(B, H, dh, dh)
    V = U.new_zeros(B, H, dh, dh)
    S_list, M_list, V_list = [], [], []
    for i in range(N):
        S_list.append(S)
        M_list.append(M)
        V_list.append(V)
        G = U[:, :, i] - torch.matmul(S, K[:, :, i])
        ai = a[:, :, i].unsqueeze(-1).unsqueeze(-1)
        if rule == 0:
            S = ai * S + G
        elif rule == 1:
            mi = m[:, :, i].unsqueeze(-1).unsqueeze(-1)
            bi = b[:, :, i].unsqueeze(-1).unsqueeze(-1)
            M = mi * M + G
            S = ai * S + bi * msign_sq(M, ns)
        elif rule == 2:
            mi = m[:, :, i].unsqueeze(-1).unsqueeze(-1)
            ni = n[:, :, i].unsqueeze(-1).unsqueeze(-1)
            bi = b[:, :, i].unsqueeze(-1).unsqueeze(-1)
            M = mi * M + (1.0 - mi) * G
            V = ni * V + (1.0 - ni) * G * G
            S = ai * S + bi * M / (torch.sqrt(V) + EPS_ADAM)
        else:
            raise ValueError(f"rule must be 0, 1 or 2, got {rule}")
    S_all = torch.stack(S_list, dim=2)
    if not return_moments:
        return S_all
    return S_all, torch.stack(M_list, dim=2), torch.stack(V_list, dim=2)


def msign_vjp(Mi: torch.Tensor, Ybar: torch.Tensor, ns: int) -> torch.Tensor:
    """Vector-Jacobian product of ``Y = msign_sq(Mi, ns)`` (fast_scan.py:107-131).

    Per NS step ``X' = a X + (b P + c P^2) X`` with ``P = X X^T`` (symmetric):
        Pbar = X'bar X^T
        Qbar = b Pbar + c (Pbar P + P Pbar)
        Xbar = a X'bar + (b P + c P^2) X'bar + (Qbar + Qbar^T) X
    and for ``X0 = Mi / (|Mi| + eps)``:
        Mbar = X0bar / nrm - <X0bar, Mi> / nrm^2 * Mi / max(|Mi|, 1e-12).
    The iterates are stored once here (the reference recomputes them, which
    gives the same values)."""
    ca, cb, cc = NS_COEFFS
    nf = _frob(Mi)
    nrm = nf + EPS_NORM
    X = Mi / nrm
    iterates = []
    for _ in range(ns):
        iterates.append(X)
        X = ns_iterate(X)
    Xbar = Ybar
    for Xk in reversed(iterates):
        P = torch.matmul(Xk, Xk.transpose(-1, -2))
        poly = cb * P + cc * torch.matmul(P, P)
        Pbar = torch.matmul(Xbar, Xk.transpose(-1, -2))
        Qbar = cb * Pbar + cc * (torch.matmul(Pbar, P) + torch.matmul(P, Pbar))
        Xbar = ca * Xbar + torch.matmul(poly, Xbar) + torch.matmul(Qbar + Qbar.transpose(-1, -2), Xk)
    inner = (Xbar * Mi).sum(dim=(-2, -1), keepdim=True)
    return Xbar / nrm - inner / (nrm * nrm) * (Mi / torch.clamp(nf, min=1e-12))


def scan_backward(U, K, a, b, m, n, S_all, M_all, V_all, gS, rule: int, ns: int):
    """Hand-derived reverse scan (fast_scan.py:134-186).

    Returns ``(dU, dK, da, db, dm, dn)``.  Gradients of scalars the rule does
    not use are zero (what autograd of ``scan_forward`` gives)."""
    B, H, N, dh, _ = U.shape
    dU = torch.zeros_like(U)
    dK = torch.zeros_like(K)
    da = torch.zeros_like(a)
    db = torch.zeros_like(b)
    dm = torch.zeros_like(m)
    dn = torch.zeros_like(n)
    Sb = U.new_zeros(B, H, dh, dh)      # dL/dS_{i+1}
    Mb = U.new_zeros(B, H, dh, dh)      # dL/dM_{i+1}
    Vb = U.new_zeros(B, H, dh, dh)      # dL/dV_{i+1}

    def col(t, i):
        return t[:, :, i].unsqueeze(-1).unsqueeze(-1)

    for i in range(N - 1, -1, -1):
        S = S_all[:, :, i]
        Ki = K[:, :, i]
        G = U[:, :, i] - torch.matmul(S, Ki)
        da[:, :, i] = (Sb * S).sum(dim=(-2, -1))
        if rule == 0:
            Gb = Sb
        elif rule == 1:
            Mp = M_all[:, :, i]
            Mi = col(m, i) * Mp + G
            db[:, :, i] = (Sb * msign_sq(Mi, ns)).sum(dim=(-2, -1))
            Mtot = Mb + msign_vjp(Mi, col(b, i) * Sb, ns)
            dm[:, :, i] = (Mtot * Mp).sum(dim=(-2, -1))
            Mb = col(m, i) * Mtot
            Gb = Mtot
        else:
            Mp, Vp = M_all[:, :, i], V_all[:, :, i]
            mi, ni, bi = col(m, i), col(n, i), col(b, i)
            Mi = mi * Mp + (1.0 - mi) * G
            Vi = ni * Vp + (1.0 - ni) * G * G
            root = torch.sqrt(Vi)
            den = root + EPS_ADAM
            db[:, :, i] = (Sb * (Mi / den)).sum(dim=(-2, -1))
            ub = bi * Sb
            Mtot = Mb + ub / den
            Vtot = Vb - ub * Mi / (den * den) / (2.0 * torch.clamp(root, min=1e-12))
            dm[:, :, i] = (Mtot * (Mp - G)).sum(dim=(-2, -1))
            dn[:, :, i] = (Vtot * (Vp - G * G)).sum(dim=(-2, -1))
            Mb = mi * Mtot
            Vb = ni * Vtot
            Gb = (1.0 - mi) * Mtot + (1.0 - ni) * 2.0 * G * Vtot
        dU[:, :, i] = Gb
        dK[:, :, i] = -torch.matmul(S.transpose(-1, -2), Gb)
        Sb = col(a, i) * Sb - torch.matmul(Gb, Ki.transpose(-1, -2)) + gS[:, :, i]
    return dU, dK, da, db, dm, dn


def make_scan_inputs(B=4, H=12, N=16, C=64, dh=64, generator=None, dtype=torch.float32):
    """``test.py:28-38``'s realistic input distribution, drawn on the CPU.

    ``K = k^T diag(w) k`` with L2-normalised k and ``w ~ U[0, 0.3)`` (PSD,
    spectral norm below about 1), ``U = (v/sqrt(dh))^T diag(w) k``, and gates
    a in [.75,.95), b in [.2,.7), m in [.3,.8), n in [.7,.9)."""
    g = generator
    k = torch.randn(B, H, N, C, dh, generator=g)
    k = k / torch.clamp(torch.sqrt((k * k).sum(-1, keepdim=True)), min=1e-12)
    v = torch.randn(B, H, N, C, dh, generator=g) / dh ** 0.5
    w = torch.rand(B, H, N, C, generator=g) * 0.3
    K = torch.matmul((k * w.unsqueeze(-1)).transpose(-1, -2), k)
    U = torch.matmul((v * w.unsqueeze(-1)).transpose(-1, -2), k)
    gates = [torch.rand(B, H, N, generator=g) * r + o
             for r, o in ((0.2, 0.75), (0.5, 0.2), (0.5, 0.3), (0.2, 0.7))]
    return [t.to(dtype) for t in [U, K] + gates]


def rel_err(x: torch.Tensor, y: torch.Tensor) -> float:
    """``max|x - y| / max|y|`` (test.py:24-25)."""
    x = x.double()
    y = y.double()
    return float((x - y).abs().max() / (y.abs().max() + 1e-30))
