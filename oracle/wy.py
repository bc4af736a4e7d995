"""Oracle: the token-exact gated delta rule and its chunked WY/UT form.

TEST INFRASTRUCTURE ONLY -- imported by tests/, never by the shipped package.

The reference trains the chunk-frozen E-form and leaves the exact WY/UT
transform out on purpose (train_ablation.py:12-18).  This module restates
the textbook token recurrence the WY mode computes exactly, per (b, h), with
S (d_v x d_k), gates alpha_t = exp(max(g_t, log 1e-6)) and beta_t:

    S_t = alpha_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T,   o_t = S_t q_t

(``token_scan``), and the chunked WY form of the same recurrence
(``wy_chunked``): within a chunk starting from S_0, with gamma_t the decay
product from the chunk start and Gamma[t, s] = gamma_t / gamma_s,

    A   = strict_lower(diag(beta) (K K^T * Gamma)),   T = (I + A)^-1
    U   = T diag(beta) V,   W = T diag(beta gamma) K
    X   = U - W S_0^T                       (X_t = beta_t (v_t - alpha_t S_{t-1} k_t))
    O   = diag(gamma) Q S_0^T + lower_incl(Q K^T * Gamma) X
    S_C = gamma_C S_0 + X^T diag(gamma_C / gamma) K

The chunked form equals the token recurrence for every chunk length; the
tests pin it that way and with closed forms.
"""
from __future__ import annotations

import math

import torch

LOG_FLOOR = math.log(1e-6)


def token_scan(q, k, v, beta, g):
    """o (B, H, T, d) of the token recurrence; q, k, v (B, H, T, d), beta, g
    (B, H, T) (g = log alpha, clamped at log 1e-6)."""
    B, H, T, d = q.shape
    S = q.new_zeros(B, H, d, d)
    eye = torch.eye(d, dtype=q.dtype, device=q.device)
    out = []
    for t in range(T):
        a = torch.exp(torch.clamp(g[:, :, t], min=LOG_FLOOR))[..., None, None]
        b = beta[:, :, t][..., None, None]
        kt, vt, qt = k[:, :, t], v[:, :, t], q[:, :, t]
        S = a * S @ (eye - b * kt[..., :, None] * kt[..., None, :]) + b * vt[..., :, None] * kt[..., None, :]
        out.append((S @ qt[..., :, None])[..., 0])
    return torch.stack(out, dim=2)


def wy_chunk_terms(q, k, v, beta, g, C: int):
    """The per-chunk WY quantities (every tensor with a chunk axis N = T / C):
    gamma (B, H, N, C), A, T, M (B, H, N, C, C), U, W (B, H, N, C, d)."""
    B, H, Tn, d = q.shape
    N = Tn // C
    Q, K, V = (x.reshape(B, H, N, C, d) for x in (q, k, v))
    bt = beta.reshape(B, H, N, C)
    gc = torch.cumsum(torch.clamp(g, min=LOG_FLOOR).reshape(B, H, N, C), -1)
    gamma = torch.exp(gc)
    strict = torch.ones(C, C, dtype=torch.bool, device=q.device).tril(-1)
    incl = torch.ones(C, C, dtype=torch.bool, device=q.device).tril()
    # the exponent is masked to the causal entries (s <= t) before exp
    Gam = torch.exp(torch.where(incl, gc[..., :, None] - gc[..., None, :], float("-inf")))
    A = torch.where(strict, bt[..., :, None] * (K @ K.transpose(-1, -2)) * Gam, 0.0)
    eye = torch.eye(C, dtype=q.dtype, device=q.device)
    T = torch.linalg.solve_triangular(eye + A, eye.expand_as(A), upper=False, unitriangular=True)
    U = T @ (bt[..., None] * V)
    W = T @ ((bt * gamma)[..., None] * K)
    M = torch.where(incl, (Q @ K.transpose(-1, -2)) * Gam, 0.0)
    return dict(gamma=gamma, A=A, T=T, U=U, W=W, M=M, Q=Q, K=K)


def wy_chunked(q, k, v, beta, g, C: int = 64):
    """o (B, H, T, d) of the chunked WY form (equal to ``token_scan``)."""
    B, H, Tn, d = q.shape
    z = wy_chunk_terms(q, k, v, beta, g, C)
    N = Tn // C
    S = q.new_zeros(B, H, d, d)
    outs = []
    for i in range(N):
        gam = z["gamma"][:, :, i]
        X = z["U"][:, :, i] - z["W"][:, :, i] @ S.transpose(-1, -2)
        O = gam[..., None] * (z["Q"][:, :, i] @ S.transpose(-1, -2)) + z["M"][:, :, i] @ X
        kd = (gam[..., -1:] / gam)[..., None] * z["K"][:, :, i]
        S = gam[..., -1, None, None] * S + X.transpose(-1, -2) @ kd
        outs.append(O)
    return torch.stack(outs, dim=2).reshape(B, H, Tn, d)


def make_wy_inputs(B, H, T, d, generator=None, dtype=torch.float64):
    """q, k L2-normalised N(0, 1); v N(0, 1); beta = sigmoid(N(0, 1));
    g = logsigmoid(N(0, 1) + 3) (the benchmark configurations' draws)."""
    gen = generator
    q = torch.nn.functional.normalize(torch.randn(B, H, T, d, generator=gen, dtype=dtype), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, H, T, d, generator=gen, dtype=dtype), dim=-1)
    v = torch.randn(B, H, T, d, generator=gen, dtype=dtype)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=gen, dtype=dtype))
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen, dtype=dtype) + 3)
    return q, k, v, beta, g
