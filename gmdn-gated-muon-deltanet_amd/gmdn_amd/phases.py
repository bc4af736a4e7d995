"""Phases 1 and 3 of the mixer core in matrix form, and their VJP in closed
form, for the muon rule's backward (reference train_ablation.py:142-187).

The fused muon forward (HIP, ``chunk_fwd_muon`` + ``chunk_out``) never forms
the per-chunk products below; the backward recomputes them in float32 and
differentiates through the drop-in muon scan's backward kernels:

    per chunk, tokens t, s (C = 64), lg = max(g, log 1e-6), lm = max(gmu, log 1e-6):
      a = exp(sum lg), b = mean beta, m = exp(sum lm), w_t = exp(sum_{s>t} lm_s)
      A  = tril(Q K^T) diag(beta)          (train_ablation.py:161-163)
      Kw = K^T diag(w) K,  Uv = V^T diag(w) K                      (:164-165)
      Qt = Q - A K,  Ov = A V                                      (:166-167)
      o  = Qt S_i^T + Ov                                           (:186)

The VJP is written out (no autograd inside), so that the whole backward is a
plain sequence of tensor operations.
"""
from __future__ import annotations

import math

import torch

CHUNK = 64
LOG_FLOOR = math.log(1e-6)


def _f(t):
    """float32 working copy (float64 inputs keep their precision)."""
    return t if t.dtype == torch.float64 else t.float()


def phase1(q, k, v, beta, g, gmu):
    """Float32 per-chunk quantities from (B, H, T, d) q, k, v and (B, H, T)
    gates.  Returns a dict with Q, K, V (B, H, N, C, d), A (B, H, N, C, C),
    Kw, Uv (B, H, N, d, d), Qt, Ov (B, H, N, C, d), a, b, m (B, H, N) and the
    token weights w (B, H, N, C)."""
    B, H, T, d = q.shape
    N = T // CHUNK
    Q, K, V = (_f(t).reshape(B, H, N, CHUNK, d) for t in (q, k, v))
    bt = _f(beta).reshape(B, H, N, CHUNK)
    lg = torch.clamp(_f(g), min=LOG_FLOOR).reshape(B, H, N, CHUNK)
    lm = torch.clamp(_f(gmu), min=LOG_FLOOR).reshape(B, H, N, CHUNK)
    a = lg.sum(-1).exp()
    b = bt.mean(-1)
    msum = lm.sum(-1)
    m = msum.exp()
    w = torch.exp(msum.unsqueeze(-1) - torch.cumsum(lm, -1))
    causal = torch.ones(CHUNK, CHUNK, dtype=torch.bool, device=q.device).tril()
    A = torch.where(causal, torch.matmul(Q, K.transpose(-1, -2)), 0.0) * bt.unsqueeze(-2)
    Kw = torch.matmul((K * w.unsqueeze(-1)).transpose(-1, -2), K)
    Uv = torch.matmul((V * w.unsqueeze(-1)).transpose(-1, -2), K)
    Qt = Q - torch.matmul(A, K)
    Ov = torch.matmul(A, V)
    return dict(Q=Q, K=K, V=V, bt=bt, A=A, Kw=Kw, Uv=Uv, Qt=Qt, Ov=Ov, a=a, b=b, m=m, w=w, causal=causal)


def phase1_vjp(ph, g, gmu, dKw, dUv, dQt, dOv, da, db, dm):
    """Cotangents of q, k, v (B, H, T, d) and beta, g, gmu (B, H, T) given those
    of Kw, Uv (B, H, N, d, d), Qt, Ov (B, H, N, C, d) and a, b, m (B, H, N)."""
    Q, K, V, bt, A, w = ph["Q"], ph["K"], ph["V"], ph["bt"], ph["A"], ph["w"]
    B, H, N, C, d = Q.shape
    KT = K.transpose(-1, -2)
    # A = mask(Q K^T) diag(beta): dA from Qt = Q - A K and Ov = A V
    dA = torch.where(ph["causal"], torch.matmul(dOv, V.transpose(-1, -2)) - torch.matmul(dQt, KT), 0.0)
    P = torch.where(ph["causal"], torch.matmul(Q, KT), 0.0)
    dbeta = (dA * P).sum(-2) + (db / C).unsqueeze(-1)
    dP = dA * bt.unsqueeze(-2)
    dQ = dQt + torch.matmul(dP, K)
    dK = torch.matmul(dP.transpose(-1, -2), Q) - torch.matmul(A.transpose(-1, -2), dQt)
    dV = torch.matmul(A.transpose(-1, -2), dOv)
    # Kw = K^T diag(w) K, Uv = V^T diag(w) K
    wk = w.unsqueeze(-1)
    KdKw = torch.matmul(K, dKw)
    dK = dK + wk * (KdKw + torch.matmul(K, dKw.transpose(-1, -2))) + wk * torch.matmul(V, dUv)
    dV = dV + wk * torch.matmul(K, dUv.transpose(-1, -2))
    dw = (KdKw * K).sum(-1) + (torch.matmul(V, dUv) * K).sum(-1)
    # gates: a = exp(sum lg), m = exp(sum lm), w_t = exp(sum_{s>t} lm_s)
    dlg = (da * ph["a"]).unsqueeze(-1).expand(B, H, N, C)
    dww = dw * w
    dlm = (dm * ph["m"]).unsqueeze(-1) + (torch.cumsum(dww, -1) - dww)
    T = N * C
    dg = torch.where(_f(g).reshape(B, H, N, C) >= LOG_FLOOR, dlg, 0.0).reshape(B, H, T)
    dgmu = torch.where(_f(gmu).reshape(B, H, N, C) >= LOG_FLOOR, dlm, 0.0).reshape(B, H, T)
    shape = (B, H, T, d)
    return dQ.reshape(shape), dK.reshape(shape), dV.reshape(shape), dbeta.reshape(B, H, T), dg, dgmu


def phase3_vjp(ph, S_all, dO):
    """o = Qt S_i^T + Ov: cotangents of Qt, Ov and of the states S_i."""
    B, H, N, C, d = ph["Q"].shape
    dOf = _f(dO).reshape(B, H, N, C, d)
    gS = torch.matmul(dOf.transpose(-1, -2), ph["Qt"])
    dQt = torch.matmul(dOf, S_all)
    return dQt, dOf, gS
