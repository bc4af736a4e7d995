"""Oracle: the outer Muon optimizer's msign and update (reference
``train_ablation.py:60-73`` and ``:264-288``).

TEST INFRASTRUCTURE ONLY -- imported by tests/ and the bench's CPU baseline,
never by the shipped package.

``msign`` restates the reference function line by line (any float dtype and
device; leading batch dimensions allowed, each matrix normalised by its own
Frobenius norm).  ``msign_svd`` is its closed form from the thin SVD, an
independent derivation used to pin it; ``muon_step`` restates one
``Muon.step`` over a list of parameters, one parameter at a time as the
reference does.
"""
from __future__ import annotations

import numpy as np
import torch

# train_ablation.py:66
NS_COEFFS = (3.4445, -4.7750, 2.0315)
EPS = 1e-7


def msign(M: torch.Tensor, steps: int = 5, eps: float = EPS, compute_dtype=torch.float32) -> torch.Tensor:
    """train_ablation.py:60-73: X = M in ``compute_dtype`` (the reference uses
    float32), transposed when it has more rows than columns, divided by its
    Frobenius norm + eps, then ``steps`` of ``A = X X^T;
    X = a X + (b A + c A A) X``; transposed back and cast to M's dtype."""
    dt = M.dtype
    X = M.to(compute_dtype)
    transposed = X.shape[-2] > X.shape[-1]
    if transposed:
        X = X.mT
    X = X / (X.norm(dim=(-2, -1), keepdim=True) + eps)
    a, b, c = NS_COEFFS
    for _ in range(steps):
        A = X @ X.mT
        X = a * X + (b * A + c * (A @ A)) @ X
    if transposed:
        X = X.mT
    return X.to(dt)


def ns_poly(x, steps: int):
    """The scalar map every NS step applies to each singular value:
    ``p(x) = a x + b x^3 + c x^5``, ``steps`` times."""
    a, b, c = NS_COEFFS
    for _ in range(steps):
        x = a * x + b * x ** 3 + c * x ** 5
    return x


def msign_svd(M: np.ndarray, steps: int = 5, eps: float = EPS) -> np.ndarray:
    """Closed form of ``msign`` for one matrix of any shape, in float64: with
    the thin SVD ``M = P diag(s) R^T``, ``msign(M) = P diag(p^steps(s / (|M|_F
    + eps))) R^T`` (each NS step keeps the singular vectors and maps the
    singular values through p; transposing changes neither)."""
    M = np.asarray(M, dtype=np.float64)
    P, s, Rt = np.linalg.svd(M, full_matrices=False)
    x = ns_poly(s / (np.sqrt((M ** 2).sum()) + eps), steps)
    return (P * x) @ Rt


def muon_step(params, grads, bufs, lr=0.02, momentum=0.95, nesterov=True, weight_decay=0.0, ns_steps=5,
              compute_dtype=torch.float32):
    """One ``Muon.step`` (train_ablation.py:271-288) over parallel lists of
    parameters, gradients and momentum buffers (``None`` for a fresh state),
    updating ``params`` in place and returning the new buffers."""
    out = []
    for p, g, buf in zip(params, grads, bufs):
        if buf is None:
            buf = torch.zeros_like(g)
        buf = buf * momentum + g
        u = g + momentum * buf if nesterov else buf
        u = msign(u, ns_steps, compute_dtype=compute_dtype)
        scale = max(1.0, p.shape[0] / p.shape[1]) ** 0.5
        if weight_decay:
            p.mul_(1 - lr * weight_decay)
        p.add_(u.to(p.dtype), alpha=-lr * scale)
        out.append(buf)
    return out
