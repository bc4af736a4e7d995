"""Oracle: the chunkwise mixer core, phases 1-3 (reference ``train_ablation.py:142-187``).

TEST INFRASTRUCTURE ONLY -- imported by tests/, smoke() and the bench's CPU
baseline, never by the shipped package.

Inputs are the hot path's per-head streams after the mixer front-end
(``train_ablation.py:124-134``):

* ``q, k`` (B, H, T, d): L2-normalised per head; ``v`` (B, H, T, d).
* ``beta`` (B, H, T): the beta gate (sigmoid output).
* ``g`` (B, H, T): log of the alpha gate.  The reference clamps alpha at 1e-6
  before the log (``train_ablation.py:170``); in log space that is
  ``max(g, log 1e-6)``, identical for alpha in (0, 1].
* ``gmu``, ``gnu`` (B, H, T) or None: log of the mu / nu gates, clamped the
  same way (``:172, :175``).

Three independent restatements are kept so they can pin each other:

* ``mixer_core``          -- the reference's matrix form (A, Kw, Uv, Qt, Ov,
                             then the state scan, then ``o = Qt S^T + Ov``).
* ``mixer_core_eform``    -- per chunk ``E = V - K S^T``, ``o = Q S^T + A E``,
                             ``G = E^T diag(w) K`` (substituting :164-167 into
                             :186 and fast_scan.py:82).
* ``mixer_core_tokens``   -- token by token:
                             ``o_t = S q_t + sum_{s<=t} beta_s (q_t.k_s)(v_s - S k_s)``.
"""
from __future__ import annotations

import math

import torch

from . import scan as _scan

LOG_GATE_FLOOR = math.log(1e-6)


def _clamp_log(x):
    return torch.clamp(x, min=LOG_GATE_FLOOR)


def gate_reductions(beta, g, gmu, gnu, rule: int, C: int):
    """Per-chunk scalars and per-token weights (train_ablation.py:150-158, 169-175, 180).

    Returns ``(a, b, m, n, w)`` with a, b, m, n of shape (B, H, N) and w of
    shape (B, H, N, C):

    * ``a = exp(sum_t max(g_t, log 1e-6))``, ``b = mean_t beta_t``
    * ``m = exp(sum_t max(gmu_t, log 1e-6))`` (ones when gmu is None)
    * ``n = exp(sum_t max(gnu_t, log 1e-6))`` for adam, else ones
    * ``w``: delta -> beta; muon -> ``exp(sum_{s>t} max(gmu_s, log 1e-6))``;
      adam -> ones.
    """
    B, H, T = beta.shape
    N = T // C
    bn = beta.reshape(B, H, N, C)
    a = torch.exp(_clamp_log(g.reshape(B, H, N, C)).sum(-1))
    b = bn.mean(-1)
    if gmu is not None:
        lmu = _clamp_log(gmu.reshape(B, H, N, C))
        m = torch.exp(lmu.sum(-1))
    else:
        lmu = None
        m = torch.ones_like(a)
    if rule == 2:
        if gnu is None:
            raise ValueError("adam rule needs gnu")
        n = torch.exp(_clamp_log(gnu.reshape(B, H, N, C)).sum(-1))
    else:
        n = torch.ones_like(a)
    if rule == 0:
        w = bn
    elif rule == 1:
        if lmu is None:
            raise ValueError("muon rule needs gmu")
        # suffix sum excluding the token itself (train_ablation.py:154-156)
        suffix = torch.flip(torch.cumsum(torch.flip(lmu, [-1]), -1), [-1]) - lmu
        w = torch.exp(suffix)
    else:
        w = torch.ones_like(bn)
    return a, b, m, n, w


def _maybe_round(x, cast):
    return x if cast is None else x.to(cast).to(x.dtype)


def mixer_core(q, k, v, beta, g, gmu=None, gnu=None, *, rule: int, ns: int = 5,
               C: int = 64, cast=None, return_states: bool = False):
    """Matrix-form phases 1-3 (train_ablation.py:142-187); returns ``o`` (B, H, T, d).

    ``cast`` (e.g. torch.bfloat16) rounds every phase-1/3 matmul output and the
    state read-out to that dtype, the points where CUDA autocast rounds in the
    reference (``:162-167``, ``:185``); None keeps full precision.
    """
    B, H, T, d = q.shape
    assert T % C == 0, "T must be a multiple of the chunk size"
    N = T // C
    qn = q.reshape(B, H, N, C, d)
    kn = k.reshape(B, H, N, C, d)
    vn = v.reshape(B, H, N, C, d)
    a, b, m, n, w = gate_reductions(beta, g, gmu, gnu, rule, C)
    bn = beta.reshape(B, H, N, C)
    causal = torch.tril(torch.ones(C, C, dtype=torch.bool))
    A = torch.matmul(qn, kn.transpose(-1, -2)) * bn.unsqueeze(-2)
    A = _maybe_round(torch.where(causal, A, torch.zeros_like(A)), cast)
    kw = kn * w.unsqueeze(-1)
    Kw = _maybe_round(torch.matmul(kw.transpose(-1, -2), kn), cast)
    Uv = _maybe_round(torch.matmul((vn * w.unsqueeze(-1)).transpose(-1, -2), kn), cast)
    Qt = _maybe_round(qn - torch.matmul(A, kn), cast)
    Ov = _maybe_round(torch.matmul(A, vn), cast)
    states = _scan.scan_forward(Uv, Kw, a, b, m, n, rule, ns)
    Sst = _maybe_round(states, cast)
    o = _maybe_round(torch.matmul(Qt, Sst.transpose(-1, -2)) + Ov, cast)
    o = o.reshape(B, H, T, d)
    if return_states:
        return o, states
    return o


def _rule_step(S, M, V, G, a, b, m, n, rule, ns):
    """One chunk-boundary update given the chunk gradient G (fast_scan.py:82-94)."""
    if rule == 0:
        return a * S + G, M, V
    if rule == 1:
        M = m * M + G
        return a * S + b * _scan.msign_sq(M, ns), M, V
    M = m * M + (1.0 - m) * G
    V = n * V + (1.0 - n) * G * G
    return a * S + b * M / (torch.sqrt(V) + _scan.EPS_ADAM), M, V


def mixer_core_eform(q, k, v, beta, g, gmu=None, gnu=None, *, rule: int, ns: int = 5,
                     C: int = 64, return_states: bool = False):
    """E-form restatement, one chunk at a time (the formulation the kernels use)."""
    B, H, T, d = q.shape
    N = T // C
    a, b, m, n, w = gate_reductions(beta, g, gmu, gnu, rule, C)
    bn = beta.reshape(B, H, N, C)
    S = q.new_zeros(B, H, d, d)
    M = q.new_zeros(B, H, d, d)
    V = q.new_zeros(B, H, d, d)
    causal = torch.tril(torch.ones(C, C, dtype=torch.bool))
    outs, states = [], []
    for i in range(N):
        sl = slice(i * C, (i + 1) * C)
        Q, Kc, Vc = q[:, :, sl], k[:, :, sl], v[:, :, sl]
        states.append(S)
        A = torch.matmul(Q, Kc.transpose(-1, -2)) * bn[:, :, i].unsqueeze(-2)
        A = torch.where(causal, A, torch.zeros_like(A))
        E = Vc - torch.matmul(Kc, S.transpose(-1, -2))
        outs.append(torch.matmul(Q, S.transpose(-1, -2)) + torch.matmul(A, E))
        G = torch.matmul((E * w[:, :, i].unsqueeze(-1)).transpose(-1, -2), Kc)
        sc = [t[:, :, i, None, None] for t in (a, b, m, n)]
        S, M, V = _rule_step(S, M, V, G, *sc, rule, ns)
    o = torch.cat(outs, dim=2)
    if return_states:
        return o, torch.stack(states, dim=2)
    return o


def mixer_core_tokens(q, k, v, beta, g, gmu=None, gnu=None, *, rule: int, ns: int = 5,
                      C: int = 64):
    """Token-by-token restatement (small shapes only)."""
    B, H, T, d = q.shape
    N = T // C
    a, b, m, n, w = gate_reductions(beta, g, gmu, gnu, rule, C)
    o = torch.zeros_like(q)
    for bb in range(B):
        for hh in range(H):
            S = q.new_zeros(d, d)
            M = q.new_zeros(d, d)
            V = q.new_zeros(d, d)
            for i in range(N):
                G = q.new_zeros(d, d)
                errs = []
                for s in range(C):
                    ts = i * C + s
                    e = v[bb, hh, ts] - S @ k[bb, hh, ts]
                    errs.append(e)
                    G = G + w[bb, hh, i, s] * torch.outer(e, k[bb, hh, ts])
                for t in range(C):
                    tt = i * C + t
                    acc = S @ q[bb, hh, tt]
                    for s in range(t + 1):
                        ts = i * C + s
                        acc = acc + beta[bb, hh, ts] * torch.dot(q[bb, hh, tt], k[bb, hh, ts]) * errs[s]
                    o[bb, hh, tt] = acc
                S, M, V = _rule_step(S, M, V, G, a[bb, hh, i], b[bb, hh, i], m[bb, hh, i],
                                     n[bb, hh, i], rule, ns)
    return o


def deltanet_textbook(q, k, v, beta):
    """Sequential DeltaNet: ``S_t = S_{t-1} + beta_t (v_t - S_{t-1} k_t) k_t^T``,
    ``o_t = S_t q_t`` -- what the mixer core reduces to at C=1, alpha=1, delta."""
    B, H, T, d = q.shape
    o = torch.zeros_like(q)
    for bb in range(B):
        for hh in range(H):
            S = q.new_zeros(d, d)
            for t in range(T):
                kt = k[bb, hh, t]
                S = S + beta[bb, hh, t] * torch.outer(v[bb, hh, t] - S @ kt, kt)
                o[bb, hh, t] = S @ q[bb, hh, t]
    return o
