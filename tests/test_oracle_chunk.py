"""Pins of the mixer-core oracle (oracle/chunk.py).

Three restatements check each other (reference matrix form, E-form, token
loop); C = 1 with alpha = 1 must reduce to textbook DeltaNet; the gate
reductions have closed forms for constant gates; gradients pass gradcheck.
"""
import math

import pytest
import torch

from oracle import chunk as oc

D64 = torch.float64


def _inputs(B, H, T, d, seed, rule):
    gen = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, H, T, d, generator=gen, dtype=D64), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, H, T, d, generator=gen, dtype=D64), dim=-1)
    v = torch.randn(B, H, T, d, generator=gen, dtype=D64)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=gen, dtype=D64))
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen, dtype=D64) + 3)
    gmu = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen, dtype=D64) + 1) if rule else None
    gnu = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen, dtype=D64) + 2) if rule == 2 else None
    return q, k, v, beta, g, gmu, gnu


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_matrix_eform_token_forms_agree(rule):
    q, k, v, beta, g, gmu, gnu = _inputs(1, 2, 24, 6, 0, rule)
    o_m = oc.mixer_core(q, k, v, beta, g, gmu, gnu, rule=rule, ns=3, C=8)
    o_e = oc.mixer_core_eform(q, k, v, beta, g, gmu, gnu, rule=rule, ns=3, C=8)
    o_t = oc.mixer_core_tokens(q, k, v, beta, g, gmu, gnu, rule=rule, ns=3, C=8)
    assert torch.allclose(o_m, o_e, atol=1e-11)
    assert torch.allclose(o_m, o_t, atol=1e-11)


def test_states_match_between_forms():
    q, k, v, beta, g, gmu, gnu = _inputs(2, 1, 32, 5, 1, 1)
    _, s_m = oc.mixer_core(q, k, v, beta, g, gmu, gnu, rule=1, ns=2, C=8, return_states=True)
    _, s_e = oc.mixer_core_eform(q, k, v, beta, g, gmu, gnu, rule=1, ns=2, C=8, return_states=True)
    assert torch.allclose(s_m, s_e, atol=1e-11)


def test_chunk_one_no_decay_is_textbook_deltanet():
    q, k, v, beta, _, _, _ = _inputs(1, 2, 12, 4, 2, 0)
    g = torch.zeros_like(beta)                      # alpha = 1
    o = oc.mixer_core(q, k, v, beta, g, rule=0, C=1)
    assert torch.allclose(o, oc.deltanet_textbook(q, k, v, beta), atol=1e-12)


def test_single_chunk_is_parallel_form():
    """With one chunk covering all tokens the state is S_0 = 0 throughout,
    so o = tril(Q K^T) diag(beta) V."""
    q, k, v, beta, g, _, _ = _inputs(1, 1, 16, 4, 3, 0)
    o = oc.mixer_core(q, k, v, beta, g, rule=0, C=16)
    A = torch.tril(q[0, 0] @ k[0, 0].T) * beta[0, 0][None, :]
    assert torch.allclose(o[0, 0], A @ v[0, 0], atol=1e-12)


def test_gate_reductions_closed_forms():
    B, H, C, N = 1, 2, 8, 3
    T = C * N
    la, lmu, lnu = math.log(0.9), math.log(0.8), math.log(0.99)
    beta = torch.linspace(0.1, 0.9, T, dtype=D64).expand(B, H, T)
    full = lambda v: torch.full((B, H, T), v, dtype=D64)
    a, b, m, n, w = oc.gate_reductions(beta, full(la), full(lmu), full(lnu), 2, C)
    assert torch.allclose(a, torch.full_like(a, 0.9 ** C))
    assert torch.allclose(m, torch.full_like(m, 0.8 ** C))
    assert torch.allclose(n, torch.full_like(n, 0.99 ** C))
    assert torch.allclose(b, beta.reshape(B, H, N, C).mean(-1))
    assert torch.allclose(w, torch.ones_like(w))
    _, _, _, n1, w1 = oc.gate_reductions(beta, full(la), full(lmu), None, 1, C)
    assert torch.allclose(n1, torch.ones_like(n1))
    exp_w = torch.tensor([0.8 ** (C - 1 - s) for s in range(C)], dtype=D64)
    assert torch.allclose(w1, exp_w.expand_as(w1))
    _, _, _, _, w0 = oc.gate_reductions(beta, full(la), None, None, 0, C)
    assert torch.allclose(w0, beta.reshape(B, H, N, C))


def test_gate_log_floor():
    """The reference clamps gates at 1e-6 before the log: g below log(1e-6)
    contributes log(1e-6) and no gradient."""
    beta = torch.full((1, 1, 4), 0.5, dtype=D64)
    g = torch.tensor([[[-30.0, -1.0, -2.0, -0.5]]], dtype=D64, requires_grad=True)
    a, *_ = oc.gate_reductions(beta, g, None, None, 0, 4)
    assert torch.allclose(a, torch.exp(torch.tensor(math.log(1e-6) - 3.5, dtype=D64)))
    a.sum().backward()
    assert g.grad[0, 0, 0] == 0 and g.grad[0, 0, 1] != 0


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_mixer_core_gradcheck(rule):
    q, k, v, beta, g, gmu, gnu = _inputs(1, 1, 8, 3, 4 + rule, rule)
    ins = [t.clone().requires_grad_(True) for t in (q, k, v, beta, g) + ((gmu,) if rule else ()) + ((gnu,) if rule == 2 else ())]

    def f(*x):
        gm = x[5] if rule else None
        gn = x[6] if rule == 2 else None
        return oc.mixer_core(x[0], x[1], x[2], x[3], x[4], gm, gn, rule=rule, ns=2, C=4)

    assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-5)


def test_eform_identity_per_chunk():
    """(Q - A K) S^T + A V == Q S^T + A (V - K S^T) for any S."""
    gen = torch.Generator().manual_seed(9)
    Q, K, V = (torch.randn(8, 5, generator=gen, dtype=D64) for _ in range(3))
    S = torch.randn(5, 5, generator=gen, dtype=D64)
    A = torch.tril(torch.randn(8, 8, generator=gen, dtype=D64))
    lhs = (Q - A @ K) @ S.T + A @ V
    rhs = Q @ S.T + A @ (V - K @ S.T)
    assert torch.allclose(lhs, rhs, atol=1e-12)


def test_planted_missing_beta_scale_is_caught(monkeypatch):
    """An oracle that forgets the beta column scale of A fails the one-chunk check."""
    orig = oc.mixer_core

    def bad(q, k, v, beta, g, gmu=None, gnu=None, **kw):
        return orig(q, k, v, torch.ones_like(beta), g, gmu, gnu, **kw)

    monkeypatch.setattr(oc, "mixer_core", bad)
    with pytest.raises(AssertionError):
        test_single_chunk_is_parallel_form()
