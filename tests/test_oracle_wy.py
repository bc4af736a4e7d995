"""Pins of the WY oracle (oracle/wy.py): the token recurrence by closed forms
and brute force, and the chunked WY form against the token recurrence for
every chunk length (the WY transform is exact, so the chunk length must not
change the result)."""
import math

import pytest
import torch

from oracle import wy

D64 = torch.float64


def test_single_token_closed_form():
    """One token from S = 0: S_1 = beta v k^T, o = beta (k . q) v."""
    gen = torch.Generator().manual_seed(0)
    q, k, v, beta, g = wy.make_wy_inputs(1, 2, 1, 8, generator=gen)
    o = wy.token_scan(q, k, v, beta, g)
    want = beta[..., None] * (k * q).sum(-1, keepdim=True) * v
    assert torch.allclose(o, want, atol=1e-14)


def test_orthogonal_keys_accumulate():
    """Orthonormal keys: S_{t-1} k_t = prod(alpha) * 0 after the first write
    along k_t, so S_t = alpha_t S_{t-1} + beta_t v_t k_t^T and
    o_t = sum_{s<=t} (prod_{s<u<=t} alpha_u) beta_s (k_s . q_t) v_s."""
    gen = torch.Generator().manual_seed(1)
    d, T = 8, 6
    Qm, _ = torch.linalg.qr(torch.randn(d, d, generator=gen, dtype=D64))
    k = Qm[:T].reshape(1, 1, T, d)
    q = torch.randn(1, 1, T, d, generator=gen, dtype=D64)
    v = torch.randn(1, 1, T, d, generator=gen, dtype=D64)
    beta = torch.rand(1, 1, T, generator=gen, dtype=D64)
    g = torch.log(0.5 + 0.5 * torch.rand(1, 1, T, generator=gen, dtype=D64))
    o = wy.token_scan(q, k, v, beta, g)
    alpha = torch.exp(g[0, 0])
    for t in range(T):
        want = torch.zeros(d, dtype=D64)
        for s in range(t + 1):
            decay = torch.prod(alpha[s + 1:t + 1]) if s < t else torch.tensor(1.0, dtype=D64)
            want += decay * beta[0, 0, s] * (k[0, 0, s] @ q[0, 0, t]) * v[0, 0, s]
        assert torch.allclose(o[0, 0, t], want, atol=1e-12)


def test_brute_force_two_tokens():
    """Two tokens by hand: S_2 = a2 S_1 (I - b2 k2 k2^T) + b2 v2 k2^T."""
    gen = torch.Generator().manual_seed(2)
    q, k, v, beta, g = wy.make_wy_inputs(1, 1, 2, 5, generator=gen)
    a = torch.exp(g[0, 0])
    k1, k2, v1, v2 = k[0, 0, 0], k[0, 0, 1], v[0, 0, 0], v[0, 0, 1]
    b1, b2 = beta[0, 0]
    S1 = b1 * torch.outer(v1, k1)
    S2 = a[1] * S1 @ (torch.eye(5, dtype=D64) - b2 * torch.outer(k2, k2)) + b2 * torch.outer(v2, k2)
    o = wy.token_scan(q, k, v, beta, g)
    assert torch.allclose(o[0, 0, 1], S2 @ q[0, 0, 1], atol=1e-14)


@pytest.mark.parametrize("C", [1, 2, 8, 16, 64])
def test_chunked_wy_equals_token_recurrence(C):
    gen = torch.Generator().manual_seed(3)
    q, k, v, beta, g = wy.make_wy_inputs(2, 2, 128, 16, generator=gen)
    g[0, 0, 7] = -40.0  # a gate below the 1e-6 floor
    o_tok = wy.token_scan(q, k, v, beta, g)
    o_wy = wy.wy_chunked(q, k, v, beta, g, C)
    assert torch.allclose(o_wy, o_tok, atol=1e-11, rtol=1e-10)


def test_triangular_inverse():
    gen = torch.Generator().manual_seed(4)
    q, k, v, beta, g = wy.make_wy_inputs(1, 2, 64, 16, generator=gen)
    z = wy.wy_chunk_terms(q, k, v, beta, g, 64)
    eye = torch.eye(64, dtype=D64)
    assert torch.allclose((eye + z["A"]) @ z["T"], eye.expand_as(z["T"]), atol=1e-12)
    assert torch.equal(torch.triu(z["A"]), torch.zeros_like(z["A"]))


def test_pin_catches_dropped_decay(monkeypatch):
    """Plant a mistake in the oracle (the decay dropped from W): the chunked
    form must then disagree with the token recurrence."""
    gen = torch.Generator().manual_seed(5)
    q, k, v, beta, g = wy.make_wy_inputs(1, 1, 64, 8, generator=gen)
    real = wy.wy_chunk_terms

    def broken(*a, **kw):
        z = real(*a, **kw)
        z["W"] = z["T"] @ ((a[3].reshape(z["gamma"].shape))[..., None] * z["K"])
        return z

    monkeypatch.setattr(wy, "wy_chunk_terms", broken)
    assert not torch.allclose(wy.wy_chunked(q, k, v, beta, g, 16), wy.token_scan(q, k, v, beta, g), atol=1e-6)
