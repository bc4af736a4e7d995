"""The WY mode's chunk algebra (gmdn_amd/wy.py: the quantities the HIP prep
kernel forms) on the CPU: with the state carried by the oracle's delta scan
(fast_scan.py:82 restated), o = Qt S_i^T + Ov reproduces the oracle's
token-exact gated delta recurrence."""
import torch

from gmdn_amd import wy as gwy
from oracle import scan as osc
from oracle import wy as owy


def test_wy_chunk_terms_reproduce_token_recurrence():
    gen = torch.Generator().manual_seed(0)
    B, H, T, d = 1, 2, 192, 16
    q, k, v, beta, g = owy.make_wy_inputs(B, H, T, d, generator=gen)
    g[0, 1, 70] = -50.0
    a, UA, KA, Qt, Ov = gwy.wy_chunk_terms(q.double(), k.double(), v.double(), beta, g)
    # float32 inside wy_chunk_terms: compare in float64 against the oracle
    ones = torch.ones_like(a).double()
    S_all = osc.scan_forward(UA.double(), KA.double(), a.double(), ones, ones, ones, 0, 0)
    o = (Qt.double() @ S_all.transpose(-1, -2) + Ov.double()).reshape(B, H, T, d)
    ref = owy.token_scan(q, k, v, beta, g)
    err = (o - ref).abs().max() / ref.pow(2).mean().sqrt()
    assert err < 1e-5, float(err)


def test_wy_chunk_terms_strong_decay_finite_gradients():
    """Strongly decaying gates (log alpha at its floor log 1e-6, and a uniform
    -2): the decay ratios gamma_t / gamma_s span exp(+-880) within a chunk.
    The chunk algebra forms them from masked exponents, so its output and its
    autograd gradients stay finite and the output still reproduces the token
    recurrence."""
    for gval in (-2.0, -20.0):
        gen = torch.Generator().manual_seed(1)
        B, H, T, d = 1, 1, 128, 16
        q, k, v, beta, g = owy.make_wy_inputs(B, H, T, d, generator=gen)
        g = torch.full_like(g, gval)
        xs = [t.clone().requires_grad_(True) for t in (q, k, v, beta, g)]
        a, UA, KA, Qt, Ov = gwy.wy_chunk_terms(*xs)
        loss = sum(t.double().sum() for t in (a, UA, KA, Qt, Ov))
        grads = torch.autograd.grad(loss, xs)
        for name, gr in zip(("q", "k", "v", "beta", "g"), grads):
            assert torch.isfinite(gr).all(), (gval, name)
        ones = torch.ones_like(a).double()
        S_all = osc.scan_forward(UA.double(), KA.double(), a.double(), ones, ones, ones, 0, 0)
        o = (Qt.double() @ S_all.transpose(-1, -2) + Ov.double()).reshape(B, H, T, d)
        ref = owy.token_scan(q, k, v, beta, g)
        err = (o.detach() - ref).abs().max() / ref.pow(2).mean().sqrt()
        assert err < 1e-5, (gval, float(err))
