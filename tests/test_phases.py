"""The closed-form VJP of phases 1 and 3 (gmdn_amd/phases.py, used by the
fused muon core's backward) against torch.autograd through the same
forward, and the forward against the oracle's matrix form."""
import math

import torch

from gmdn_amd import phases
from gmdn_amd.workloads import Workload, make_inputs
from oracle import chunk as oc

D64 = torch.float64


def _inputs(seed, T=128, d=16, floor_hits=True):
    gen = torch.Generator().manual_seed(seed)
    B, H = 1, 2
    q = torch.nn.functional.normalize(torch.randn(B, H, T, d, generator=gen, dtype=D64), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, H, T, d, generator=gen, dtype=D64), dim=-1)
    v = torch.randn(B, H, T, d, generator=gen, dtype=D64)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=gen, dtype=D64))
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen, dtype=D64) + 3)
    gmu = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen, dtype=D64) + 1)
    if floor_hits:  # some gates below the 1e-6 floor: their gradient is zero
        g[..., 5] = -20.0
        gmu[..., 17] = -30.0
    return q, k, v, beta, g, gmu


def test_phase1_vjp_matches_autograd():
    xs = [t.requires_grad_(True) for t in _inputs(0)]
    ph = phases.phase1(*xs)
    gen = torch.Generator().manual_seed(1)
    names = ("Kw", "Uv", "Qt", "Ov", "a", "b", "m")
    cots = {n: torch.randn(ph[n].shape, generator=gen, dtype=D64) for n in names}
    total = sum((ph[n] * cots[n]).sum() for n in names)
    want = torch.autograd.grad(total, xs)
    got = phases.phase1_vjp({k_: (t.detach() if torch.is_tensor(t) else t) for k_, t in ph.items()},
                            xs[4].detach(), xs[5].detach(), cots["Kw"], cots["Uv"], cots["Qt"], cots["Ov"],
                            cots["a"], cots["b"], cots["m"])
    for name, a, b in zip(("q", "k", "v", "beta", "g", "gmu"), got, want):
        assert torch.allclose(a, b, atol=1e-10, rtol=1e-9), name
    # the floored gates get no gradient
    assert got[4][..., 5].abs().max() == 0 and got[5][..., 17].abs().max() == 0


def test_phase3_vjp_matches_autograd():
    q, k, v, beta, g, gmu = _inputs(2)
    ph = phases.phase1(q, k, v, beta, g, gmu)
    B, H, N, C, d = ph["Q"].shape
    gen = torch.Generator().manual_seed(3)
    S = torch.randn(B, H, N, d, d, generator=gen, dtype=D64, requires_grad=True)
    Qt = ph["Qt"].detach().requires_grad_(True)
    Ov = ph["Ov"].detach().requires_grad_(True)
    o = torch.matmul(Qt, S.transpose(-1, -2)) + Ov
    dO = torch.randn(B, H, N * C, d, generator=gen, dtype=D64)
    want = torch.autograd.grad(o, (Qt, Ov, S), dO.reshape(o.shape))
    got = phases.phase3_vjp({"Q": ph["Q"], "Qt": Qt.detach()}, S.detach(), dO)
    for a, b in zip(got, want):
        assert torch.allclose(a, b, atol=1e-12)


def test_phase1_matches_oracle_gate_reductions():
    """The per-chunk scalars and token weights agree with the oracle's
    restatement of train_ablation.py:150-158."""
    q, k, v, beta, g, gmu = _inputs(4)
    ph = phases.phase1(q, k, v, beta, g, gmu)
    a, b, m, n, w = oc.gate_reductions(beta, g, gmu, None, 1, 64)
    for x, y in ((ph["a"], a), (ph["b"], b), (ph["m"], m), (ph["w"], w)):
        assert torch.allclose(x, y, atol=1e-12, rtol=1e-12)
