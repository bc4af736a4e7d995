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
