"""The mixer layer and LM stack around the fused core (gmdn_amd/mixer.py).

The reference layer (train_ablation.py:113-190) ends in a per-head RMSNorm
whose rows can be near zero: rounding q, k, v and o to bf16 alone, as the
reference's autocast does, moves its output by 0.10 (delta), 0.04 (muon) and
0.30 (adam) of its RMS at B=1, T=256.  So the layer is checked in its three
parts against the reference restated on the CPU in float32, with the same
weights:
* the front-end (projection, conv, SiLU, L2 norm, gates) to float32 rounding;
* the fused core on those very inputs against the oracle's matrix-form
  phases 1-3 in float64, to the bf16 bound: the error in excess of half a
  bf16 ulp of the reference (the output's own rounding), at most 2e-2 of its
  RMS;
* the tail (RMSNorm, output projection) applied to the core's output at the
  layer's own precision.
A float32 layer (autocast off) is also checked whole, against the reference
layer restated in float64.
The backward is checked for reaching every parameter with finite values."""
import copy
import math

import pytest
import torch
import torch.nn.functional as F

from gmdn_amd.chunk import chunk_scan
from gmdn_amd.mixer import LM, FastWeightMixer
from oracle import chunk as oc

pytestmark = pytest.mark.gpu
CASES = [("delta", 256, 2), ("muon", 256, 2), ("adam", 128, 2), ("muon", 1024, 8)]


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _reference_front_end(m: FastWeightMixer, x: torch.Tensor):
    """train_ablation.py:124-134 and the phase-1 gate logs (:155, :170-175)."""
    B, T, D = x.shape
    H, dh = m.h, m.dh
    qkv = m.conv(m.qkv(x).transpose(1, 2))[..., :T].transpose(1, 2)
    qkv = F.silu(qkv)
    q, k, v = qkv.chunk(3, dim=-1)
    q = F.normalize(q.view(B, T, H, dh).transpose(1, 2), dim=-1)
    k = F.normalize(k.view(B, T, H, dh).transpose(1, 2), dim=-1)
    v = v.reshape(B, T, H, dh).transpose(1, 2)
    g = torch.sigmoid(m.gates(x)).view(B, T, m.n_gates, H).permute(2, 0, 3, 1)
    logs = [torch.log(t.clamp_min(1e-6)) for t in g]
    return q, k, v, g[1], logs[0], logs[2], logs[3] if m.n_gates == 4 else None


def _layer(inner, d_model, dev, heads=2):
    torch.manual_seed(0)
    ref = FastWeightMixer(d_model, heads, inner, ns_steps=3)
    with torch.no_grad():  # weights off the zero-bias init
        for p in ref.parameters():
            p.add_(0.02 * torch.randn_like(p))
    return ref, copy.deepcopy(ref).to(dev)


@pytest.mark.parametrize("inner,d_model,heads", CASES)
def test_mixer_parts_match_reference(inner, d_model, heads):
    """Layer parts at d_model 256 / 128 with two heads, and at the LM's
    layer shape (d_model 1024, 8 heads x 128, muon, ns = 3) on one batch row."""
    dev = _dev()
    ref, mine = _layer(inner, d_model, dev, heads)
    x = torch.randn(1, 256, d_model)
    with torch.no_grad():
        want = _reference_front_end(ref, x)
        got = mine.front_end(x.to(dev))
        names = ("q", "k", "v", "beta", "log_alpha", "log_mu", "log_nu")
        for name, a, b in zip(names, got, want):
            if b is None:
                assert a is None, name
                continue
            torch.testing.assert_close(a.cpu(), b, rtol=1e-4, atol=1e-5, msg=name)
        # the core on the layer's own inputs (q, k, v in bf16 as the layer passes them)
        q, k, v = (t.to(torch.bfloat16) for t in got[:3])
        o = chunk_scan(q, k, v, *got[3:], rule=inner, ns=mine.ns_steps)
        rule = {"delta": 0, "muon": 1, "adam": 2}[inner]
        f64 = lambda t: None if t is None else t.cpu().double()
        o_ref = oc.mixer_core(*(f64(t) for t in (q, k, v)), *(f64(t) for t in got[3:]), rule=rule,
                              ns=mine.ns_steps, C=64)
        # error in excess of the bf16 rounding of the output itself
        half_ulp = torch.pow(2.0, torch.floor(torch.log2(o_ref.abs().clamp_min(1e-30))) - 8)
        excess = ((o.double().cpu() - o_ref).abs() - half_ulp).clamp_min(0).max() / o_ref.pow(2).mean().sqrt()
        assert excess <= 2e-2, float(excess)
        # the tail on the core's output at the layer's own precision (the
        # float32 module passes float32 streams to the core)
        B, T, D = x.shape
        y = mine(x.to(dev))
        o_layer = chunk_scan(*got[:3], *got[3:], rule=inner, ns=mine.ns_steps)
        y_tail = mine.out(mine.norm(o_layer.float()).transpose(1, 2).reshape(B, T, D))
        torch.testing.assert_close(y, y_tail, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("inner", ["delta", "muon", "adam"])
def test_mixer_fp32_layer_matches_reference(inner):
    """Without autocast the layer runs in float32 end to end, as the
    reference's does (train_ablation.py:424, 465): front-end, the fused core
    on float32 streams (the matrix form in exact float32) and the tail.  The
    whole layer is checked against the reference layer restated in float64
    with the same weights, rel = max|y - y_ref| / max|y_ref| <= 1e-4."""
    dev = _dev()
    ref, mine = _layer(inner, 128, dev, 2)  # 2 heads x 64
    x = torch.randn(1, 256, 128)
    with torch.no_grad():
        y = mine(x.to(dev))
        assert y.dtype == torch.float32
        r = copy.deepcopy(ref).double()
        r.norm.eps = torch.finfo(torch.float32).eps  # the float32 layer's RMSNorm epsilon
        q, k, v, beta, la, lm, ln = _reference_front_end(r, x.double())
        rule = {"delta": 0, "muon": 1, "adam": 2}[inner]
        o = oc.mixer_core(q, k, v, beta, la, lm, ln, rule=rule, ns=r.ns_steps, C=64)
        B, T, D = x.shape
        y_ref = r.out(r.norm(o).transpose(1, 2).reshape(B, T, D))
    err = ((y.double().cpu() - y_ref).abs().max() / y_ref.abs().max()).item()
    print(f"float32 {inner} layer: rel {err:.2e}")
    assert err <= 1e-4


@pytest.mark.parametrize("inner,d_model,heads", CASES)
def test_mixer_backward_reaches_every_parameter(inner, d_model, heads):
    dev = _dev()
    _, mine = _layer(inner, d_model, dev, heads)
    x = torch.randn(1, 256, d_model, device=dev, requires_grad=True)
    mine(x).square().mean().backward()
    assert torch.isfinite(x.grad).all() and x.grad.abs().max() > 0
    for name, p in mine.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().max() > 0, name


def test_lm_step_bf16():
    """A 2-layer muon LM in bf16: next-token loss at init is ~log(vocab), the
    backward reaches every parameter with finite gradients."""
    dev = _dev()
    torch.manual_seed(0)
    vocab = 1000
    model = LM(vocab, 256, 2, 2, "muon", ns_steps=3).to(dev, torch.bfloat16)
    idx = torch.randint(0, vocab, (2, 257), device=dev)
    _, loss = model(idx[:, :-1], idx[:, 1:])
    assert abs(loss.item() - math.log(vocab)) < 0.5
    loss.backward()
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name


def test_lm_full_size_step():
    """The 12-layer LM at its benchmark size: d_model 1024, 8 heads x 128,
    muon inner rule with ns = 3, vocab 32000, B = 8, T = 2048, bf16 weights
    from the reference's N(0, 0.02) init (train_ablation.py:212-246), token
    ids uniform over the vocabulary.  The next-token loss at init is within
    0.5 of ln 32000, and the backward reaches every parameter with finite,
    non-zero gradients."""
    dev = _dev()
    torch.manual_seed(0)
    vocab, B, T = 32000, 8, 2048
    model = LM(vocab, 1024, 12, 8, "muon", ns_steps=3).to(dev, torch.bfloat16)
    gen = torch.Generator(device=dev).manual_seed(0)
    idx = torch.randint(0, vocab, (B, T + 1), device=dev, generator=gen)
    _, loss = model(idx[:, :-1], idx[:, 1:])
    print(f"LM 12L d1024 B8 T2048: loss at init {loss.item():.4f} (ln 32000 = {math.log(vocab):.4f})")
    assert abs(loss.item() - math.log(vocab)) < 0.5
    loss.backward()
    for name, p in model.named_parameters():
        assert p.grad is not None, name
        assert torch.isfinite(p.grad).all(), name
        assert p.grad.abs().max() > 0, name
