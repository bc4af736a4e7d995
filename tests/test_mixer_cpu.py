"""CPU checks of the mixer layer's pieces that are plain torch."""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "gmdn-gated-muon-deltanet_amd"))

from gmdn_amd.mixer import LM, FastWeightMixer, causal_depthwise_conv  # noqa: E402


@pytest.mark.parametrize("K", [1, 3, 4])
def test_causal_depthwise_conv_matches_conv1d(K):
    """train_ablation.py:93-94, :124: a depthwise Conv1d with K-1 padding, the
    first T outputs -- values and gradients, in float64."""
    torch.manual_seed(K)
    C, T = 12, 37
    conv = torch.nn.Conv1d(C, C, K, groups=C, padding=K - 1).double()
    y = torch.randn(2, T, C, dtype=torch.float64, requires_grad=True)
    ref = conv(y.transpose(1, 2))[..., :T].transpose(1, 2)
    got = causal_depthwise_conv(y, conv.weight, conv.bias)
    torch.testing.assert_close(got, ref, rtol=0, atol=1e-12)
    g = torch.randn_like(ref)
    want = torch.autograd.grad(ref, (y, conv.weight, conv.bias), g)
    have = torch.autograd.grad(got, (y, conv.weight, conv.bias), g)
    for a, b in zip(have, want):
        torch.testing.assert_close(a, b, rtol=0, atol=1e-12)


def test_parameters_match_the_reference_layout():
    """The reference's parameter names and shapes (train_ablation.py:92-98,
    199-220), so its state_dict loads unchanged."""
    m = FastWeightMixer(256, 2, "adam")
    assert {n: tuple(p.shape) for n, p in m.named_parameters()} == {
        "qkv.weight": (768, 256), "conv.weight": (768, 1, 4), "conv.bias": (768,),
        "gates.weight": (8, 256), "gates.bias": (8,), "norm.weight": (128,), "out.weight": (256, 256)}
    assert torch.equal(m.gates.bias, torch.tensor([3.0, 3.0, -1.0, -1.0, 1.0, 1.0, 2.0, 2.0]))
    lm = LM(100, 64, 2, 2, "muon")
    assert lm.lm_head.weight is lm.emb.weight
    assert len(lm.blocks) == 2 and lm.blocks[0].mlp[0].weight.shape == (256, 64)
