"""CPU checks of the mixer layer's parameter layout and initialisation."""
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "gmdn-gated-muon-deltanet_amd"))

from gmdn_amd.mixer import LM, FastWeightMixer  # noqa: E402


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
