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


def test_build_optimizers_splits_parameters_like_the_reference():
    """train_ablation.py:291-307: every 2-D weight except the (tied) embedding
    goes to Muon, everything else to AdamW(betas 0.9, 0.95)."""
    import types

    from gmdn_amd.mixer import LM
    from gmdn_amd.muon import Muon, build_optimizers

    model = LM(vocab=64, d_model=32, n_layers=2, n_heads=2, inner="muon")
    args = types.SimpleNamespace(muon_lr=0.02, adam_lr=4e-4, weight_decay=0.1)
    muon, adamw = build_optimizers(model, "muon", args)
    assert isinstance(muon, Muon) and isinstance(adamw, torch.optim.AdamW)
    m_ids = {id(p) for g in muon.param_groups for p in g["params"]}
    a_ids = {id(p) for g in adamw.param_groups for p in g["params"]}
    params = list(model.parameters())
    assert m_ids | a_ids == {id(p) for p in params} and not (m_ids & a_ids)
    assert id(model.emb.weight) in a_ids and model.lm_head.weight is model.emb.weight
    for p in params:
        assert (id(p) in m_ids) == (p.ndim == 2 and p is not model.emb.weight)
    assert muon.param_groups[0]["lr"] == 0.02 and muon.param_groups[0]["weight_decay"] == 0.1
    assert adamw.param_groups[0]["betas"] == (0.9, 0.95) and adamw.param_groups[0]["lr"] == 4e-4
    plain = build_optimizers(model, "adamw", args)
    assert all(isinstance(o, torch.optim.AdamW) for o in plain)


def test_mixer_accepts_the_reference_chunk_knob():
    """--chunk (train_ablation.py:555) other than 64 builds the same layer
    (it runs the reference's schedule around the drop-in scan); T must be a
    multiple of it."""
    m = FastWeightMixer(128, 4, "muon", chunk=32)
    assert m.chunk == 32 and m.dh == 32
    import pytest
    with pytest.raises(ValueError):
        m(torch.zeros(1, 48, 128))
