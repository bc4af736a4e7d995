"""The drop-in module keeps the reference fast_scan API (fast_scan.py:29-56,
:334-414) and its dispatch semantics on the host side."""
import inspect

import pytest
import torch

import fast_scan
from oracle import scan as osc


def test_public_names():
    for name in ("fast_state_scan", "scan_eager", "manual_backward", "set_backend", "set_precision",
                 "HAS_TRITON", "_TritonScan", "NS_A", "NS_B", "NS_C", "_EPS_NORM", "_EPS_ADAM",
                 "_msign_sq", "_msign_vjp", "_ns_step"):
        assert hasattr(fast_scan, name), name
    assert (fast_scan.NS_A, fast_scan.NS_B, fast_scan.NS_C) == (3.4445, -4.7750, 2.0315)
    assert fast_scan._EPS_NORM == 1e-7 and fast_scan._EPS_ADAM == 1e-6
    params = list(inspect.signature(fast_scan.fast_state_scan).parameters)
    assert params == ["U", "K", "a", "b", "m", "n", "rule", "ns"]


def test_knob_names_are_validated():
    with pytest.raises(AssertionError):
        fast_scan.set_backend("cuda")
    with pytest.raises(AssertionError):
        fast_scan.set_precision("fp16")
    for name in ("auto", "triton", "eager", "hip"):
        fast_scan.set_backend(name)
    fast_scan.set_backend("auto")
    for name in ("ieee", "tf32"):
        fast_scan.set_precision(name)


def test_cpu_tensors_take_eager_path_and_match_oracle():
    gen = torch.Generator().manual_seed(0)
    ins = osc.make_scan_inputs(2, 2, 5, 16, 8, generator=gen, dtype=torch.float64)
    for rule in (0, 1, 2):
        S = fast_scan.fast_state_scan(*ins, rule, 3)
        assert torch.allclose(S, osc.scan_forward(*ins, rule, 3), atol=1e-12)


def test_forced_native_backend_rejects_cpu_tensors():
    ins = osc.make_scan_inputs(1, 1, 2, 8, 32)
    fast_scan.set_backend("triton")
    try:
        with pytest.raises(RuntimeError):
            fast_scan.fast_state_scan(*ins, 0, 3)
    finally:
        fast_scan.set_backend("auto")


def test_hip_op_rejects_cpu_tensors():
    ins = osc.make_scan_inputs(1, 1, 2, 8, 32)
    with pytest.raises(RuntimeError):
        fast_scan._TritonScan.apply(*ins, 0, 3)


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_manual_backward_matches_oracle(rule):
    gen = torch.Generator().manual_seed(1)
    ins = [t.double() for t in osc.make_scan_inputs(1, 2, 4, 16, 8, generator=gen)]
    S_all, M_all, V_all = osc.scan_forward(*ins, rule, 3, return_moments=True)
    gS = torch.randn(S_all.shape, generator=gen, dtype=torch.float64)
    mine = fast_scan.manual_backward(*ins, S_all, M_all, V_all, gS, rule, 3)
    ref = osc.scan_backward(*ins, S_all, M_all, V_all, gS, rule, 3)
    for a, b in zip(mine, ref):
        assert torch.allclose(a, b, atol=1e-12)
