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


@pytest.mark.parametrize("rule,ns", [(0, 3), (1, 0), (1, 1), (1, 5), (2, 3)])
def test_manual_backward_matches_autograd_of_scan_eager(rule, ns):
    """The hand-derived reverse scan against torch.autograd through the
    module's own eager forward (two derivations of the same VJP)."""
    gen = torch.Generator().manual_seed(7)
    ins = [t.double().requires_grad_(True) for t in osc.make_scan_inputs(1, 2, 4, 16, 8, generator=gen)]
    S = fast_scan.scan_eager(*ins, rule, ns)
    gS = torch.randn(S.shape, generator=gen, dtype=torch.float64)
    auto = torch.autograd.grad(S, ins, gS, allow_unused=True)
    auto = [torch.zeros_like(t) if g is None else g for g, t in zip(auto, ins)]
    _, M_all, V_all = osc.scan_forward(*[t.detach() for t in ins], rule, ns, return_moments=True)
    mine = fast_scan.manual_backward(*[t.detach() for t in ins], S.detach(), M_all, V_all, gS, rule, ns)
    for name, a, b in zip("U K a b m n".split(), mine, auto):
        assert torch.allclose(a, b, atol=1e-10, rtol=1e-9), name


def test_eager_msign_matches_svd_closed_form():
    """_msign_sq against the SVD form P p^{ns}(sigma / (|M|_F + eps)) R^T."""
    gen = torch.Generator().manual_seed(3)
    M = torch.randn(3, 8, 8, generator=gen, dtype=torch.float64)
    for ns in (0, 1, 3, 5):
        X = fast_scan._msign_sq(M, ns)
        for j in range(3):
            ref = torch.from_numpy(osc.msign_svd(M[j].numpy(), ns))
            assert torch.allclose(X[j], ref, atol=1e-10)


def test_empty_sequence():
    ins = osc.make_scan_inputs(1, 2, 0, 16, 8)
    for rule in (0, 1, 2):
        assert fast_scan.scan_eager(*ins, rule, 3).shape == (1, 2, 0, 8, 8)
        grads = fast_scan.manual_backward(*ins, *(torch.zeros(1, 2, 0, 8, 8),) * 4, rule, 3)
        assert [tuple(g.shape) for g in grads] == [tuple(t.shape) for t in ins]
