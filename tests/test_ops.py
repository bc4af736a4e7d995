"""CPU checks of the registered operators (torch.ops.gmdn.*): registration,
shape-only fake implementations, and whole-graph capture by torch.compile
(the reference trainer compiles its model, train_ablation.py:420-422) on
fake GPU tensors, so nothing runs on a device."""
import os
import sys

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "gmdn-gated-muon-deltanet_amd"))

import fast_scan  # noqa: E402
from gmdn_amd import _native, chunk, ops  # noqa: E402,F401

OPS = ("state_scan", "state_scan_bwd", "chunk_fwd", "chunk_bwd", "chunk_bwd_muon", "front_fwd", "front_bwd", "msign")


def _capture(fn, *args):
    """torch.compile(fullgraph=True) of fn on fake tensors; the captured graph's call targets."""
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    torch._dynamo.reset()
    out = torch.compile(fn, backend=backend, fullgraph=True)(*args)
    assert len(graphs) == 1
    return out, [str(n.target) for n in graphs[0].graph.nodes if n.op == "call_function"]


def test_ops_registered():
    for name in OPS:
        assert hasattr(torch.ops.gmdn, name), name


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_state_scan_compiles_to_one_graph(rule):
    with FakeTensorMode():
        U, K = (torch.empty(2, 3, 4, 64, 64, device="cuda") for _ in range(2))
        g = [torch.empty(2, 3, 4, device="cuda") for _ in range(4)]
        out, targets = _capture(lambda *x: fast_scan.fast_state_scan(*x, rule, 3) * 2, U, K, *g)
    assert "gmdn.state_scan" in targets
    assert tuple(out.shape) == (2, 3, 4, 64, 64) and out.dtype == torch.float32


@pytest.mark.parametrize("rule,d", [("delta", 128), ("adam", 64), ("muon", 64)])
def test_chunk_scan_compiles_to_one_graph(rule, d):
    with FakeTensorMode():
        q, k, v = (torch.empty(1, 2, 128, d, device="cuda", dtype=torch.bfloat16) for _ in range(3))
        gates = [torch.empty(1, 2, 128, device="cuda") for _ in range(4)]
        out, targets = _capture(lambda *x: chunk.chunk_scan(*x, rule=rule, ns=3), q, k, v, *gates)
    # every rule's forward is the one fused operator
    assert "gmdn.chunk_fwd" in targets
    assert tuple(out.shape) == (1, 2, 128, d) and out.dtype == torch.bfloat16


def test_fake_shapes():
    with FakeTensorMode():
        U, K = (torch.empty(2, 3, 4, 32, 32, device="cuda") for _ in range(2))
        g = [torch.empty(2, 3, 4, device="cuda") for _ in range(4)]
        for rule, moments in ((0, 0), (1, 1), (2, 2)):
            S, M, V = torch.ops.gmdn.state_scan(U, K, *g, rule, 3, 0, True)
            assert S.shape == U.shape
            assert [t.numel() > 0 for t in (M, V)] == [moments >= 1, moments >= 2]
            S, M, V = torch.ops.gmdn.state_scan(U, K, *g, rule, 3, 0, False)
            assert M.numel() == 0 and V.numel() == 0
        grads = torch.ops.gmdn.state_scan_bwd(U, K, *g, U, U, U, U, 2, 3, 0)
        assert [tuple(t.shape) for t in grads] == [tuple(U.shape)] * 2 + [(2, 3, 4)] * 4

        q, k, v = (torch.empty(2, 4, 256, 128, device="cuda", dtype=torch.bfloat16) for _ in range(3))
        beta, gg = (torch.empty(2, 4, 256, device="cuda") for _ in range(2))
        o, states = torch.ops.gmdn.chunk_fwd(q, k, v, beta, gg, None, None, 0, 3, 1e-6, True)
        assert o.shape == q.shape and o.dtype == torch.bfloat16
        # the delta checkpoint holds one d x d fp32 state per (b, h, even chunk)
        assert states.numel() == 2 * 4 * ((256 // 64 + 1) // 2) * 128 * 128
        o, states = torch.ops.gmdn.chunk_fwd(q, k, v, beta, gg, None, None, 0, 3, 1e-6, False)
        assert states.numel() == 0
        dq, dk, dv, db, dg, dgmu, dgnu = torch.ops.gmdn.chunk_bwd(q, k, v, beta, gg, None, None, states, q,
                                                                 0, 3, 1e-6)
        assert dq.shape == q.shape and dq.dtype == torch.bfloat16 and db.shape == beta.shape
        assert dgmu.numel() == 0 and dgnu.numel() == 0
        # a head-interleaved (B, T, H, d) stream keeps its strides in the gradients
        qi = torch.empty(2, 256, 4, 128, device="cuda", dtype=torch.bfloat16).transpose(1, 2)
        dqi = torch.ops.gmdn.chunk_bwd(qi, qi, qi, beta, gg, None, None, states, q, 0, 3, 1e-6)[0]
        assert dqi.stride() == qi.stride()


def test_cpu_tensors_never_reach_the_ops():
    q = torch.zeros(1, 1, 64, 64, dtype=torch.bfloat16)
    gg = torch.zeros(1, 1, 64)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        chunk.chunk_scan(q, q, q, gg, gg, rule="delta")


def test_front_fake_shapes():
    with FakeTensorMode():
        y = torch.empty(2, 100, 768, device="cuda", dtype=torch.bfloat16)
        w, b = torch.empty(768, 1, 4, device="cuda"), torch.empty(768, device="cuda")
        q, k, v = torch.ops.gmdn.front_fwd(y, w, b, 128)
        assert all(tuple(t.shape) == (2, 100, 256) and t.dtype == torch.bfloat16 for t in (q, k, v))
        dy, dw, db = torch.ops.gmdn.front_bwd(y, w, b, q, k, v, 128)
        assert dy.shape == y.shape and dw.shape == w.shape and db.shape == b.shape
