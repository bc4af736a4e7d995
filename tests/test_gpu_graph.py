"""The fused mixer core's training step under HIP graph capture.

The library's launches take the caller's stream and allocate, clear and
synchronise nothing themselves (torch allocates the outputs and workspace),
so a forward + backward of ``chunk_scan`` captures into one graph.  Each
test captures the step, then replays it several times with the program's own
eager work and synchronisations in between, and requires every replay to
reproduce the eager step bit for bit (the kernels are deterministic, the
gate-gradient sums included).
"""
import pytest
import torch

from gmdn_amd import chunk as gc
from gmdn_amd.workloads import Workload, make_inputs

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


# muon at B=2, H=16, T=1024, d=128: sixteen chunks in segments of fourteen,
# so the backward runs its pipelined segment launches (two iterate buffers)
@pytest.mark.parametrize("rule,d,T,H", [("delta", 128, 512, 2), ("delta", 64, 320, 2), ("adam", 64, 512, 2),
                                        ("adam", 64, 2560, 2), ("muon", 128, 1024, 16)])
def test_training_step_graph_replays_match_eager(rule, d, T, H):
    dev = _dev()
    w = Workload(f"graph_{rule}", rule, 2, H, T, d)
    print(f"case graph rule={rule} d={d} T={T} H={H}", flush=True)
    inp = make_inputs(w, seed=3, device=dev)
    names = ("q", "k", "v", "beta", "g", "gmu", "gnu")
    xs = [None if inp[n] is None else inp[n].detach().requires_grad_(True) for n in names]
    wrt = [x for x in xs if x is not None]
    dO = inp["dO"]

    def step():
        o = gc.chunk_scan(*xs, rule=rule, ns=w.ns)
        return (o,) + tuple(torch.autograd.grad(o, wrt, dO))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    torch.cuda.synchronize()
    ref = [t.detach().clone() for t in step()]
    torch.cuda.synchronize()

    for rep in range(3):
        # eager work and a synchronisation between the replays
        other = step()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, (a, b) in enumerate(zip(outs, ref)):
            assert torch.equal(a, b), f"replay {rep}: output {k} differs from the eager step"
        for k, (a, b) in enumerate(zip(other, ref)):
            assert torch.equal(a, b), f"eager step {rep}: output {k} differs"
