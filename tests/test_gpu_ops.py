"""GPU checks of the registered operators: torch.library.opcheck (schema,
fake implementation and autograd registration against the real kernels) and
a torch.compile'd forward + backward (whole graph, aot_eager: torch's
autograd tracing with no code generation) equal to the eager call."""
import pytest
import torch

from gmdn_amd import chunk, ops  # noqa: F401
from gmdn_amd.workloads import Workload, make_inputs
from oracle import scan as osc

pytestmark = pytest.mark.gpu

STATIC_CHECKS = ("test_schema", "test_autograd_registration", "test_faketensor", "test_aot_dispatch_static")


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _scan_inputs(dev, rule, dh=32):
    gen = torch.Generator().manual_seed(rule)
    return [t.to(dev) for t in osc.make_scan_inputs(1, 2, 3, 16, dh, generator=gen)]


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_opcheck_state_scan(rule):
    dev = _dev()
    ins = [t.requires_grad_(True) for t in _scan_inputs(dev, rule)]
    torch.library.opcheck(torch.ops.gmdn.state_scan.default, (*ins, rule, 2, 0, True), test_utils=STATIC_CHECKS)


@pytest.mark.parametrize("rule,d,dtype", [("delta", 64, torch.bfloat16), ("adam", 64, torch.bfloat16),
                                           ("muon", 64, torch.bfloat16), ("muon", 128, torch.bfloat16),
                                           ("delta", 32, torch.float32), ("adam", 64, torch.float32),
                                           ("muon", 64, torch.float32)])
def test_opcheck_chunk_fwd(rule, d, dtype):
    dev = _dev()
    inp = make_inputs(Workload("t", rule, 1, 2, 128, d), seed=0, device=dev, dtype=dtype)
    r = chunk.RULES[rule]
    args = (inp["q"], inp["k"], inp["v"], inp["beta"], inp["g"], inp["gmu"] if r >= 1 else None,
            inp["gnu"] if r == 2 else None)
    args = tuple(t if t is None else t.detach().requires_grad_(True) for t in args)
    torch.library.opcheck(torch.ops.gmdn.chunk_fwd.default, (*args, r, 3, 1e-6, True), test_utils=STATIC_CHECKS)


def _compiled_vs_eager(fn, xs, cot):
    def step(f):
        ys = [x.detach().requires_grad_(True) for x in xs]
        out = f(*ys)
        grads = torch.autograd.grad(out, ys, cot)
        return out.detach(), grads

    torch._dynamo.reset()
    out_e, g_e = step(fn)
    out_c, g_c = step(torch.compile(fn, backend="aot_eager", fullgraph=True))
    # the same kernels run both ways (the fused kernels' sums have a fixed
    # order); the traced graph may still order or lay out the torch ops
    # around them differently, hence a tolerance of a few fp32 ulps
    torch.testing.assert_close(out_c, out_e, rtol=1e-5, atol=1e-6)
    for a, b in zip(g_c, g_e):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_compiled_state_scan_matches_eager(rule):
    import fast_scan
    dev = _dev()
    fast_scan.set_backend("triton")
    try:
        ins = _scan_inputs(dev, rule, dh=64)
        gS = torch.randn(ins[0].shape, generator=torch.Generator().manual_seed(9)).to(dev)
        _compiled_vs_eager(lambda *x: fast_scan.fast_state_scan(*x, rule, 3), ins, gS)
    finally:
        fast_scan.set_backend("auto")


@pytest.mark.parametrize("rule", ["delta", "adam", "muon"])
def test_compiled_chunk_scan_matches_eager(rule):
    dev = _dev()
    inp = make_inputs(Workload("t", rule, 1, 2, 256, 64), seed=1, device=dev, with_grad_out=True)
    names = ["q", "k", "v", "beta", "g"] + (["gmu"] if rule != "delta" else []) + (["gnu"] if rule == "adam" else [])
    _compiled_vs_eager(lambda *x: chunk.chunk_scan(*x, rule=rule, ns=3), [inp[n] for n in names], inp["dO"])


@pytest.mark.parametrize("view", ["expanded", "qkv_slice"])
def test_chunk_scan_on_aliased_and_gapped_streams(view):
    """q as an expanded view (one head's stream broadcast over the heads: zero
    stride, rows alias) and as a slice of a fused (B, H, T, 3 d) projection
    (gaps between rows): outputs and gradients equal those of contiguous
    copies, and o and dq come back dense (no aliased rows, no holes)."""
    dev = _dev()
    inp = make_inputs(Workload("t", "delta", 1, 4, 256, 64), seed=6, device=dev, with_grad_out=True)
    if view == "expanded":
        base = inp["q"][:, :1].detach().requires_grad_(True)
        q = base.expand(-1, 4, -1, -1)
    else:
        fused = torch.cat([inp["q"], inp["k"], inp["v"]], dim=-1).detach().requires_grad_(True)
        base = fused
        q = fused[..., :64]
    assert q.stride(1) == 0 or q.stride(2) == 192
    k, v = (inp[n].detach().requires_grad_(True) for n in ("k", "v"))
    o = chunk.chunk_scan(q, k, v, inp["beta"], inp["g"], rule="delta")
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), inp["dO"])
    qc = q.detach().contiguous().requires_grad_(True)
    kc, vc = (t.detach().clone().requires_grad_(True) for t in (k, v))
    oc_ = chunk.chunk_scan(qc, kc, vc, inp["beta"], inp["g"], rule="delta")
    gc_ = torch.autograd.grad(oc_, (qc, kc, vc), inp["dO"])
    torch.cuda.synchronize()
    assert torch.equal(o, oc_)
    for a, b in zip((dq, dk, dv), gc_):
        assert torch.equal(a, b)
    for t in (o, dq):
        assert ops._dense_permutation(t), t.stride()
