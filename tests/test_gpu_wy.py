"""GPU parity of the exact WY/UT mode (gmdn_amd/wy.py: gmdn_wy_fwd's prep,
delta-scan and output kernels; the composed training path) against the
oracle's token-exact gated delta recurrence in float64 (oracle/wy.py), on
the bf16-rounded inputs the kernels see.  Bar: the error in excess of half a
bf16 ulp of the reference (the output's own rounding) at most 2e-2 of its
RMS; gate gradients (float32) directly."""
import pytest
import torch

from gmdn_amd import wy as gwy
from oracle import wy as owy

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _half_ulp(x):
    return torch.pow(2.0, torch.floor(torch.log2(x.abs().clamp_min(1e-30))) - 8)


def _inputs(B, H, T, d, seed):
    gen = torch.Generator().manual_seed(seed)
    q, k, v, beta, g = owy.make_wy_inputs(B, H, T, d, generator=gen, dtype=torch.float32)
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    return q, k, v, beta, g


def _excess(got, ref):
    rms = ref.pow(2).mean().sqrt()
    raw = ((got - ref).abs().max() / rms).item()
    exc = (((got - ref).abs() - _half_ulp(ref)).clamp_min(0).max() / rms).item()
    return raw, exc


@pytest.mark.parametrize("B,H,T,d", [(1, 2, 64, 64), (1, 2, 256, 128), (2, 4, 1024, 128), (2, 2, 512, 64)])
def test_wy_forward_matches_token_recurrence(B, H, T, d):
    dev = _dev()
    q, k, v, beta, g = _inputs(B, H, T, d, seed=T + d)
    ref = owy.token_scan(*(t.double() for t in (q, k, v, beta, g)))
    with torch.no_grad():
        o = gwy.wy_scan(*(t.to(dev) for t in (q, k, v, beta, g)))
    torch.cuda.synchronize()
    raw, exc = _excess(o.double().cpu(), ref)
    print(f"wy B{B} H{H} T{T} d{d}: max-abs/rms {raw:.2e}, excess over half-ulp {exc:.2e}")
    assert exc <= TOL


def test_wy_recording_forward_equals_inference_forward():
    """The forward that keeps its checkpoint for a backward and the inference
    forward run the same kernels: bit-identical outputs."""
    dev = _dev()
    q, k, v, beta, g = (t.to(dev) for t in _inputs(1, 2, 512, 128, seed=7))
    with torch.no_grad():
        o_k = gwy.wy_scan(q, k, v, beta, g)
    xs = [t.detach().requires_grad_(True) for t in (q, k, v, beta, g)]
    o_c = gwy.wy_scan(*xs)
    torch.cuda.synchronize()
    assert o_c.grad_fn is not None and o_k.grad_fn is None
    assert torch.equal(o_c.detach(), o_k)


@pytest.mark.parametrize("B,H,T,d", [(1, 2, 128, 64), (1, 2, 128, 128), (2, 2, 320, 64), (1, 2, 1024, 128)])
def test_wy_gradients_match_token_recurrence(B, H, T, d):
    """The HIP backward (reverse delta scan + the chunk algebra's VJP) against
    float64 autograd of the token recurrence, up to T = 1024 at d = 128."""
    dev = _dev()
    q, k, v, beta, g = _inputs(B, H, T, d, seed=11 + d + T)
    # the cotangent as the bf16 output's gradient arrives: bf16, on both sides
    dO = torch.randn(B, H, T, d, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    xs = [t.to(dev).requires_grad_(True) for t in (q, k, v, beta, g)]
    o = gwy.wy_scan(*xs)
    got = torch.autograd.grad(o, xs, dO.to(dev))
    rs = [t.double().requires_grad_(True) for t in (q, k, v, beta, g)]
    ro = owy.token_scan(*rs)
    ref = torch.autograd.grad(ro, rs, dO.double())
    for name, a, r in zip(("q", "k", "v", "beta", "g"), got, ref):
        raw, exc = _excess(a.double().cpu(), r)
        print(f"wy B{B} H{H} T{T} d{d} d{name}: max-abs/rms {raw:.2e}, excess {exc:.2e}")
        assert (exc if name in ("q", "k", "v") else raw) <= TOL, name


@pytest.mark.parametrize("gval", [-2.0, -20.0])
def test_wy_strong_decay(gval):
    """Log-gates of -2 per token, and at the floor log 1e-6 (-20 is clamped
    to it): the decay products underflow within a chunk.  Output and
    gradients stay finite and match the token recurrence."""
    dev = _dev()
    q, k, v, beta, g = _inputs(1, 2, 256, 64, seed=21)
    g = torch.full_like(g, gval)
    ref = owy.token_scan(*(t.double() for t in (q, k, v, beta, g)))
    with torch.no_grad():
        o = gwy.wy_scan(*(t.to(dev) for t in (q, k, v, beta, g)))
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    raw, exc = _excess(o.double().cpu(), ref)
    print(f"wy strong decay g={gval}: max-abs/rms {raw:.2e}, excess {exc:.2e}")
    assert exc <= TOL
    dO = torch.randn(q.shape, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    xs = [t.to(dev).requires_grad_(True) for t in (q, k, v, beta, g)]
    got = torch.autograd.grad(gwy.wy_scan(*xs), xs, dO.to(dev))
    rs = [t.double().requires_grad_(True) for t in (q, k, v, beta, g)]
    ref_g = torch.autograd.grad(owy.token_scan(*rs), rs, dO.double())
    for name, a, r in zip(("q", "k", "v", "beta", "g"), got, ref_g):
        assert torch.isfinite(a).all(), name
        if r.abs().max() == 0:
            assert a.abs().max() == 0, name
            continue
        raw, exc = _excess(a.double().cpu(), r)
        print(f"wy strong decay g={gval} d{name}: max-abs/rms {raw:.2e}, excess {exc:.2e}")
        assert (exc if name in ("q", "k", "v") else raw) <= TOL, name


def test_wy_gradients_strided_layout():
    """q, k, v as (B, T, H, d) storage viewed as (B, H, T, d): gradients equal
    those of contiguous inputs bit for bit, in the inputs' layout."""
    dev = _dev()
    q, k, v, beta, g = (t.to(dev) for t in _inputs(2, 2, 256, 64, seed=5))
    dO = torch.randn(q.shape, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(dev)
    runs = []
    for layout in ("bhtd", "bthd"):
        xs = [t.detach().clone() for t in (q, k, v)]
        if layout == "bthd":
            xs = [t.transpose(1, 2).contiguous().transpose(1, 2) for t in xs]
        xs = [t.requires_grad_(True) for t in xs] + [t.detach().requires_grad_(True) for t in (beta, g)]
        o = gwy.wy_scan(*xs)
        runs.append((o.detach(), torch.autograd.grad(o, xs, dO)))
    torch.cuda.synchronize()
    assert torch.equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)
