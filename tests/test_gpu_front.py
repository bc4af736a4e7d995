"""The mixer front-end kernels (torch.ops.gmdn.front_fwd / front_bwd) against
the reference lines they replace, train_ablation.py:124-128 -- depthwise
Conv1d with left padding K - 1, SiLU, split, F.normalize of q and k per
head -- evaluated in float64 on the CPU with autograd for the backward.
float32 inputs: max |x - y| / max |y| <= 1e-5 (the kernels' fp32
arithmetic); bfloat16 inputs: the reference runs on the same bf16 values
in float64 and the bound is 1e-2 of the largest magnitude (bf16 output
rounding is 4e-3 of it)."""
import pytest
import torch
import torch.nn.functional as F

from gmdn_amd import ops  # noqa: F401

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _reference(y, w, b, H):
    B, T, C3 = y.shape
    D = C3 // 3
    z = F.conv1d(y.transpose(1, 2), w, b, padding=w.shape[-1] - 1, groups=C3)[..., :T].transpose(1, 2)
    a = F.silu(z)
    q, k, v = a.chunk(3, dim=-1)
    q = F.normalize(q.reshape(B, T, H, D // H), dim=-1).reshape(B, T, D)
    k = F.normalize(k.reshape(B, T, H, D // H), dim=-1).reshape(B, T, D)
    return q, k, v


def _rel(a, b):
    return ((a.double().cpu() - b).abs().max() / b.abs().max()).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,D,dh,K", [(2, 200, 256, 128, 4), (1, 64, 512, 64, 4), (3, 1, 256, 128, 4),
                                         (1, 130, 1024, 128, 3), (2, 70, 128, 64, 1), (2, 256, 128, 32, 4),
                                         (1, 100, 96, 32, 2), (2, 65, 160, 16, 4)])
def test_front_matches_reference(B, T, D, dh, K, dtype):
    dev = _dev()
    gen = torch.Generator().manual_seed(T + D + K)
    y = torch.randn(B, T, 3 * D, generator=gen).to(dtype)
    w = 0.5 * torch.randn(3 * D, 1, K, generator=gen)
    b = 0.1 * torch.randn(3 * D, generator=gen)
    dq, dk, dv = (torch.randn(B, T, D, generator=gen).to(dtype) for _ in range(3))
    # reference in float64 with autograd
    y64, w64, b64 = (t.double().requires_grad_(True) for t in (y, w, b))
    want = _reference(y64, w64, b64, D // dh)
    grads_want = torch.autograd.grad(want, (y64, w64, b64), tuple(t.double() for t in (dq, dk, dv)))
    # kernels
    yd, wd, bd = y.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    got = torch.ops.gmdn.front_fwd(yd, wd, bd, dh)
    grads = torch.autograd.grad(got, (yd, wd, bd), tuple(t.to(dev) for t in (dq, dk, dv)))
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    for name, a, r in zip("qkv", got, want):
        assert a.dtype == dtype and _rel(a.detach(), r.detach()) <= tol, (name, _rel(a.detach(), r.detach()))
    # weight and bias gradients are float32 sums over B * T terms
    gtol = (1e-5, 1e-5, 1e-5) if dtype == torch.float32 else (1e-2, 1e-2, 1e-2)
    for name, a, r, t in zip(("dy", "dweight", "dbias"), grads, grads_want, gtol):
        assert _rel(a, r) <= t, (name, _rel(a, r))


def test_front_opcheck():
    dev = _dev()
    gen = torch.Generator().manual_seed(0)
    y = torch.randn(2, 70, 384, generator=gen).to(dev).requires_grad_(True)
    w = torch.randn(384, 1, 4, generator=gen).to(dev).requires_grad_(True)
    b = torch.randn(384, generator=gen).to(dev).requires_grad_(True)
    torch.library.opcheck(torch.ops.gmdn.front_fwd.default, (y, w, b, 64),
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor",
                                      "test_aot_dispatch_static"))
