"""GPU parity of the mixer's gate-activation and per-head RMSNorm kernels
(csrc/tail.hip, through torch.ops.gmdn.*) against torch in float64: the
reference's torch.sigmoid(self.gates(x)) with the gates' clamped logs
(train_ablation.py:131-134, :152-175) and nn.RMSNorm(dh) on each head's
output (:188), forward and backward."""
import math

import pytest
import torch
import torch.nn.functional as F

from gmdn_amd import ops  # noqa: F401

pytestmark = pytest.mark.gpu
FLOOR = math.log(1e-6)


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _gates_ref(y, H, nG):
    B, T, _ = y.shape
    g = y.view(B, T, nG, H).permute(2, 0, 3, 1)
    out = torch.log(torch.sigmoid(g).clamp_min(1e-6))
    out = torch.cat([out[:1], torch.sigmoid(g[1:2]), out[2:]], 0)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,nG", [(2, 256, 8, 3), (1, 200, 16, 4), (3, 64, 2, 3)])
def test_gates_forward_backward(B, T, H, nG, dtype):
    dev = _dev()
    gen = torch.Generator().manual_seed(B * T + H)
    y = (4 * torch.randn(B, T, nG * H, generator=gen)).to(dtype)
    y[0, :3, :] = -20.0   # gates below the 1e-6 floor: clamped, no gradient
    y[0, 3:5, :] = 30.0
    dout = torch.randn(nG, B, H, T, generator=gen, dtype=torch.float64)
    y64 = y.double().requires_grad_(True)
    ref = _gates_ref(y64, H, nG)
    (dy_ref,) = torch.autograd.grad(ref, y64, dout)
    yd = y.to(dev).requires_grad_(True)
    got = torch.ops.gmdn.gates_fwd(yd, H, nG)
    (dy,) = torch.autograd.grad(got, yd, dout.float().to(dev))
    torch.cuda.synchronize()
    assert got.shape == (nG, B, H, T) and got.dtype == torch.float32
    err = (got.double().cpu() - ref).abs().max().item()
    # float32 evaluation of sigmoid / log sigmoid of the (exact) inputs
    assert err <= 1e-5 * max(1.0, ref.abs().max().item()), err
    derr = (dy.double().cpu() - dy_ref).abs().max().item() / dy_ref.abs().max().item()
    tol = 1e-5 if dtype == torch.float32 else 8e-3  # dy in y's dtype: bf16 rounding
    assert derr <= tol, derr
    # floored log gates get no gradient (beta's channels keep sigmoid')
    logs = [g for g in range(nG) if g != 1]
    assert all(dy[0, :3, g * H:(g + 1) * H].abs().max().item() == 0.0 for g in logs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,d", [(4096, 128), (999, 64), (1, 128), (777, 32), (300, 16)])
def test_head_norm_forward_backward(rows, d, dtype):
    dev = _dev()
    gen = torch.Generator().manual_seed(rows + d)
    x = torch.randn(rows, d, generator=gen).to(dtype)
    w = 1 + 0.1 * torch.randn(d, generator=gen)
    eps = torch.finfo(dtype).eps
    dout = torch.randn(rows, d, generator=gen, dtype=torch.float64)
    x64, w64 = x.double().requires_grad_(True), w.double().requires_grad_(True)
    ref = F.rms_norm(x64, (d,), w64, eps)
    dx_ref, dw_ref = torch.autograd.grad(ref, (x64, w64), dout)
    xd, wd = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
    out, rstd = torch.ops.gmdn.head_norm_fwd(xd, wd, eps)
    dx, dw = torch.autograd.grad(out, (xd, wd), dout.to(dtype).to(dev))
    torch.cuda.synchronize()
    scale = ref.abs().max().item()
    tol = 1e-5 if dtype == torch.float32 else 8e-3  # outputs in x's dtype
    assert (out.double().cpu() - ref).abs().max().item() <= tol * scale
    assert (dx.double().cpu() - dx_ref).abs().max().item() <= tol * 2 * dx_ref.abs().max().item()
    dwtol = 1e-5 if dtype == torch.float32 else 2e-2
    assert (dw.double().cpu() - dw_ref).abs().max().item() <= dwtol * dw_ref.abs().max().item()
    r64 = 1 / torch.sqrt(x.double().pow(2).mean(-1) + eps)
    assert torch.allclose(rstd.double().cpu(), r64, rtol=1e-5)


def test_head_norm_weight_gradient_is_deterministic():
    """The weight gradient is summed per workgroup and then in a fixed order:
    two calls give bit-identical results."""
    dev = _dev()
    x = torch.randn(20000, 128, device=dev)
    w = torch.ones(128, device=dev, requires_grad=True)
    g = torch.randn(20000, 128, device=dev)
    dws = []
    for _ in range(2):
        out, _ = torch.ops.gmdn.head_norm_fwd(x, w, 1e-6)
        (dw,) = torch.autograd.grad(out, w, g)
        dws.append(dw)
    assert torch.equal(dws[0], dws[1])


@pytest.mark.parametrize("d", [64, 128])
def test_head_norm_bf16_io_equals_float32_then_rounded(d):
    """Under bfloat16 autocast the mixer runs the head norm on the bfloat16
    output directly (no float32 copy): that is bit for bit the float32 norm
    rounded to bfloat16, as autocast rounds it before the projection (and its
    input gradient likewise)."""
    dev = _dev()
    torch.manual_seed(0)
    x = torch.randn(3000, d, device=dev).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(d, device=dev)).requires_grad_(True)
    g = torch.randn(3000, d, device=dev).to(torch.bfloat16)
    xa = x.clone().requires_grad_(True)
    ya, _ = torch.ops.gmdn.head_norm_fwd(xa, w, 1e-6)
    dxa, dwa = torch.autograd.grad(ya, (xa, w), g)
    xb = x.float().requires_grad_(True)
    yb, _ = torch.ops.gmdn.head_norm_fwd(xb, w, 1e-6)
    dxb, dwb = torch.autograd.grad(yb, (xb, w), g.float())
    torch.cuda.synchronize()
    assert ya.dtype == torch.bfloat16 and torch.equal(ya, yb.to(torch.bfloat16))
    assert torch.equal(dxa, dxb.to(torch.bfloat16))
    assert torch.equal(dwa, dwb)
