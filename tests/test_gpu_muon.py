"""Parity of the outer-Muon msign kernels (csrc/msign.hip) with the oracle.

fp32 inputs: max|x - y| / max|y| <= 1e-4 against the oracle's float64 msign
(the reference computes in float32 with TF32 matmuls, train_ablation.py:60-73,
608-610; the kernels' split bf16 products carry about 2^-16 relative error,
and five NS steps stay inside the bar for the N(0, 1) inputs of the
reference's tests).  bf16 inputs: max-abs / RMS <= 2e-2 after the cast back to
bf16.  At the LM's full weight shapes: one matrix of each batch against the
oracle, and every batch entry bit-identical to the same matrix alone.
"""
import pytest
import torch

from oracle import muon as om
from oracle.scan import rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _msign():
    from gmdn_amd import muon
    return muon.msign


SHAPES = [(128, 128), (256, 384), (384, 256), (24, 1024), (1024, 24), (100, 37), (37, 100), (1, 1), (3, 5),
          (1, 300), (300, 1), (129, 257)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("steps", [0, 1, 5])
def test_msign_fp32_matches_oracle(shape, steps):
    print(f"msign fp32 shape={shape} steps={steps}", flush=True)
    g = torch.Generator().manual_seed(1000 + 7 * steps + shape[0] + 3 * shape[1])
    M = torch.randn(*shape, generator=g)
    ref = om.msign(M.double(), steps, compute_dtype=torch.float64)
    got = _msign()(M.to(DEV), steps).cpu()
    assert got.dtype == torch.float32 and got.shape == M.shape
    assert rel_err(got, ref) <= 1e-4, rel_err(got, ref)


def test_msign_batched_and_ragged():
    g = torch.Generator().manual_seed(5)
    M = torch.randn(5, 96, 200, generator=g)
    got = _msign()(M.to(DEV), 5).cpu()
    for i in range(5):
        ref = om.msign(M[i].double(), 5, compute_dtype=torch.float64)
        assert rel_err(got[i], ref) <= 1e-4


def test_msign_bf16_and_other_dtypes():
    g = torch.Generator().manual_seed(6)
    M = torch.randn(3, 200, 120, generator=g).bfloat16()
    got = _msign()(M.to(DEV), 5).cpu()
    assert got.dtype == torch.bfloat16
    ref = om.msign(M.double(), 5, compute_dtype=torch.float64)
    err = (got.double() - ref).abs().max() / ref.pow(2).mean().sqrt()
    assert err <= 2e-2, float(err)
    # float16 goes through float32 and comes back as float16
    h = _msign()(M.half().to(DEV), 5)
    assert h.dtype == torch.float16


def test_msign_empty_and_scaled_input():
    assert _msign()(torch.empty(0, 4, 4, device=DEV), 5).shape == (0, 4, 4)
    g = torch.Generator().manual_seed(7)
    M = torch.randn(64, 96, generator=g)
    a = _msign()(M.to(DEV), 5).cpu()
    b = _msign()((1000.0 * M).to(DEV), 5).cpu()  # msign is scale-invariant up to eps
    assert rel_err(b, a) <= 1e-4


@pytest.mark.parametrize("rows,cols", [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)])
def test_msign_lm_shapes(rows, cols):
    """The LM's hidden weight shapes (qkv, out, mlp in, mlp out), a batch of 3."""
    print(f"msign lm shape=({rows},{cols})", flush=True)
    g = torch.Generator().manual_seed(rows + cols)
    M = torch.randn(3, rows, cols, generator=g)
    got = _msign()(M.to(DEV), 5)
    ref = om.msign(M[1].double(), 5, compute_dtype=torch.float64)
    assert rel_err(got[1].cpu(), ref) <= 1e-4
    alone = _msign()(M[2:3].to(DEV), 5)
    assert torch.equal(alone[0], got[2])


@pytest.mark.parametrize("nesterov,wd", [(True, 0.1), (False, 0.0)])
def test_muon_optimizer_matches_oracle(nesterov, wd):
    from gmdn_amd.muon import Muon
    g = torch.Generator().manual_seed(8)
    shapes = [(64, 96), (96, 64), (32, 32), (32, 32), (24, 128)]
    init = [torch.randn(*s, generator=g) * 0.02 for s in shapes]
    grads = [[torch.randn(*s, generator=g) for s in shapes] for _ in range(3)]
    params = [torch.nn.Parameter(p.clone().to(DEV)) for p in init]
    opt = Muon(params, lr=0.02, momentum=0.95, nesterov=nesterov, weight_decay=wd, ns_steps=5)
    ref = [p.clone().double() for p in init]
    bufs = [None] * len(shapes)
    for step in range(3):
        for p, gr in zip(params, grads[step]):
            p.grad = gr.to(DEV)
        opt.step()
        bufs = om.muon_step(ref, [gr.double() for gr in grads[step]], bufs, lr=0.02, momentum=0.95, nesterov=nesterov,
                            weight_decay=wd, ns_steps=5, compute_dtype=torch.float64)
    for i, (p, r, p0) in enumerate(zip(params, ref, init)):
        upd, upd_ref = p.detach().cpu().double() - p0.double(), r - p0.double()
        assert rel_err(upd, upd_ref) <= 1e-4
        torch.testing.assert_close(opt.state[p]["buf"].cpu().double(), bufs[i], rtol=1e-6, atol=1e-6)
