"""gmdn_scan_bwd_noalloc (the drop-in backward with the library's own device
scratch in place of a caller workspace) against gmdn_scan_bwd, through the
C ABI: two calls in a row, the second on a smaller problem, must give the
same results as the allocating entry point with a fresh workspace."""
import ctypes

import pytest
import torch

from gmdn_amd import _native as nat
from gmdn_amd import ops  # noqa: F401  -- registers torch.ops.gmdn.*
from oracle import scan as osc

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _problem(B, H, N, dh, rule, ns, seed, dev):
    """Forward states of a seeded problem (through gmdn_scan_fwd) and a state
    cotangent, all float32 contiguous on the device."""
    gen = torch.Generator().manual_seed(seed)
    ins = [t.to(dev).float().contiguous() for t in osc.make_scan_inputs(B, H, N, 64, dh, generator=gen)]
    gS = torch.randn(B, H, N, dh, dh, generator=gen).to(dev)
    S_all, M_all, V_all = torch.ops.gmdn.state_scan(*ins, rule, ns, nat.PREC_TF32, True)
    return ins, S_all, M_all, V_all, gS


def _bwd(lib, ins, S_all, M_all, V_all, gS, rule, ns, noalloc):
    B, H, N, dh, _ = ins[0].shape
    U = ins[0]
    dU, dK = torch.full_like(U, float("nan")), torch.full_like(U, float("nan"))
    ds = [torch.full_like(ins[2], float("nan")) for _ in range(4)]
    mp = nat.ptr(M_all) if M_all.numel() else None
    vp = nat.ptr(V_all) if V_all.numel() else None
    common = [nat.ptr(t) for t in ins] + [nat.ptr(S_all), mp, vp, nat.ptr(gS), nat.ptr(dU), nat.ptr(dK)]
    common += [nat.ptr(t) for t in ds]
    stream = nat.stream_of(U)
    if noalloc:
        rc = lib.gmdn_scan_bwd_noalloc(*common, B * H, N, dh, rule, ns, nat.PREC_TF32, stream)
    else:
        need = lib.gmdn_scan_bwd_workspace_bytes(B * H, N, dh, rule, ns)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=U.device)
        rc = lib.gmdn_scan_bwd(*common, nat.ptr(ws), need, B * H, N, dh, rule, ns, nat.PREC_TF32, stream)
    nat.check(rc, "gmdn_scan_bwd_noalloc" if noalloc else "gmdn_scan_bwd")
    torch.cuda.synchronize()
    return [dU, dK] + ds


@pytest.mark.parametrize("rule,ns", [(0, 3), (1, 5), (2, 3)])
def test_noalloc_matches_workspace_entry_point(rule, ns):
    dev = _dev()
    lib = nat.load()
    # two calls in a row, the second smaller (fewer heads, chunks and a
    # smaller head dim): its results must not depend on what the first left
    for B, H, N, dh in ((2, 3, 9, 128), (1, 2, 4, 64)):
        print(f"noalloc rule={rule} ns={ns} B{B} H{H} N{N} d{dh}", flush=True)
        assert lib.gmdn_scan_bwd_workspace_bytes(B * H, N, dh, rule, ns) <= SCRATCH
        prob = _problem(B, H, N, dh, rule, ns, seed=B * 100 + N, dev=dev)
        want = _bwd(lib, *prob, rule, ns, noalloc=False)
        got = _bwd(lib, *prob, rule, ns, noalloc=True)
        for name, g_, w_ in zip("dU dK da db dm dn".split(), got, want):
            assert torch.equal(g_, w_), name


def _muon_min_workspace(BH, dh, ns):
    """Bytes of the muon backward's one-chunk segments: per (b, h) 3 ns + 2
    dh^2 matrices and |M_i|, plus the two carried dh^2 matrices."""
    mat = dh * dh
    return 4 * (BH * ((3 * ns + 2) * mat + 1) + 2 * BH * mat)


def test_noalloc_refuses_problems_beyond_the_scratch():
    """A muon backward whose smallest workspace (one-chunk segments) exceeds
    the 64 MiB scratch is refused with GMDN_ERR_WORKSPACE before any launch
    (the pointers are never read)."""
    lib = nat.load()
    BH, N, dh, ns = 128, 64, 128, 5
    assert _muon_min_workspace(BH, dh, ns) > SCRATCH
    assert lib.gmdn_scan_bwd_workspace_bytes(BH, N, dh, 1, ns) > SCRATCH
    p = [0x1000] * 16
    assert lib.gmdn_scan_bwd_noalloc(*p, BH, N, dh, 1, ns, nat.PREC_TF32, None) == 3
    # argument errors are reported as by gmdn_scan_bwd
    assert lib.gmdn_scan_bwd_noalloc(*p, BH, N, 48, 1, ns, nat.PREC_TF32, None) == 2
    assert lib.gmdn_scan_bwd_noalloc(*p, BH, N, dh, 5, ns, nat.PREC_TF32, None) == 1
