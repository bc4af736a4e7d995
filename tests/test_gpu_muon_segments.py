"""The drop-in muon backward (gmdn_scan_bwd, rule 1, 'tf32') runs its chunks
in segments from the end, as many chunks per segment as the workspace holds,
in one iterate buffer (each segment's iterates, then its reverse pass) or two
(the next segment's iterates formed in the launch of the current segment's
reverse pass).  With workspaces of one to six one-chunk segment buffers (one
buffer of one chunk; two of one, two and three chunks; one of all chunks) the
results are bit-identical to the default workspace (the same per-chunk
arithmetic; the state and momentum cotangents carry across segments as exact
float32)."""
import pytest
import torch

from gmdn_amd import _native as nat
from gmdn_amd import ops  # noqa: F401  -- registers torch.ops.gmdn.*
from oracle import scan as osc

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _segment_bytes(BH, nseg, dh, ns):
    mat = dh * dh
    return 4 * (BH * nseg * ((3 * ns + 2) * mat + 1) + 2 * BH * mat)


def _bwd(lib, ins, S_all, M_all, gS, ns, ws_bytes):
    B, H, N, dh, _ = ins[0].shape
    U = ins[0]
    dU, dK = torch.full_like(U, float("nan")), torch.full_like(U, float("nan"))
    ds = [torch.full_like(ins[2], float("nan")) for _ in range(4)]
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=U.device)
    args = [nat.ptr(t) for t in ins] + [nat.ptr(S_all), nat.ptr(M_all), None, nat.ptr(gS), nat.ptr(dU),
                                        nat.ptr(dK)] + [nat.ptr(t) for t in ds]
    rc = lib.gmdn_scan_bwd(*args, nat.ptr(ws), ws_bytes, B * H, N, dh, 1, ns, nat.PREC_TF32, nat.stream_of(U))
    nat.check(rc, "gmdn_scan_bwd")
    torch.cuda.synchronize()
    return [dU, dK] + ds


@pytest.mark.parametrize("B,H,N,dh,ns", [(1, 3, 7, 64, 3), (1, 2, 5, 128, 5)])
def test_muon_backward_segments_bit_identical(B, H, N, dh, ns):
    dev = _dev()
    lib = nat.load()
    print(f"muon segments B{B} H{H} N{N} d{dh} ns{ns}", flush=True)
    gen = torch.Generator().manual_seed(N * 10 + dh)
    ins = [t.to(dev).float().contiguous() for t in osc.make_scan_inputs(B, H, N, 64, dh, generator=gen)]
    gS = torch.randn(B, H, N, dh, dh, generator=gen).to(dev)
    S_all, M_all, _ = torch.ops.gmdn.state_scan(*ins, 1, ns, nat.PREC_TF32, True)
    full = lib.gmdn_scan_bwd_workspace_bytes(B * H, N, dh, 1, ns)
    assert full == _segment_bytes(B * H, N, dh, ns)  # small problems: one segment
    want = _bwd(lib, ins, S_all, M_all, gS, ns, full)
    assert all(torch.isfinite(t).all() for t in want)
    for nseg in (1, 2, 3, 4, 6):
        got = _bwd(lib, ins, S_all, M_all, gS, ns, _segment_bytes(B * H, nseg, dh, ns))
        for name, g_, w_ in zip("dU dK da db dm dn".split(), got, want):
            assert torch.equal(g_, w_), (nseg, name)


def test_muon_backward_refuses_workspace_below_one_chunk():
    """Below the one-chunk segment the call is refused before any launch."""
    lib = nat.load()
    BH, N, dh, ns = 2, 4, 64, 3
    p = [0x1000] * 16
    small = _segment_bytes(BH, 1, dh, ns) - 4
    assert lib.gmdn_scan_bwd(*p, 0x1000, small, BH, N, dh, 1, ns, nat.PREC_TF32, None) == 3


def _fused_bwd(lib, ins, states, ns, ws_bytes):
    """gmdn_chunk_bwd (muon, 'tf32') with a workspace of ws_bytes."""
    from gmdn_amd import ops
    q, k, v, beta, g, gmu, dO = ins
    outs = [torch.full_like(t, float("nan")) for t in (q, k, v, beta, g, gmu)]
    desc = ops.chunk_desc(q, k, v, dO, 1, ns, 1e-6, nat.PREC_TF32)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    rc = lib.gmdn_chunk_bwd(desc, *[nat.ptr(t) for t in (q, k, v, beta, g, gmu)], None, nat.ptr(states),
                            nat.ptr(dO), *[nat.ptr(t) for t in outs], None, nat.ptr(ws), ws_bytes,
                            nat.stream_of(q))
    nat.check(rc, "gmdn_chunk_bwd")
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("d,ns", [(64, 3), (128, 5)])
def test_fused_muon_backward_segments_bit_identical(d, ns):
    """The fused core's muon backward (gmdn_chunk_bwd, 'tf32') accepts any
    workspace down to one-chunk segments.  With two iterate buffers its
    matrix-form stage, iterate rebuild and token gradients run in the
    launches of the serial reverse scan, a segment or two ahead or behind;
    with one-chunk segments in one buffer and with two buffers of one, two
    and three chunks the gradients equal the default workspace's (one segment
    of every chunk here) bit for bit."""
    from gmdn_amd.workloads import Workload, make_inputs
    dev = _dev()
    lib = nat.load()
    B, H, N = 1, 3, 7
    print(f"fused muon segments B{B} H{H} N{N} d{d} ns{ns}", flush=True)
    inp = make_inputs(Workload("seg", "muon", B, H, N * 64, d, ns=ns), seed=N + d, with_grad_out=True)
    ins = [inp[n].to(dev).contiguous() for n in ("q", "k", "v", "beta", "g", "gmu", "dO")]
    _, states = torch.ops.gmdn.chunk_fwd(*ins[:6], None, 1, ns, 1e-6, True)
    BH, BHN, mat = B * H, B * H * N, d * d
    prefix = (4 * BHN * mat + 8 * BHN + 63) // 64 * 64

    def ws(nseg, nbuf):
        return 4 * (prefix + nbuf * BH * nseg * ((3 * ns + 2) * mat + 1) + 2 * BH * mat)

    full = lib.gmdn_chunk_bwd_workspace_bytes(ops_desc(ins, ns))
    assert full >= ws(N, 1)
    want = _fused_bwd(lib, ins, states, ns, full)
    assert all(torch.isfinite(t).all() for t in want)
    for nseg, nbuf in ((1, 1), (1, 2), (2, 2), (3, 2)):
        got = _fused_bwd(lib, ins, states, ns, ws(nseg, nbuf))
        for name, g_, w_ in zip("dq dk dv dbeta dg dgmu".split(), got, want):
            assert torch.equal(g_, w_), (nseg, nbuf, name)


def ops_desc(ins, ns):
    from gmdn_amd import ops
    q, k, v = ins[:3]
    return ops.chunk_desc(q, k, v, ins[6], 1, ns, 1e-6, nat.PREC_TF32)


@pytest.mark.parametrize("N", [16, 40, 64])
def test_fused_adam_backward_segments_bit_identical(N):
    """Adam at d = 64: with its default workspace (which holds the carry of
    Sb, Mb, Vb between segments) gmdn_chunk_bwd runs the reverse scan in
    chunk segments and each segment's token gradients on a second stream
    beside the next segment's scan; a workspace without the carry runs one
    scan pass, then the token kernel.  The gradients are equal bit for bit
    (two segments: N / 2 each at B H = 2)."""
    from gmdn_amd import ops
    from gmdn_amd.workloads import Workload, make_inputs
    dev = _dev()
    lib = nat.load()
    B, H, d = 1, 2, 64
    print(f"fused adam segments B{B} H{H} N{N} d{d}", flush=True)
    inp = make_inputs(Workload("seg", "adam", B, H, N * 64, d), seed=N, with_grad_out=True)
    ins = [inp[n].to(dev).contiguous() for n in ("q", "k", "v", "beta", "g", "gmu", "gnu", "dO")]
    q, k, v, beta, g, gmu, gnu, dO = ins
    _, states = torch.ops.gmdn.chunk_fwd(q, k, v, beta, g, gmu, gnu, 2, 3, 1e-6, True)
    desc = ops.chunk_desc(q, k, v, dO, 2, 3, 1e-6, nat.PREC_TF32)
    full = lib.gmdn_chunk_bwd_workspace_bytes(desc)
    carry = B * H * d * d * 3 * 4
    assert full > carry

    def run(ws_bytes):
        outs = [torch.full_like(t, float("nan")) for t in (q, k, v, beta, g, gmu, gnu)]
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        rc = lib.gmdn_chunk_bwd(desc, *[nat.ptr(t) for t in (q, k, v, beta, g, gmu, gnu)], nat.ptr(states),
                                nat.ptr(dO), *[nat.ptr(t) for t in outs], nat.ptr(ws), ws_bytes,
                                nat.stream_of(q))
        nat.check(rc, "gmdn_chunk_bwd")
        torch.cuda.synchronize()
        return outs

    want = run(full - carry)
    assert all(torch.isfinite(t).all() for t in want)
    got = run(full)
    for name, g_, w_ in zip("dq dk dv dbeta dg dgmu dgnu".split(), got, want):
        assert torch.equal(g_, w_), name
