"""Fused mixer-core op (Level B): phases 1-3 of the reference mixer in one
HIP kernel per direction.

``chunk_scan(q, k, v, beta, g, gmu=None, gnu=None, rule='delta', ns=3)``
computes what ``FastWeightMixer.forward`` computes between its front-end and
its per-head RMSNorm (reference train_ablation.py:142-187): the chunk
transform A, Kw, Uv, Qt, Ov, the state scan, and ``o = Qt S^T + Ov``.

* ``q, k, v``: (B, H, T, d) bfloat16, d contiguous (any strides over B, H, T
  that are multiples of 8 elements), q and k L2-normalised per head.
* ``beta``: (B, H, T) beta gate (sigmoid output).
* ``g, gmu, gnu``: (B, H, T) log alpha, log mu, log nu gates.  The reference
  clamps each gate at 1e-6 before its log (train_ablation.py:155, :170-175);
  the kernel clamps the log at log(1e-6), which is the same function.
  ``gmu`` is needed by the muon and adam rules, ``gnu`` by adam.
* returns ``o`` (B, H, T, d) in q's dtype.

Chunk length is 64 (the reference default and every configuration's).

Delta and adam run as one fused HIP kernel per direction (forward: the
chunk transform, the scan and the output; backward: a reverse scan of the
state cotangent and a chunk-parallel token-gradient kernel).  Muon's msign
couples the whole state, so its recurrence runs in the drop-in scan's muon
kernel (Newton-Schulz fused into the scan step) with phases 1 and 3 as
batched GEMMs around it.
"""
from __future__ import annotations

import math

import torch

from . import _native as nat
from .scan import HipScan

RULES = {"delta": 0, "muon": 1, "adam": 2}
CHUNK = 64
LOG_FLOOR = math.log(1e-6)
SUPPORTED_D = (64, 128)


BWD_RULES = (0, 1, 2)  # rules with a backward (muon: through the scan kernel's VJP)


def backward_supported(rule, d: int = 128) -> bool:
    """Whether the fused backward of ``rule`` at head dim ``d`` is built.  The
    adam backward is limited to d = 64: at d = 128 its sign-like update
    amplifies the rounding of the split-bf16 state products past the
    gradient tolerance."""
    r = _rule_id(rule)
    return r in BWD_RULES and (r != 2 or d == 64)


def _rule_id(rule) -> int:
    if isinstance(rule, str):
        if rule not in RULES:
            raise ValueError(f"rule must be one of {tuple(RULES)}, got {rule!r}")
        return RULES[rule]
    if rule not in (0, 1, 2):
        raise ValueError(f"rule must be 0, 1 or 2, got {rule}")
    return int(rule)


def _desc(q, k, v, o, rule, ns, eps):
    B, H, T, d = q.shape
    desc = nat.ChunkDesc()
    desc.B, desc.H, desc.T, desc.d, desc.C = B, H, T, d, CHUNK
    desc.rule, desc.ns, desc.dtype, desc.eps = rule, ns, nat.DTYPE_BF16, eps
    for name, t in (("sq", q), ("sk", k), ("sv", v), ("so", o)):
        arr = getattr(desc, name)
        for i in range(3):
            arr[i] = t.stride(i)
    return desc


def _check(q, k, v, beta, g, gmu, gnu, rule):
    if not q.is_cuda:
        raise RuntimeError("chunk_scan needs GPU tensors")
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise RuntimeError(f"q, k, v must be (B, H, T, d) of equal shape, got {tuple(q.shape)}, "
                           f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, H, T, d = q.shape
    if d not in SUPPORTED_D:
        raise RuntimeError(f"chunk_scan supports head dims {SUPPORTED_D}, got {d}")
    if T % CHUNK:
        raise RuntimeError(f"T must be a multiple of the chunk length {CHUNK}, got {T}")
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise RuntimeError("chunk_scan takes bfloat16 q, k, v")
    for name, t in (("beta", beta), ("g", g), ("gmu", gmu), ("gnu", gnu)):
        if t is not None and tuple(t.shape) != (B, H, T):
            raise RuntimeError(f"{name} must be (B, H, T) = {(B, H, T)}, got {tuple(t.shape)}")
    if rule >= 1 and gmu is None:
        raise RuntimeError("muon and adam rules need gmu")
    if rule == 2 and gnu is None:
        raise RuntimeError("adam rule needs gnu")


def _tok(t):
    """bf16 token stream with a unit-stride last dim and 16-byte-aligned rows."""
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _gate(t):
    """float32 (B, H, T) gate stream, contiguous and 16-byte aligned."""
    if t is None:
        return None
    t = t.detach().to(torch.float32).contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class ChunkScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, beta, g, gmu, gnu, rule, ns, eps, record):
        _check(q, k, v, beta, g, gmu, gnu, rule)
        lib = nat.load()
        qc, kc, vc = _tok(q.detach()), _tok(k.detach()), _tok(v.detach())
        bc, gc, mc, nc = _gate(beta), _gate(g), _gate(gmu), _gate(gnu)
        o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        desc = _desc(qc, kc, vc, o, rule, ns, eps)
        # `record`: grad mode was on at the call (inside forward it is always
        # off, and needs_input_grad ignores it), so a backward may follow
        need_grad = record and any(ctx.needs_input_grad[:7])
        states = None
        if need_grad:
            nbytes = lib.gmdn_chunk_states_bytes(desc)
            states = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
        with torch.cuda.device(q.device):
            rc = lib.gmdn_chunk_fwd(desc, nat.ptr(qc), nat.ptr(kc), nat.ptr(vc), nat.ptr(bc), nat.ptr(gc),
                                    nat.ptr(mc), nat.ptr(nc), nat.ptr(o), nat.ptr(states), nat.stream_of(q))
        nat.check(rc, "gmdn_chunk_fwd")
        if need_grad:
            ctx.save_for_backward(qc, kc, vc, bc, gc, mc, nc, states)
        ctx.rule, ctx.ns, ctx.eps = rule, ns, eps
        ctx.gate_dtypes = tuple(None if t is None else t.dtype for t in (beta, g, gmu, gnu))
        return o

    @staticmethod
    def backward(ctx, dO):
        qc, kc, vc, bc, gc, mc, nc, states = ctx.saved_tensors
        lib = nat.load()
        dOc = _tok(dO.to(torch.bfloat16))
        if not backward_supported(ctx.rule, qc.shape[-1]):
            raise RuntimeError(f"the fused backward of rule {ctx.rule} at head dim {qc.shape[-1]} is not built")
        # gradients share the strides of q, k, v (the kernels write them with those strides)
        dq, dk, dv = (torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=t.device)
                      for t in (qc, kc, vc))
        dbeta, dg = torch.empty_like(bc), torch.empty_like(gc)
        dgmu = torch.empty_like(mc) if mc is not None else None
        dgnu = torch.empty_like(nc) if nc is not None else None
        desc = _desc(qc, kc, vc, dOc, ctx.rule, ctx.ns, ctx.eps)
        ws_bytes = lib.gmdn_chunk_bwd_workspace_bytes(desc)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=qc.device) if ws_bytes else None
        with torch.cuda.device(qc.device):
            rc = lib.gmdn_chunk_bwd(desc, nat.ptr(qc), nat.ptr(kc), nat.ptr(vc), nat.ptr(bc), nat.ptr(gc),
                                    nat.ptr(mc), nat.ptr(nc), nat.ptr(states), nat.ptr(dOc), nat.ptr(dq),
                                    nat.ptr(dk), nat.ptr(dv), nat.ptr(dbeta), nat.ptr(dg), nat.ptr(dgmu),
                                    nat.ptr(dgnu), nat.ptr(ws), ws_bytes, nat.stream_of(qc))
        nat.check(rc, "gmdn_chunk_bwd")
        gates = [None if t is None else t.to(dt) for t, dt in zip((dbeta, dg, dgmu, dgnu), ctx.gate_dtypes)]
        return (dq, dk, dv, *gates, None, None, None, None)


def _muon_core(q, k, v, beta, g, gmu, ns):
    """The muon rule's mixer core.  msign couples every entry of the d x d
    state, so the recurrence runs as the drop-in scan's muon kernel (one
    workgroup per (b, h), Newton-Schulz fused into the scan step); phases 1
    and 3 of the reference mixer (train_ablation.py:150-167, :184-187) are
    plain batched GEMMs in float32 around it.  Autograd supplies the
    backward, through the scan kernel's fused msign VJP."""
    B, H, T, d = q.shape
    N = T // CHUNK
    qf, kf, vf = (t.float().reshape(B, H, N, CHUNK, d) for t in (q, k, v))
    bt = beta.float().reshape(B, H, N, CHUNK)
    lg = torch.clamp(g.float(), min=LOG_FLOOR).reshape(B, H, N, CHUNK)
    lmu = torch.clamp(gmu.float(), min=LOG_FLOOR).reshape(B, H, N, CHUNK)
    a = lg.sum(-1).exp()
    b = bt.mean(-1)
    m = lmu.sum(-1).exp()
    n = torch.ones_like(m)
    # token weights prod_{s' > s} mu_{s'} (train_ablation.py:154-156)
    w = torch.exp(torch.flip(torch.cumsum(torch.flip(lmu, [-1]), -1), [-1]) - lmu)
    causal = torch.tril(torch.ones(CHUNK, CHUNK, dtype=torch.bool, device=q.device))
    kT = kf.transpose(-1, -2).contiguous()
    A = torch.where(causal, torch.matmul(qf, kT) * bt.unsqueeze(-2), 0.0)
    Kw = torch.matmul((kf * w.unsqueeze(-1)).transpose(-1, -2).contiguous(), kf)
    Uv = torch.matmul((vf * w.unsqueeze(-1)).transpose(-1, -2).contiguous(), kf)
    Qt = qf - torch.matmul(A, kf)
    Ov = torch.matmul(A, vf)
    S_all = HipScan.apply(Uv, Kw, a, b, m, n, 1, ns)
    o = torch.matmul(Qt, S_all.transpose(-1, -2).contiguous()) + Ov
    return o.reshape(B, H, T, d).to(q.dtype)


def chunk_scan(q, k, v, beta, g, gmu=None, gnu=None, *, rule="delta", ns: int = 3, eps: float = 1e-6):
    """Fused mixer core; see the module docstring."""
    r = _rule_id(rule)
    if r == 1:
        _check(q, k, v, beta, g, gmu, gnu, r)
        return _muon_core(q, k, v, beta, g, gmu, ns)
    return ChunkScan.apply(q, k, v, beta, g, gmu if r >= 1 else None, gnu if r == 2 else None, r, ns, eps,
                           torch.is_grad_enabled())
