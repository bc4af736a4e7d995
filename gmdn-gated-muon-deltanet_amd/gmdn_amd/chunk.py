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
couples the whole state: its forward is a serial HIP kernel per (b, h) that
streams the k, v tiles and forms each chunk's update in the E-form before
the Newton-Schulz steps, plus a chunk-parallel output kernel; its backward
is HIP too: a chunk-parallel kernel forms each chunk's Kw, Uv and dL/dS_i,
the drop-in muon scan's backward kernels run the Newton-Schulz VJP, and the
token-gradient kernel finishes in the E-form.  Adam at d = 128 trains through the drop-in scan with
phases 1 and 3 as batched GEMMs around it, the scan in exact float32 (its
inference forward stays fused).
"""
from __future__ import annotations

import math

import torch

from . import ops  # noqa: F401  -- registers torch.ops.gmdn.*
from .scan import hip_state_scan

RULES = {"delta": 0, "muon": 1, "adam": 2}
CHUNK = 64
LOG_FLOOR = math.log(1e-6)
SUPPORTED_D = (64, 128)


BWD_RULES = (0, 1, 2)  # rules with a backward


def backward_supported(rule, d: int = 128) -> bool:
    """Whether ``rule`` at head dim ``d`` has a backward: every rule and head
    dim.  (The fused adam backward kernel is limited to d = 64 -- at d = 128
    its sign-like update amplifies the rounding of the split-bf16 state
    products past the gradient tolerance -- so adam at d = 128 trains through
    the composed path of ``_composed_core``.)"""
    return _rule_id(rule) in BWD_RULES


def fused_backward(rule, d: int) -> bool:
    """Whether ``rule`` at head dim ``d`` trains through the fused forward
    (delta and adam at d = 64; muon at both head dims, its Newton-Schulz
    VJP through the drop-in scan's backward kernels)."""
    r = _rule_id(rule)
    return r in (0, 1) or (r == 2 and d == 64)


def _rule_id(rule) -> int:
    if isinstance(rule, str):
        if rule not in RULES:
            raise ValueError(f"rule must be one of {tuple(RULES)}, got {rule!r}")
        return RULES[rule]
    if rule not in (0, 1, 2):
        raise ValueError(f"rule must be 0, 1 or 2, got {rule}")
    return int(rule)


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


def _composed_core(q, k, v, beta, g, gmu, gnu, rule, ns, precision=None):
    """The mixer core as the reference composes it: phases 1 and 3
    (train_ablation.py:150-167, :184-187) as plain batched GEMMs in float32
    around the drop-in scan kernels, with autograd supplying the backward
    through the scan's own backward kernels.

    Adam at d = 128 trains this way with the scan in exact float32
    (precision 'ieee'), where the fused kernels' split products would exceed
    the gradient tolerance."""
    B, H, T, d = q.shape
    N = T // CHUNK
    qf, kf, vf = (t.float().reshape(B, H, N, CHUNK, d) for t in (q, k, v))
    bt = beta.float().reshape(B, H, N, CHUNK)
    lg = torch.clamp(g.float(), min=LOG_FLOOR).reshape(B, H, N, CHUNK)
    lmu = torch.clamp(gmu.float(), min=LOG_FLOOR).reshape(B, H, N, CHUNK)
    a = lg.sum(-1).exp()
    b = bt.mean(-1)
    m = lmu.sum(-1).exp()
    if rule == 2:
        n = torch.clamp(gnu.float(), min=LOG_FLOOR).reshape(B, H, N, CHUNK).sum(-1).exp()
        w = torch.ones_like(bt)  # adam weighs every token of a chunk equally (train_ablation.py:158)
    else:
        n = torch.ones_like(m)
        # token weights prod_{s' > s} mu_{s'} (train_ablation.py:154-156)
        w = torch.exp(torch.flip(torch.cumsum(torch.flip(lmu, [-1]), -1), [-1]) - lmu)
    causal = torch.tril(torch.ones(CHUNK, CHUNK, dtype=torch.bool, device=q.device))
    # float32 batched products take the transposed views as they are (strided
    # GEMM operands), so no transposed copy is made of k, the weighted tiles
    # or the (B, H, N, d, d) state stack
    A = torch.where(causal, torch.matmul(qf, kf.transpose(-1, -2)) * bt.unsqueeze(-2), 0.0)
    Kw = torch.matmul((kf * w.unsqueeze(-1)).transpose(-1, -2), kf)
    Uv = torch.matmul((vf * w.unsqueeze(-1)).transpose(-1, -2), kf)
    Qt = qf - torch.matmul(A, kf)
    Ov = torch.matmul(A, vf)
    S_all = hip_state_scan(Uv, Kw, a, b, m, n, rule, ns, precision)
    o = torch.matmul(Qt, S_all.transpose(-1, -2)) + Ov
    return o.reshape(B, H, T, d).to(q.dtype)


def chunk_scan(q, k, v, beta, g, gmu=None, gnu=None, *, rule="delta", ns: int = 3, eps: float = 1e-6):
    """Fused mixer core; see the module docstring."""
    r = _rule_id(rule)
    gmu = gmu if r >= 1 else None
    gnu = gnu if r == 2 else None
    _check(q, k, v, beta, g, gmu, gnu, r)
    # the state checkpoint is written only when a backward can follow
    record = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, beta, g, gmu, gnu))
    if record and not fused_backward(r, q.shape[-1]):
        if eps != 1e-6:
            raise RuntimeError("adam at d = 128 trains through the drop-in scan, whose epsilon is 1e-6 "
                               f"(fast_scan.py:94); got eps={eps}")
        return _composed_core(q, k, v, beta, g, gmu, gnu, r, ns, precision="ieee")
    gates = [None if t is None else t.to(torch.float32) for t in (beta, g, gmu, gnu)]
    o, _ = torch.ops.gmdn.chunk_fwd(q, k, v, *gates, r, ns, eps, record)
    return o
