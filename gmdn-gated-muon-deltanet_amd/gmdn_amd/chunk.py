"""Fused mixer-core op (Level B): phases 1-3 of the reference mixer in one
HIP kernel per direction.

``chunk_scan(q, k, v, beta, g, gmu=None, gnu=None, rule='delta', ns=3)``
computes what ``FastWeightMixer.forward`` computes between its front-end and
its per-head RMSNorm (reference train_ablation.py:142-187): the chunk
transform A, Kw, Uv, Qt, Ov, the state scan, and ``o = Qt S^T + Ov``.

* ``q, k, v``: (B, H, T, d) bfloat16 or float32 (one dtype for all three),
  d contiguous (any strides over B, H, T that are multiples of 8 elements),
  q and k L2-normalised per head.  Head dims: 64 and 128 in bfloat16 (16
  and 32 are zero-padded to 64), 32, 64 and 128 in float32 (16 is padded to
  32).  Zero columns of q, k, v leave every rule's result unchanged in the
  other columns: the padded rows and columns of S, M and V stay zero
  (msign of a block-diagonal matrix with a zero block keeps the block zero
  and has the same Frobenius norm; adam's update is 0 / (0 + eps) there).
* ``beta``: (B, H, T) beta gate (sigmoid output).
* ``g, gmu, gnu``: (B, H, T) log alpha, log mu, log nu gates.  The reference
  clamps each gate at 1e-6 before its log (train_ablation.py:155, :170-175);
  the kernel clamps the log at log(1e-6), which is the same function.
  ``gmu`` is needed by the muon and adam rules, ``gnu`` by adam.
* returns ``o`` (B, H, T, d) in q's dtype.

Chunk length 64 (the reference default and every configuration's) runs the
fused kernels below.  Other chunk lengths (the reference trainer's
``--chunk``, train_ablation.py:555) run the reference's own schedule: phases
1 and 3 as float32 library GEMMs over all chunks at once and phase 2 as the
drop-in HIP scan (``hip_state_scan``, the precision ``set_precision``
selects), with autograd through both.

Float32 streams (the reference's precision when autocast is off, its CPU
path, train_ablation.py:424, 465) run the reference's matrix form with exact
float32 products: chunk-parallel HIP kernels form Kw, Uv and the chunk
scalars, the drop-in scan's kernels run every rule in 'ieee', and
chunk-parallel kernels form o and, backward, dL/dS_i and the token and gate
gradients.

Delta and adam run as one fused HIP kernel per direction (forward: the
chunk transform, the scan and the output; backward: a reverse scan of the
state cotangent and a chunk-parallel token-gradient kernel).  Muon's msign
couples the whole state: its forward is a serial HIP kernel per (b, h) that
streams the k, v tiles and forms each chunk's update in the E-form before
the Newton-Schulz steps, plus a chunk-parallel output kernel; its backward
is HIP too: a chunk-parallel kernel forms each chunk's Kw, Uv and dL/dS_i,
the drop-in muon scan's backward kernels run the Newton-Schulz VJP, and the
token-gradient kernel finishes in the E-form.  Adam at d = 128 trains with
its scan in exact float32: a chunk-parallel kernel forms Kw, Uv, the drop-in
adam scan kernels run forward and backward, the output and token-gradient
kernels work from the float32 states (its inference forward stays fused).
"""
from __future__ import annotations

import math

import torch

from . import ops  # noqa: F401  -- registers torch.ops.gmdn.*

RULES = {"delta": 0, "muon": 1, "adam": 2}
CHUNK = 64
LOG_FLOOR = math.log(1e-6)
SUPPORTED_D = (64, 128)          # bfloat16 head dims with kernels
SUPPORTED_D_F32 = (32, 64, 128)  # float32 head dims with kernels
PADDED_D = {torch.bfloat16: {16: 64, 32: 64}, torch.float32: {16: 32}}


BWD_RULES = (0, 1, 2)  # rules with a backward


def backward_supported(rule, d: int = 128) -> bool:
    """Whether ``rule`` at head dim ``d`` has a backward: every rule and head
    dim.  (Adam at d = 128 trains with its scan in exact float32: at that head
    dim its sign-like update amplifies the rounding of split-bf16 state
    products past the gradient tolerance.)"""
    return _rule_id(rule) in BWD_RULES


def fused_backward(rule, d: int, dtype=torch.bfloat16) -> bool:
    """Whether ``rule`` at head dim ``d`` trains through the fused op
    ``gmdn::chunk_fwd`` and its HIP backward: every rule and head dim the
    kernels are built for (padded head dims go through a padded call)."""
    _rule_id(rule)
    return d in (SUPPORTED_D_F32 if dtype == torch.float32 else SUPPORTED_D)


def _rule_id(rule) -> int:
    if isinstance(rule, str):
        if rule not in RULES:
            raise ValueError(f"rule must be one of {tuple(RULES)}, got {rule!r}")
        return RULES[rule]
    if rule not in (0, 1, 2):
        raise ValueError(f"rule must be 0, 1 or 2, got {rule}")
    return int(rule)


def _check(q, k, v, beta, g, gmu, gnu, rule, chunk=CHUNK):
    if not q.is_cuda:
        raise RuntimeError("chunk_scan needs GPU tensors")
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise RuntimeError(f"q, k, v must be (B, H, T, d) of equal shape, got {tuple(q.shape)}, "
                           f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, H, T, d = q.shape
    if q.dtype not in (torch.bfloat16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise RuntimeError(f"chunk_scan takes bfloat16 or float32 q, k, v of one dtype, got "
                           f"{q.dtype}, {k.dtype}, {v.dtype}")
    built = SUPPORTED_D_F32 if q.dtype == torch.float32 else SUPPORTED_D
    if chunk != CHUNK:
        from .scan import SUPPORTED_DH
        if d not in SUPPORTED_DH:
            raise RuntimeError(f"chunk lengths other than {CHUNK} run the drop-in scan, which supports head "
                               f"dims {SUPPORTED_DH}, got {d}")
    elif d not in built and d not in PADDED_D[q.dtype]:
        raise RuntimeError(f"chunk_scan supports head dims {tuple(sorted(built + tuple(PADDED_D[q.dtype])))} "
                           f"for {q.dtype}, got {d}")
    if chunk < 1 or T % chunk:
        raise RuntimeError(f"T must be a multiple of the chunk length {chunk}, got {T}")
    for name, t in (("beta", beta), ("g", g), ("gmu", gmu), ("gnu", gnu)):
        if t is not None and tuple(t.shape) != (B, H, T):
            raise RuntimeError(f"{name} must be (B, H, T) = {(B, H, T)}, got {tuple(t.shape)}")
    if rule >= 1 and gmu is None:
        raise RuntimeError("muon and adam rules need gmu")
    if rule == 2 and gnu is None:
        raise RuntimeError("adam rule needs gnu")


def _matrix_form(q, k, v, beta, g, gmu, gnu, rule: int, ns: int, C: int):
    """Phases 1-3 of the reference mixer at chunk length C, its own schedule
    (train_ablation.py:142-187): the chunk transform and the output as float32
    GEMMs batched over every chunk, the state scan through the drop-in HIP
    scan.  Gate floors as the fused kernels apply them (log 1e-6)."""
    from .scan import hip_state_scan
    B, H, T, d = q.shape
    N = T // C
    f = torch.float32
    qn, kn, vn = (t.to(f).reshape(B, H, N, C, d) for t in (q, k, v))
    bn = beta.to(f).reshape(B, H, N, C)

    def logs(t):
        return t.to(f).clamp_min(LOG_FLOOR).reshape(B, H, N, C)

    if rule == 0:
        w = bn
    elif rule == 1:
        lm = logs(gmu)
        # w_t = mu_{t+1} ... mu_C, the residual momentum decay to the chunk end
        w = torch.exp(torch.flip(torch.cumsum(torch.flip(lm, [-1]), -1), [-1]) - lm)
    else:
        w = torch.ones_like(bn)
    causal = torch.tril(torch.ones(C, C, device=q.device, dtype=torch.bool))
    A = torch.matmul(qn, kn.transpose(-1, -2).contiguous()) * bn.unsqueeze(-2)
    A = A.masked_fill(~causal, 0.0)
    Kw = torch.matmul((kn * w.unsqueeze(-1)).transpose(-1, -2).contiguous(), kn)
    Uv = torch.matmul((vn * w.unsqueeze(-1)).transpose(-1, -2).contiguous(), kn)
    Qt = qn - torch.matmul(A, kn)
    Ov = torch.matmul(A, vn)
    a_c = torch.exp(logs(g).sum(-1))
    b_c = bn.mean(-1)
    m_c = torch.exp(logs(gmu).sum(-1)) if gmu is not None else torch.ones_like(a_c)
    n_c = torch.exp(logs(gnu).sum(-1)) if gnu is not None else torch.ones_like(a_c)
    S = hip_state_scan(Uv, Kw, a_c, b_c, m_c, n_c, rule, ns)
    o = torch.matmul(Qt, S.transpose(-1, -2).contiguous()) + Ov
    return o.reshape(B, H, T, d).to(q.dtype)


def chunk_scan(q, k, v, beta, g, gmu=None, gnu=None, *, rule="delta", ns: int = 3, eps: float = 1e-6,
               chunk: int = CHUNK):
    """Fused mixer core; see the module docstring."""
    r = _rule_id(rule)
    gmu = gmu if r >= 1 else None
    gnu = gnu if r == 2 else None
    _check(q, k, v, beta, g, gmu, gnu, r, chunk)
    if chunk != CHUNK:
        if r == 2 and eps != 1e-6:
            raise RuntimeError(f"the drop-in adam scan's epsilon is 1e-6 (fast_scan.py:94), got eps={eps}")
        return _matrix_form(q, k, v, beta, g, gmu, gnu, r, ns, chunk)
    # the state checkpoint is written only when a backward can follow
    record = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, beta, g, gmu, gnu))
    d = q.shape[-1]
    dp = PADDED_D[q.dtype].get(d, d)
    f32 = q.dtype == torch.float32
    if r == 2 and eps != 1e-6 and (f32 or (record and dp == 128)):
        raise RuntimeError("adam runs through the drop-in scan here (float32 streams; bfloat16 training at "
                           f"d = 128), whose epsilon is 1e-6 (fast_scan.py:94); got eps={eps}")
    gates = [None if t is None else t.to(torch.float32) for t in (beta, g, gmu, gnu)]
    if dp != d:
        q, k, v = (torch.nn.functional.pad(t, (0, dp - d)) for t in (q, k, v))
    o, _ = torch.ops.gmdn.chunk_fwd(q, k, v, *gates, r, ns, eps, record)
    return o if dp == d else o[..., :d]
