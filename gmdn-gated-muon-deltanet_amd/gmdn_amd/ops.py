"""``torch.ops.gmdn.*``: the C-ABI entry points as registered torch operators.

Each operator wraps one call of ``libgmdn_scan.so`` (include/gmdn_scan.h) on
the tensors' current stream, with a shape-only fake implementation so that
``torch.compile`` traces through the scan without a graph break (the
reference trainer compiles its model, train_ablation.py:420-422), and with
autograd registered on the forward operators:

* ``gmdn::state_scan(U, K, a, b, m, n, rule, ns, precision, save_moments)
  -> (S_all, M_all, V_all)`` -- the drop-in scan's forward (reference
  ``_TritonScan.forward``, fast_scan.py:360-377).  Inputs are float32 and
  contiguous; ``M_all`` / ``V_all`` are the moment stacks the backward needs
  (empty unless ``save_moments`` and the rule keeps them).
* ``gmdn::state_scan_bwd(...) -> (dU, dK, da, db, dm, dn)`` (reference
  ``_TritonScan.backward``, fast_scan.py:379-396).
* ``gmdn::chunk_fwd(q, k, v, beta, g, gmu, gnu, rule, ns, eps, record)
  -> (o, states)`` -- the fused mixer core (reference train_ablation.py:142-187);
  ``states`` is the library-private state checkpoint (empty unless
  ``record``).
* ``gmdn::chunk_bwd(...) -> (dq, dk, dv, dbeta, dg, dgmu, dgnu)``.
* ``gmdn::front_fwd`` / ``gmdn::front_bwd`` -- the mixer front-end (causal
  depthwise conv, SiLU, q/k norms; train_ablation.py:124-128).
* ``gmdn::gates_fwd`` / ``gmdn::gates_bwd`` -- the gate activations and their
  clamped logs (train_ablation.py:131-134); ``gmdn::head_norm_fwd`` /
  ``gmdn::head_norm_bwd`` -- the per-head RMSNorm of the output (:188).
* ``gmdn::chunk_bwd_muon`` -- the muon core's backward.
* ``gmdn::msign(M, steps, eps) -> X`` -- the outer Muon optimizer's msign of
  a batch of matrices (train_ablation.py:60-73); no autograd (the optimizer
  runs it under ``no_grad``).

Operators cannot return ``None``: absent optional results are empty tensors.
There is no CPU implementation; CPU tensors never reach these operators (the
drop-in dispatcher sends them to its eager path).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _native as nat

CHUNK = 64


def _empty(like: Tensor) -> Tensor:
    return like.new_empty((0,), dtype=torch.float32)


# ------------------------------------------------------------------ Level A
@torch.library.custom_op("gmdn::state_scan", mutates_args=(), device_types="cuda")
def state_scan(U: Tensor, K: Tensor, a: Tensor, b: Tensor, m: Tensor, n: Tensor, rule: int, ns: int,
               precision: int, save_moments: bool) -> tuple[Tensor, Tensor, Tensor]:
    lib = nat.load()
    B, H, N, dh, _ = U.shape
    S_all = torch.empty_like(U)
    M_all = torch.empty_like(U) if (rule != 0 and save_moments) else _empty(U)
    V_all = torch.empty_like(U) if (rule == 2 and save_moments) else _empty(U)
    with torch.cuda.device(U.device):
        rc = lib.gmdn_scan_fwd(
            nat.ptr(U), nat.ptr(K), nat.ptr(a), nat.ptr(b), nat.ptr(m), nat.ptr(n), nat.ptr(S_all),
            nat.ptr(M_all) if M_all.numel() else None, nat.ptr(V_all) if V_all.numel() else None,
            B * H, N, dh, rule, ns, precision, nat.stream_of(U))
    nat.check(rc, "gmdn_scan_fwd")
    return S_all, M_all, V_all


@state_scan.register_fake
def _state_scan_fake(U, K, a, b, m, n, rule, ns, precision, save_moments):
    S_all = torch.empty_like(U)
    M_all = torch.empty_like(U) if (rule != 0 and save_moments) else _empty(U)
    V_all = torch.empty_like(U) if (rule == 2 and save_moments) else _empty(U)
    return S_all, M_all, V_all


@torch.library.custom_op("gmdn::state_scan_bwd", mutates_args=(), device_types="cuda")
def state_scan_bwd(U: Tensor, K: Tensor, a: Tensor, b: Tensor, m: Tensor, n: Tensor, S_all: Tensor,
                   M_all: Tensor, V_all: Tensor, gS: Tensor, rule: int, ns: int,
                   precision: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    lib = nat.load()
    B, H, N, dh, _ = U.shape
    gS = gS.to(torch.float32).contiguous()
    dU, dK = torch.empty_like(U), torch.empty_like(K)
    da, db, dm, dn = (torch.empty_like(a) for _ in range(4))
    ws_bytes = lib.gmdn_scan_bwd_workspace_bytes(B * H, N, dh, rule, ns)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=U.device) if ws_bytes else None
    with torch.cuda.device(U.device):
        rc = lib.gmdn_scan_bwd(
            nat.ptr(U), nat.ptr(K), nat.ptr(a), nat.ptr(b), nat.ptr(m), nat.ptr(n), nat.ptr(S_all),
            nat.ptr(M_all) if M_all.numel() else None, nat.ptr(V_all) if V_all.numel() else None,
            nat.ptr(gS), nat.ptr(dU), nat.ptr(dK), nat.ptr(da), nat.ptr(db), nat.ptr(dm), nat.ptr(dn),
            nat.ptr(ws), ws_bytes, B * H, N, dh, rule, ns, precision, nat.stream_of(U))
    nat.check(rc, "gmdn_scan_bwd")
    return dU, dK, da, db, dm, dn


@state_scan_bwd.register_fake
def _state_scan_bwd_fake(U, K, a, b, m, n, S_all, M_all, V_all, gS, rule, ns, precision):
    return (torch.empty_like(U), torch.empty_like(K), *(torch.empty_like(a) for _ in range(4)))


def _state_scan_setup(ctx, inputs, output):
    U, K, a, b, m, n, rule, ns, precision, save_moments = inputs
    S_all, M_all, V_all = output
    # the moment stacks are saved intermediates: no cotangent is formed for
    # them (materialised zeros would cost a d x d memset per chunk)
    ctx.mark_non_differentiable(M_all, V_all)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(U, K, a, b, m, n, S_all, M_all, V_all)
    ctx.rule, ctx.ns, ctx.precision = rule, ns, precision


def _state_scan_backward(ctx, gS, gM, gV):
    U, K, a, b, m, n, S_all, M_all, V_all = ctx.saved_tensors
    if gS is None:
        gS = torch.zeros_like(S_all)
    grads = torch.ops.gmdn.state_scan_bwd(U, K, a, b, m, n, S_all, M_all, V_all, gS, ctx.rule, ctx.ns,
                                          ctx.precision)
    return (*grads, None, None, None, None)


state_scan.register_autograd(_state_scan_backward, setup_context=_state_scan_setup)


# ------------------------------------------------------------------ Level B
def chunk_desc(q: Tensor, k: Tensor, v: Tensor, o: Tensor, rule: int, ns: int, eps: float,
               precision: int = nat.PREC_TF32):
    """The ``gmdn_chunk_desc`` of a call: sizes, rule and the element strides
    of the (B, H, T, d) token streams (``precision``: rule 1's Newton-Schulz
    VJP in the backward)."""
    B, H, T, d = q.shape
    desc = nat.ChunkDesc()
    desc.B, desc.H, desc.T, desc.d, desc.C = B, H, T, d, CHUNK
    dtype = nat.DTYPE_F32 if q.dtype == torch.float32 else nat.DTYPE_BF16
    desc.rule, desc.ns, desc.dtype, desc.eps = rule, ns, dtype, eps
    desc.precision = precision
    for name, t in (("sq", q), ("sk", k), ("sv", v), ("so", o)):
        arr = getattr(desc, name)
        for i in range(3):
            arr[i] = t.stride(i)
    return desc


def _tok(t: Tensor, dense: bool = False) -> Tensor:
    """Token stream with a unit-stride last dim, B/H/T strides in multiples
    of 8 elements and a 16-byte-aligned base.  ``dense``: also a dense
    permutation -- the backward writes each stream's gradient with the
    stream's own strides, which must then neither alias (expanded views) nor
    leave holes (a slice of a wider tensor)."""
    if (t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16
            or (dense and not _dense_permutation(t))):
        t = t.contiguous()
    return t


def _check_tokens(*ts: Tensor) -> None:
    """The fused core reads and writes bfloat16 or float32 token streams, all
    of one dtype (``chunk_desc`` passes it to the C ABI)."""
    for t in ts:
        if t.dtype not in (torch.bfloat16, torch.float32):
            raise RuntimeError(f"gmdn::chunk_fwd / chunk_bwd take bfloat16 or float32 q, k, v, got {t.dtype}")
        if t.dtype != ts[0].dtype:
            raise RuntimeError(f"q, k, v must share one dtype, got {[x.dtype for x in ts]}")
        if t.dim() != 4:
            raise RuntimeError(f"token streams are (B, H, T, d), got shape {tuple(t.shape)}")


def _gate(t: Optional[Tensor]) -> Optional[Tensor]:
    """float32 (B, H, T) gate stream, contiguous and 16-byte aligned."""
    if t is None:
        return None
    t = t.to(torch.float32).contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _states_numel(q: Tensor, rule: int, ns: int, eps: float) -> int:
    # the checkpoint size depends on the sizes and the rule only
    return nat.load().gmdn_chunk_states_bytes(chunk_desc(q, q, q, q, rule, ns, eps)) // 4


@torch.library.custom_op("gmdn::chunk_fwd", mutates_args=(), device_types="cuda")
def chunk_fwd(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, g: Tensor, gmu: Optional[Tensor],
              gnu: Optional[Tensor], rule: int, ns: int, eps: float, record: bool) -> tuple[Tensor, Tensor]:
    lib = nat.load()
    _check_tokens(q, k, v)
    qc, kc, vc = _tok(q), _tok(k), _tok(v)
    bc, gc, mc, nc = _gate(beta), _gate(g), _gate(gmu), _gate(gnu)
    # o takes q's layout (the mixer's (B, T, H, d) storage, so that the head
    # norm and output projection read it without a transposing copy)
    o = torch.empty_strided(q.shape, _kernel_strides(q), dtype=q.dtype, device=q.device)
    desc = chunk_desc(qc, kc, vc, o, rule, ns, eps)
    keep = _keeps_states(q, rule, record)
    states = (torch.empty(lib.gmdn_chunk_states_bytes(desc) // 4, dtype=torch.float32, device=q.device)
              if keep else _empty(q))
    with torch.cuda.device(q.device):
        rc = lib.gmdn_chunk_fwd(desc, nat.ptr(qc), nat.ptr(kc), nat.ptr(vc), nat.ptr(bc), nat.ptr(gc),
                                nat.ptr(mc), nat.ptr(nc), nat.ptr(o),
                                nat.ptr(states) if keep else None, nat.stream_of(q))
    nat.check(rc, "gmdn_chunk_fwd")
    return o, states


def _keeps_states(q: Tensor, rule: int, record: bool) -> bool:
    """Whether the forward writes the chunk states: for a backward, and always
    where the output kernel reads them (muon; float32 streams, whose matrix
    form runs the drop-in scan between chunk-parallel kernels)."""
    return record or rule == 1 or q.dtype == torch.float32


@chunk_fwd.register_fake
def _chunk_fwd_fake(q, k, v, beta, g, gmu, gnu, rule, ns, eps, record):
    o = q.new_empty_strided(q.shape, _kernel_strides(q))
    keep = _keeps_states(q, rule, record)
    states = q.new_empty((_states_numel(q, rule, ns, eps),), dtype=torch.float32) if keep else _empty(q)
    return o, states


@torch.library.custom_op("gmdn::chunk_bwd", mutates_args=(), device_types="cuda")
def chunk_bwd(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, g: Tensor, gmu: Optional[Tensor],
              gnu: Optional[Tensor], states: Tensor, dO: Tensor, rule: int, ns: int,
              eps: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    return _chunk_bwd_call(q, k, v, beta, g, gmu, gnu, states, dO, rule, ns, eps, nat.PREC_TF32)


def _chunk_bwd_call(q, k, v, beta, g, gmu, gnu, states, dO, rule, ns, eps, precision):
    """gmdn_chunk_bwd: the fused backward of every rule (muon: the drop-in
    scan's Newton-Schulz VJP in ``precision`` between chunk-parallel kernels)."""
    lib = nat.load()
    _check_tokens(q, k, v)
    qc, kc, vc = _tok(q, dense=True), _tok(k, dense=True), _tok(v, dense=True)
    bc, gc, mc, nc = _gate(beta), _gate(g), _gate(gmu), _gate(gnu)
    dOc = _tok(dO.to(q.dtype))
    # the kernels write dq, dk, dv with the strides of q, k, v (dense here)
    dq, dk, dv = (torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=t.device) for t in (qc, kc, vc))
    dbeta, dg = torch.empty_like(bc), torch.empty_like(gc)
    dgmu = torch.empty_like(mc) if mc is not None else _empty(q)
    dgnu = torch.empty_like(nc) if nc is not None else _empty(q)
    desc = chunk_desc(qc, kc, vc, dOc, rule, ns, eps, precision)
    ws_bytes = lib.gmdn_chunk_bwd_workspace_bytes(desc)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    with torch.cuda.device(q.device):
        rc = lib.gmdn_chunk_bwd(desc, nat.ptr(qc), nat.ptr(kc), nat.ptr(vc), nat.ptr(bc), nat.ptr(gc),
                                nat.ptr(mc), nat.ptr(nc), nat.ptr(states), nat.ptr(dOc), nat.ptr(dq),
                                nat.ptr(dk), nat.ptr(dv), nat.ptr(dbeta), nat.ptr(dg),
                                nat.ptr(dgmu) if mc is not None else None,
                                nat.ptr(dgnu) if nc is not None else None,
                                nat.ptr(ws), ws_bytes, nat.stream_of(q))
    nat.check(rc, "gmdn_chunk_bwd")
    # the fake implementation cannot see data pointers: a stream that _tok
    # copied for its alignment or density gets its gradient back in the
    # strides the fake reports
    dq, dk, dv = (_as_strided_like(d_, t) for d_, t in ((dq, q), (dk, k), (dv, v)))
    return dq, dk, dv, dbeta, dg, dgmu, dgnu


def _dense_permutation(t: Tensor) -> bool:
    """Whether ``t``'s elements fill its storage extent exactly once: its
    strides are those of a contiguous tensor with permuted dimensions (no
    zero strides from ``expand``, no gaps as in a slice of a wider tensor)."""
    dims = sorted((st, sz) for st, sz in zip(t.stride(), t.shape) if sz != 1)
    want = 1
    for st, sz in dims:
        if st != want:
            return False
        want *= sz
    return True


def _kernel_strides(t: Tensor):
    """The strides of the output and gradient of token stream ``t``: its own
    when they suit the kernels (unit-stride d, B/H/T strides in multiples of
    8 elements) and ``t`` is a dense permutation (an expanded stream would
    make rows alias, a gapped one would leave holes), else contiguous.  The
    data pointer does not enter, so the real and fake implementations agree."""
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or not _dense_permutation(t):
        return t.new_empty(t.shape).stride()
    return t.stride()


def _as_strided_like(x: Tensor, t: Tensor) -> Tensor:
    """``x`` laid out with ``_kernel_strides(t)`` (a copy only when they differ)."""
    want = _kernel_strides(t)
    if x.stride() == want:
        return x
    return torch.empty_strided(x.shape, want, dtype=x.dtype, device=x.device).copy_(x)


@chunk_bwd.register_fake
def _chunk_bwd_fake(q, k, v, beta, g, gmu, gnu, states, dO, rule, ns, eps):
    dq, dk, dv = (t.new_empty_strided(t.shape, _kernel_strides(t)) for t in (q, k, v))
    dbeta = beta.new_empty(beta.shape, dtype=torch.float32)
    dg = g.new_empty(g.shape, dtype=torch.float32)
    dgmu = gmu.new_empty(gmu.shape, dtype=torch.float32) if gmu is not None else _empty(q)
    dgnu = gnu.new_empty(gnu.shape, dtype=torch.float32) if gnu is not None else _empty(q)
    return dq, dk, dv, dbeta, dg, dgmu, dgnu


def _chunk_fwd_setup(ctx, inputs, output):
    q, k, v, beta, g, gmu, gnu, rule, ns, eps, record = inputs
    o, states = output
    # the checkpoint is a saved intermediate (see _state_scan_setup)
    ctx.mark_non_differentiable(states)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, k, v, beta, g, gmu, gnu, states)
    ctx.rule, ctx.ns, ctx.eps, ctx.record = rule, ns, eps, record


def _chunk_fwd_backward(ctx, dO, dstates):
    q, k, v, beta, g, gmu, gnu, states = ctx.saved_tensors
    if dO is None:
        dO = torch.zeros_like(q)
    if not ctx.record:
        raise RuntimeError("gmdn::chunk_fwd ran without recording its state checkpoint "
                           "(grad mode was off at the call); it has no backward")
    if ctx.rule == 1:
        from .scan import _prec_code
        dq, dk, dv, dbeta, dg, dgmu = torch.ops.gmdn.chunk_bwd_muon(q, k, v, beta, g, gmu, states, dO, ctx.ns,
                                                                    _prec_code())
        return dq, dk, dv, dbeta, dg, dgmu, None, None, None, None, None
    dq, dk, dv, dbeta, dg, dgmu, dgnu = torch.ops.gmdn.chunk_bwd(q, k, v, beta, g, gmu, gnu, states, dO,
                                                                 ctx.rule, ctx.ns, ctx.eps)
    return (dq, dk, dv, dbeta, dg, dgmu if gmu is not None else None, dgnu if gnu is not None else None,
            None, None, None, None)


chunk_fwd.register_autograd(_chunk_fwd_backward, setup_context=_chunk_fwd_setup)


@torch.library.custom_op("gmdn::chunk_bwd_muon", mutates_args=(), device_types="cuda")
def chunk_bwd_muon(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, g: Tensor, gmu: Tensor, states: Tensor,
                   dO: Tensor, ns: int, precision: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of the fused muon core given the forward's chunk states
    (S_i, M_i), all in HIP (``gmdn_chunk_bwd`` with rule 1): the per-chunk
    Kw, Uv and dL/dS_i, the drop-in muon scan's backward (Newton-Schulz VJP
    in ``precision``), then the token gradients."""
    dq, dk, dv, dbeta, dg, dgmu, _ = _chunk_bwd_call(q, k, v, beta, g, gmu, None, states, dO, 1, ns, 1e-6,
                                                     precision)
    return dq, dk, dv, dbeta.to(beta.dtype), dg.to(g.dtype), dgmu.to(gmu.dtype)


@chunk_bwd_muon.register_fake
def _chunk_bwd_muon_fake(q, k, v, beta, g, gmu, states, dO, ns, precision):
    dq, dk, dv = (t.new_empty_strided(t.shape, _kernel_strides(t)) for t in (q, k, v))
    return dq, dk, dv, beta.new_empty(beta.shape), g.new_empty(g.shape), gmu.new_empty(gmu.shape)


# ------------------------------------------------------- mixer front-end
def _dtype_code(t: Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return nat.DTYPE_BF16
    if t.dtype == torch.float32:
        return nat.DTYPE_F32
    raise RuntimeError(f"the mixer front-end kernels take bfloat16 or float32, got {t.dtype}")


@torch.library.custom_op("gmdn::front_fwd", mutates_args=(), device_types="cuda")
def front_fwd(y: Tensor, weight: Tensor, bias: Tensor, dh: int) -> tuple[Tensor, Tensor, Tensor]:
    """q, k, v (B, T, D) from the qkv projection output y (B, T, 3 D):
    causal depthwise conv (weight (3 D, 1, K), bias), SiLU, per-head L2 norm
    of q and k (reference train_ablation.py:124-128)."""
    lib = nat.load()
    B, T, C3 = y.shape
    D, K = C3 // 3, weight.shape[-1]
    yc = y.contiguous()
    w = weight.reshape(C3, K).to(torch.float32).contiguous()
    bc = bias.to(torch.float32).contiguous()
    q, k, v = (torch.empty(B, T, D, dtype=y.dtype, device=y.device) for _ in range(3))
    with torch.cuda.device(y.device):
        rc = lib.gmdn_front_fwd(nat.ptr(yc), nat.ptr(w), nat.ptr(bc), nat.ptr(q), nat.ptr(k), nat.ptr(v), B, T, D,
                                dh, K, _dtype_code(y), nat.stream_of(y))
    nat.check(rc, "gmdn_front_fwd")
    return q, k, v


@front_fwd.register_fake
def _front_fwd_fake(y, weight, bias, dh):
    B, T, C3 = y.shape
    return tuple(y.new_empty(B, T, C3 // 3) for _ in range(3))


@torch.library.custom_op("gmdn::front_bwd", mutates_args=(), device_types="cuda")
def front_bwd(y: Tensor, weight: Tensor, bias: Tensor, dq: Tensor, dk: Tensor, dv: Tensor,
              dh: int) -> tuple[Tensor, Tensor, Tensor]:
    """dy, dweight, dbias of ``front_fwd`` given the cotangents of q, k, v."""
    lib = nat.load()
    B, T, C3 = y.shape
    D, K = C3 // 3, weight.shape[-1]
    yc = y.contiguous()
    w = weight.reshape(C3, K).to(torch.float32).contiguous()
    bc = bias.to(torch.float32).contiguous()
    g = [t.to(y.dtype).contiguous() for t in (dq, dk, dv)]
    dy = torch.empty_like(yc)
    partial = torch.empty(lib.gmdn_front_bwd_workspace_floats(B, T, D, K), dtype=torch.float32, device=y.device)
    with torch.cuda.device(y.device):
        rc = lib.gmdn_front_bwd(nat.ptr(yc), nat.ptr(w), nat.ptr(bc), *(nat.ptr(t) for t in g), nat.ptr(dy),
                                nat.ptr(partial), B, T, D, dh, K, _dtype_code(y), nat.stream_of(y))
    nat.check(rc, "gmdn_front_bwd")
    sums = partial.view(-1, C3, K + 1).sum(0)
    return dy, sums[:, :K].reshape(weight.shape).to(weight.dtype), sums[:, K].to(bias.dtype).contiguous()


@front_bwd.register_fake
def _front_bwd_fake(y, weight, bias, dq, dk, dv, dh):
    return y.new_empty(y.shape), torch.empty_like(weight), torch.empty_like(bias)


def _front_setup(ctx, inputs, output):
    y, weight, bias, dh = inputs
    ctx.save_for_backward(y, weight, bias)
    ctx.dh = dh


def _front_backward(ctx, dq, dk, dv):
    y, weight, bias = ctx.saved_tensors
    dq, dk, dv = (torch.zeros_like(t) if g is None else g for g, t in zip((dq, dk, dv), (y, y, y)))
    dy, dw, db = torch.ops.gmdn.front_bwd(y, weight, bias, dq, dk, dv, ctx.dh)
    return dy, dw, db, None


front_fwd.register_autograd(_front_backward, setup_context=_front_setup)


# ------------------------------------------------ gates and head norm
@torch.library.custom_op("gmdn::gates_fwd", mutates_args=(), device_types="cuda")
def gates_fwd(y: Tensor, heads: int, n_gates: int) -> Tensor:
    """(n_gates, B, H, T) float32 from the gate projection y (B, T, n_gates H):
    sigmoid for gate 1 (beta), log sigmoid clamped at log 1e-6 for the others
    (reference train_ablation.py:131-134, :155, :169-175)."""
    lib = nat.load()
    B, T, C = y.shape
    yc = y.contiguous()
    out = torch.empty(n_gates, B, heads, T, dtype=torch.float32, device=y.device)
    with torch.cuda.device(y.device):
        rc = lib.gmdn_gates_fwd(nat.ptr(yc), nat.ptr(out), B, T, heads, n_gates, _dtype_code(yc), nat.stream_of(y))
    nat.check(rc, "gmdn_gates_fwd")
    return out


@gates_fwd.register_fake
def _gates_fwd_fake(y, heads, n_gates):
    B, T, C = y.shape
    return y.new_empty((n_gates, B, heads, T), dtype=torch.float32)


@torch.library.custom_op("gmdn::gates_bwd", mutates_args=(), device_types="cuda")
def gates_bwd(y: Tensor, dout: Tensor, heads: int, n_gates: int) -> Tensor:
    lib = nat.load()
    B, T, C = y.shape
    yc = y.contiguous()
    dc = dout.to(torch.float32).contiguous()
    dy = torch.empty_like(yc)
    with torch.cuda.device(y.device):
        rc = lib.gmdn_gates_bwd(nat.ptr(yc), nat.ptr(dc), nat.ptr(dy), B, T, heads, n_gates, _dtype_code(yc),
                                nat.stream_of(y))
    nat.check(rc, "gmdn_gates_bwd")
    return dy


@gates_bwd.register_fake
def _gates_bwd_fake(y, dout, heads, n_gates):
    return torch.empty_like(y, memory_format=torch.contiguous_format)


def _gates_setup(ctx, inputs, output):
    y, heads, n_gates = inputs
    ctx.save_for_backward(y)
    ctx.heads, ctx.n_gates = heads, n_gates


def _gates_backward(ctx, dout):
    (y,) = ctx.saved_tensors
    return torch.ops.gmdn.gates_bwd(y, dout, ctx.heads, ctx.n_gates), None, None


gates_fwd.register_autograd(_gates_backward, setup_context=_gates_setup)


@torch.library.custom_op("gmdn::head_norm_fwd", mutates_args=(), device_types="cuda")
def head_norm_fwd(x: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """RMSNorm of every row of d elements of x (..., d) with a float32 weight
    (d): the mixer's per-head output norm (train_ablation.py:188).  Returns
    the output (x's dtype and shape, contiguous) and 1 / rms per row."""
    lib = nat.load()
    d = x.shape[-1]
    xc = x.contiguous()
    rows = xc.numel() // d if d else 0
    out = torch.empty_like(xc)
    rstd = torch.empty(xc.shape[:-1], dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.gmdn_head_norm_fwd(nat.ptr(xc), nat.ptr(weight.contiguous()), nat.ptr(out), nat.ptr(rstd), rows, d,
                                    eps, _dtype_code(xc), nat.stream_of(x))
    nat.check(rc, "gmdn_head_norm_fwd")
    return out, rstd


@head_norm_fwd.register_fake
def _head_norm_fwd_fake(x, weight, eps):
    return (torch.empty_like(x, memory_format=torch.contiguous_format),
            x.new_empty(x.shape[:-1], dtype=torch.float32))


@torch.library.custom_op("gmdn::head_norm_bwd", mutates_args=(), device_types="cuda")
def head_norm_bwd(x: Tensor, weight: Tensor, rstd: Tensor, dout: Tensor) -> tuple[Tensor, Tensor]:
    lib = nat.load()
    d = x.shape[-1]
    xc = x.contiguous()
    rows = xc.numel() // d
    dc = dout.to(x.dtype).contiguous()
    dx = torch.empty_like(xc)
    dw = torch.empty(d, dtype=torch.float32, device=x.device)
    ws = torch.empty(max(lib.gmdn_head_norm_bwd_workspace_floats(rows, d), 1), dtype=torch.float32,
                     device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.gmdn_head_norm_bwd(nat.ptr(xc), nat.ptr(weight.contiguous()), nat.ptr(rstd.contiguous()),
                                    nat.ptr(dc), nat.ptr(dx), nat.ptr(dw), nat.ptr(ws), ws.numel(), rows, d,
                                    _dtype_code(xc), nat.stream_of(x))
    nat.check(rc, "gmdn_head_norm_bwd")
    return dx, dw


@head_norm_bwd.register_fake
def _head_norm_bwd_fake(x, weight, rstd, dout):
    return torch.empty_like(x, memory_format=torch.contiguous_format), weight.new_empty(weight.shape)


def _head_norm_setup(ctx, inputs, output):
    x, weight, eps = inputs
    out, rstd = output
    ctx.mark_non_differentiable(rstd)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, weight, rstd)


def _head_norm_backward(ctx, dout, drstd):
    x, weight, rstd = ctx.saved_tensors
    if dout is None:
        return None, None, None
    dx, dw = torch.ops.gmdn.head_norm_bwd(x, weight, rstd, dout)
    return dx, dw, None


head_norm_fwd.register_autograd(_head_norm_backward, setup_context=_head_norm_setup)


# ------------------------------------------------------------ outer msign
@torch.library.custom_op("gmdn::msign", mutates_args=(), device_types="cuda")
def msign(M: Tensor, steps: int, eps: float) -> Tensor:
    """msign of each matrix of ``M`` (..., rows, cols), float32 or bfloat16,
    result in ``M``'s dtype (reference train_ablation.py:60-73)."""
    lib = nat.load()
    if M.dim() < 2:
        raise RuntimeError(f"msign needs a matrix or a batch of matrices, got shape {tuple(M.shape)}")
    if M.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"gmdn::msign takes float32 or bfloat16, got {M.dtype}")
    rows, cols = M.shape[-2], M.shape[-1]
    Mc = M.contiguous()
    out = torch.empty_like(Mc)
    batch = Mc.numel() // max(rows * cols, 1) if rows * cols else 0
    if batch == 0:
        return out
    ws = torch.empty(lib.gmdn_msign_workspace_bytes(batch, rows, cols), dtype=torch.uint8, device=M.device)
    with torch.cuda.device(M.device):
        rc = lib.gmdn_msign(nat.ptr(Mc), nat.ptr(out), batch, rows, cols, steps, eps, _dtype_code(Mc), nat.ptr(ws),
                            ws.numel(), nat.stream_of(Mc))
    nat.check(rc, "gmdn_msign")
    return out


@msign.register_fake
def _msign_fake(M, steps, eps):
    return torch.empty_like(M, memory_format=torch.contiguous_format)
