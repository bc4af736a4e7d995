"""Exact WY/UT mode: the token-exact gated delta rule, chunked by the WY/UT
transform (the reference leaves this mode out and trains the chunk-frozen
E-form, train_ablation.py:12-18).

``wy_scan(q, k, v, beta, g)`` returns o (B, H, T, d) of

    S_t = alpha_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T,   o_t = S_t q_t,
    alpha_t = exp(max(g_t, log 1e-6)),

for bfloat16 q, k, v (B, H, T, d) (d = 64 or 128, T a multiple of 64) and
float32 beta, g (B, H, T).  Forward and backward are HIP:

* forward (``gmdn_wy_fwd``): a chunk-parallel prep kernel (decay masks, the
  triangular inverse T = (I + A)^-1 by float32 forward substitution, and
  the products that reduce each chunk to the affine state update
  S' = a S + U_A - S K_A and the output o = Qt S^T + Ov), the drop-in delta
  scan kernels and an output kernel.  Its workspace is the backward's
  checkpoint.
* backward (``gmdn_wy_bwd``): dL/dS_i through o, the drop-in delta scan's
  reverse kernel for the state cotangents, then chunk-parallel kernels that
  differentiate the chunk algebra (T, U, W, the decay masks) back to q, k,
  v, beta and g.

Every product is split-bf16 MFMA: bf16 q, k, v enter exactly, float32
operands as hi + lo bf16 (about 2^-16 relative error per product).

``wy_chunk_terms`` restates the chunk algebra as float32 tensor operations;
it documents the prep kernel's quantities and is checked on the CPU against
the oracle's token recurrence.
"""
from __future__ import annotations

import math

import torch

from . import _native as nat
from . import ops  # noqa: F401  -- registers torch.ops.gmdn.*

CHUNK = 64
LOG_FLOOR = math.log(1e-6)


def _ckpt_numel(q):
    desc = ops.chunk_desc(q, q, q, q, 0, 0, 1e-6)
    return max(nat.load().gmdn_wy_fwd_workspace_bytes(desc) // 4, 4)


@torch.library.custom_op("gmdn::wy_fwd", mutates_args=(), device_types="cuda")
def wy_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, g: torch.Tensor,
           record: bool) -> tuple[torch.Tensor, torch.Tensor]:
    lib = nat.load()
    ops._check_tokens(q, k, v)
    qc, kc, vc = ops._tok(q), ops._tok(k), ops._tok(v)
    bc, gc = ops._gate(beta), ops._gate(g)
    o = torch.empty_strided(q.shape, ops._kernel_strides(q), dtype=q.dtype, device=q.device)
    desc = ops.chunk_desc(qc, kc, vc, o, 0, 0, 1e-6)
    # the forward's workspace is the backward's checkpoint
    ws = torch.empty(_ckpt_numel(q), dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        rc = lib.gmdn_wy_fwd(desc, nat.ptr(qc), nat.ptr(kc), nat.ptr(vc), nat.ptr(bc), nat.ptr(gc), nat.ptr(o),
                             nat.ptr(ws), ws.numel() * 4, nat.stream_of(q))
    nat.check(rc, "gmdn_wy_fwd")
    return o, (ws if record else ops._empty(q))


@wy_fwd.register_fake
def _wy_fwd_fake(q, k, v, beta, g, record):
    o = q.new_empty_strided(q.shape, ops._kernel_strides(q))
    return o, (q.new_empty((_ckpt_numel(q),), dtype=torch.float32) if record else ops._empty(q))


@torch.library.custom_op("gmdn::wy_bwd", mutates_args=(), device_types="cuda")
def wy_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, g: torch.Tensor,
           ckpt: torch.Tensor, dO: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                                          torch.Tensor]:
    lib = nat.load()
    ops._check_tokens(q, k, v)
    qc, kc, vc = ops._tok(q, dense=True), ops._tok(k, dense=True), ops._tok(v, dense=True)
    bc, gc = ops._gate(beta), ops._gate(g)
    dOc = ops._tok(dO.to(q.dtype))
    dq, dk, dv = (torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=t.device) for t in (qc, kc, vc))
    dbeta, dg = torch.empty_like(bc), torch.empty_like(gc)
    desc = ops.chunk_desc(qc, kc, vc, dOc, 0, 0, 1e-6)
    ws = torch.empty(max(lib.gmdn_wy_bwd_workspace_bytes(desc), 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        rc = lib.gmdn_wy_bwd(desc, nat.ptr(qc), nat.ptr(kc), nat.ptr(vc), nat.ptr(bc), nat.ptr(gc), nat.ptr(ckpt),
                             nat.ptr(dOc), nat.ptr(dq), nat.ptr(dk), nat.ptr(dv), nat.ptr(dbeta), nat.ptr(dg),
                             nat.ptr(ws), ws.numel(), nat.stream_of(q))
    nat.check(rc, "gmdn_wy_bwd")
    dq, dk, dv = (ops._as_strided_like(d_, t) for d_, t in ((dq, q), (dk, k), (dv, v)))
    return dq, dk, dv, dbeta, dg


@wy_bwd.register_fake
def _wy_bwd_fake(q, k, v, beta, g, ckpt, dO):
    dq, dk, dv = (t.new_empty_strided(t.shape, ops._kernel_strides(t)) for t in (q, k, v))
    return (dq, dk, dv, beta.new_empty(beta.shape, dtype=torch.float32),
            g.new_empty(g.shape, dtype=torch.float32))


def _wy_setup(ctx, inputs, output):
    q, k, v, beta, g, record = inputs
    o, ckpt = output
    ctx.mark_non_differentiable(ckpt)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, k, v, beta, g, ckpt)
    ctx.record = record


def _wy_backward(ctx, dO, dckpt):
    q, k, v, beta, g, ckpt = ctx.saved_tensors
    if not ctx.record:
        raise RuntimeError("gmdn::wy_fwd ran without its checkpoint (grad mode was off at the call); "
                           "it has no backward")
    if dO is None:
        dO = torch.zeros_like(q)
    dq, dk, dv, dbeta, dg = torch.ops.gmdn.wy_bwd(q, k, v, beta, g, ckpt, dO)
    return dq, dk, dv, dbeta.to(beta.dtype), dg.to(g.dtype), None


wy_fwd.register_autograd(_wy_backward, setup_context=_wy_setup)


def wy_chunk_terms(q, k, v, beta, g):
    """Per chunk, in float32: a (B, H, N), U_A, K_A (B, H, N, d, d), Qt, Ov
    (B, H, N, C, d) -- the quantities the prep kernel forms."""
    B, H, T, d = q.shape
    N, C = T // CHUNK, CHUNK
    Q, K, V = (t.float().reshape(B, H, N, C, d) for t in (q, k, v))
    bt = beta.float().reshape(B, H, N, C)
    gcum = torch.cumsum(torch.clamp(g.float(), min=LOG_FLOOR).reshape(B, H, N, C), -1)
    gam = torch.exp(gcum)
    strict = torch.ones(C, C, dtype=torch.bool, device=q.device).tril(-1)
    incl = torch.ones(C, C, dtype=torch.bool, device=q.device).tril()
    # Gamma[t, s] = gamma_t / gamma_s on the causal entries; the exponent is
    # masked before exp, so the (unused) upper triangle is exp(-inf) = 0 and
    # never overflows (an inf there would turn where()'s backward into NaN)
    Gam = torch.exp(torch.where(incl, gcum.unsqueeze(-1) - gcum.unsqueeze(-2), float("-inf")))
    A = torch.where(strict, bt.unsqueeze(-1) * torch.matmul(K, K.transpose(-1, -2)) * Gam, 0.0)
    eye = torch.eye(C, dtype=torch.float32, device=q.device)
    T_ = torch.linalg.solve_triangular(eye + A, eye.expand_as(A), upper=False, unitriangular=True)
    M = torch.where(incl, torch.matmul(Q, K.transpose(-1, -2)) * Gam, 0.0)
    MT = torch.matmul(M, T_)
    kd = torch.exp(gcum[..., -1:] - gcum)
    P = torch.matmul((T_ * kd.unsqueeze(-1)).transpose(-1, -2), K)
    UA = torch.matmul((V * bt.unsqueeze(-1)).transpose(-1, -2), P)
    KA = torch.matmul((K * (bt * gam).unsqueeze(-1)).transpose(-1, -2), P)
    Qt = gam.unsqueeze(-1) * Q - torch.matmul(MT * (bt * gam).unsqueeze(-2), K)
    Ov = torch.matmul(MT * bt.unsqueeze(-2), V)
    return gam[..., -1], UA, KA, Qt, Ov


def wy_scan(q, k, v, beta, g):
    """o of the token-exact gated delta rule; see the module docstring."""
    if not q.is_cuda:
        raise RuntimeError("wy_scan needs GPU tensors")
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise RuntimeError(f"q, k, v must be (B, H, T, d) of equal shape, got {tuple(q.shape)}")
    B, H, T, d = q.shape
    if d not in (64, 128) or T % CHUNK:
        raise RuntimeError(f"wy_scan supports d in (64, 128) and T a multiple of {CHUNK}, got d={d}, T={T}")
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise RuntimeError("wy_scan takes bfloat16 q, k, v")
    for name, t in (("beta", beta), ("g", g)):
        if tuple(t.shape) != (B, H, T):
            raise RuntimeError(f"{name} must be (B, H, T) = {(B, H, T)}, got {tuple(t.shape)}")
    record = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, beta, g))
    o, _ = torch.ops.gmdn.wy_fwd(q, k, v, beta.float(), g.float(), record)
    return o
