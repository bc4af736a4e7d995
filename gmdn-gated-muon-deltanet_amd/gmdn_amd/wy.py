"""Exact WY/UT mode: the token-exact gated delta rule, chunked by the WY/UT
transform (the reference leaves this mode out and trains the chunk-frozen
E-form, train_ablation.py:12-18).

``wy_scan(q, k, v, beta, g)`` returns o (B, H, T, d) of

    S_t = alpha_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T,   o_t = S_t q_t,
    alpha_t = exp(max(g_t, log 1e-6)),

for bfloat16 q, k, v (B, H, T, d) (d = 64 or 128, T a multiple of 64) and
float32 beta, g (B, H, T).  The inference forward is the HIP path of
``gmdn_wy_fwd``: a chunk-parallel prep kernel (decay masks, the triangular
inverse T = (I + A)^-1 and the products that reduce each chunk to the
affine state update S' = a S + U_A - S K_A and the output o = Qt S^T + Ov,
all in exact float32 MFMA), the drop-in delta scan kernels, and an output
kernel.  A call that needs gradients runs the same chunk algebra as float32
tensor operations (``wy_chunk_terms``) around the drop-in delta scan's
operator, whose backward is the HIP reverse scan; autograd differentiates
the rest.
"""
from __future__ import annotations

import math

import torch

from . import _native as nat
from . import ops  # noqa: F401  -- registers torch.ops.gmdn.*
from .scan import hip_state_scan

CHUNK = 64
LOG_FLOOR = math.log(1e-6)


@torch.library.custom_op("gmdn::wy_fwd", mutates_args=(), device_types="cuda")
def wy_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    lib = nat.load()
    ops._check_tokens(q, k, v)
    qc, kc, vc = ops._tok(q), ops._tok(k), ops._tok(v)
    bc, gc = ops._gate(beta), ops._gate(g)
    o = torch.empty_strided(q.shape, ops._kernel_strides(q), dtype=q.dtype, device=q.device)
    desc = ops.chunk_desc(qc, kc, vc, o, 0, 0, 1e-6)
    ws = torch.empty(max(lib.gmdn_wy_fwd_workspace_bytes(desc), 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        rc = lib.gmdn_wy_fwd(desc, nat.ptr(qc), nat.ptr(kc), nat.ptr(vc), nat.ptr(bc), nat.ptr(gc), nat.ptr(o),
                             nat.ptr(ws), ws.numel(), nat.stream_of(q))
    nat.check(rc, "gmdn_wy_fwd")
    return o


@wy_fwd.register_fake
def _wy_fwd_fake(q, k, v, beta, g):
    return q.new_empty_strided(q.shape, ops._kernel_strides(q))


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


def _composed(q, k, v, beta, g):
    B, H, T, d = q.shape
    a, UA, KA, Qt, Ov = wy_chunk_terms(q, k, v, beta, g)
    ones = torch.ones_like(a)
    S_all = hip_state_scan(UA, KA, a, ones, ones, ones, 0, 0, precision="ieee")
    o = torch.matmul(Qt, S_all.transpose(-1, -2)) + Ov
    return o.reshape(B, H, T, d).to(q.dtype)


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
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, beta, g))
    if grad:
        return _composed(q, k, v, beta, g)
    return torch.ops.gmdn.wy_fwd(q, k, v, beta.float(), g.float())
