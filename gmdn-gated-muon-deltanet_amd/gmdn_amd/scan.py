"""Autograd op of the drop-in chunk state scan (Level A).

``HipScan.apply(U, K, a, b, m, n, rule, ns)`` has the signature and
semantics of the reference's ``_TritonScan`` (fast_scan.py:334-396): U, K are
(B, H, N, dh, dh), a, b, m, n are (B, H, N); the result is the stack of
pre-update states S_0..S_{N-1}, and the backward returns gradients for the
six tensor inputs (``None`` for rule and ns).  Both directions run the HIP
kernels of ``libgmdn_scan.so`` on the tensors' current stream.
"""
from __future__ import annotations

import torch

from . import _native as nat

SUPPORTED_DH = (32, 64, 128)
_state = {"precision": "tf32"}


def set_precision(name: str) -> None:
    """'tf32' (bf16x3 split MFMA on gfx950) or 'ieee' (fp32 MFMA)."""
    if name not in ("tf32", "ieee"):
        raise ValueError(f"precision must be 'tf32' or 'ieee', got {name!r}")
    _state["precision"] = name


def get_precision() -> str:
    return _state["precision"]


def _prec_code() -> int:
    return nat.PREC_TF32 if _state["precision"] == "tf32" else nat.PREC_IEEE


def _check_inputs(U, K, a, b, m, n, rule, ns):
    if not (U.is_cuda and K.is_cuda):
        raise RuntimeError("HIP scan needs GPU tensors")
    if U.dim() != 5 or U.shape[-1] != U.shape[-2] or K.shape != U.shape:
        raise RuntimeError(f"U and K must be (B, H, N, dh, dh) with equal shapes, got {tuple(U.shape)}, {tuple(K.shape)}")
    dh = U.shape[-1]
    if dh not in SUPPORTED_DH:
        raise RuntimeError(f"HIP scan supports head dims {SUPPORTED_DH}, got {dh}")
    for name, t in (("a", a), ("b", b), ("m", m), ("n", n)):
        if tuple(t.shape) != tuple(U.shape[:3]):
            raise RuntimeError(f"{name} must have shape {tuple(U.shape[:3])}, got {tuple(t.shape)}")
    if rule not in (0, 1, 2):
        raise RuntimeError(f"rule must be 0, 1 or 2, got {rule}")
    if not 0 <= ns <= 8:
        raise RuntimeError(f"ns must be in [0, 8], got {ns}")


def _f32(t):
    return t.detach().to(torch.float32).contiguous()


class HipScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, U, K, a, b, m, n, rule, ns):
        _check_inputs(U, K, a, b, m, n, rule, ns)
        lib = nat.load()
        B, H, N, dh, _ = U.shape
        Uc, Kc = _f32(U), _f32(K)
        ac, bc, mc, nc = (_f32(t) for t in (a, b, m, n))
        S_all = torch.empty_like(Uc)
        need_grad = any(ctx.needs_input_grad[:6])
        M_all = torch.empty_like(Uc) if (rule != 0 and need_grad) else None
        V_all = torch.empty_like(Uc) if (rule == 2 and need_grad) else None
        prec = _prec_code()
        with torch.cuda.device(U.device):
            rc = lib.gmdn_scan_fwd(
                nat.ptr(Uc), nat.ptr(Kc), nat.ptr(ac), nat.ptr(bc), nat.ptr(mc), nat.ptr(nc),
                nat.ptr(S_all), nat.ptr(M_all), nat.ptr(V_all),
                B * H, N, dh, rule, ns, prec, nat.stream_of(U))
        nat.check(rc, "gmdn_scan_fwd")
        ctx.save_for_backward(Uc, Kc, ac, bc, mc, nc, S_all, M_all, V_all)
        ctx.rule, ctx.ns, ctx.prec = rule, ns, prec
        ctx.dtypes = tuple(t.dtype for t in (U, K, a, b, m, n))
        return S_all if U.dtype == torch.float32 else S_all.to(U.dtype)

    @staticmethod
    def backward(ctx, gS):
        Uc, Kc, ac, bc, mc, nc, S_all, M_all, V_all = ctx.saved_tensors
        lib = nat.load()
        B, H, N, dh, _ = Uc.shape
        gSc = _f32(gS)
        dU, dK = torch.empty_like(Uc), torch.empty_like(Kc)
        da, db, dm, dn = (torch.empty_like(ac) for _ in range(4))
        ws_bytes = lib.gmdn_scan_bwd_workspace_bytes(B * H, N, dh, ctx.rule, ctx.ns)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=Uc.device) if ws_bytes else None
        with torch.cuda.device(Uc.device):
            rc = lib.gmdn_scan_bwd(
                nat.ptr(Uc), nat.ptr(Kc), nat.ptr(ac), nat.ptr(bc), nat.ptr(mc), nat.ptr(nc),
                nat.ptr(S_all), nat.ptr(M_all), nat.ptr(V_all), nat.ptr(gSc),
                nat.ptr(dU), nat.ptr(dK), nat.ptr(da), nat.ptr(db), nat.ptr(dm), nat.ptr(dn),
                nat.ptr(ws), ws_bytes, B * H, N, dh, ctx.rule, ctx.ns, ctx.prec,
                nat.stream_of(Uc))
        nat.check(rc, "gmdn_scan_bwd")
        grads = [g if g.dtype == dt else g.to(dt) for g, dt in zip((dU, dK, da, db, dm, dn), ctx.dtypes)]
        return (*grads, None, None)
