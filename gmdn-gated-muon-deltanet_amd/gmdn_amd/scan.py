"""Autograd op of the drop-in chunk state scan (Level A).

``HipScan.apply(U, K, a, b, m, n, rule, ns)`` has the signature and
semantics of the reference's ``_TritonScan`` (fast_scan.py:334-396): U, K are
(B, H, N, dh, dh), a, b, m, n are (B, H, N); the result is the stack of
pre-update states S_0..S_{N-1}, and the backward returns gradients for the
six tensor inputs (``None`` for rule and ns).  ``hip_state_scan`` is the same
computation through the registered operator's autograd, which
``torch.compile`` traces.  Both run the HIP kernels of ``libgmdn_scan.so``
(``torch.ops.gmdn.state_scan`` / ``state_scan_bwd``) on the tensors'
current stream.
"""
from __future__ import annotations

import torch

from . import _native as nat
from . import ops  # noqa: F401  -- registers torch.ops.gmdn.*

KERNEL_DH = (32, 64, 128)       # head dims the kernels are built for
SUPPORTED_DH = (16,) + KERNEL_DH  # 16: zero-padded to 32 on the way in
_state = {"precision": "tf32"}


def _padded_dh(dh: int) -> int:
    """Kernel head dim that serves ``dh``.  Zero-padding U and K to 32 x 32
    is exact for every rule: the padded state, moments, Newton-Schulz
    iterates and gradients stay block-diagonal with the dh x dh problem in
    the leading block (rows and columns past dh are identically zero)."""
    return 32 if dh < 32 else dh


def _pad_sq(x, d: int):
    p = d - x.shape[-1]
    return x if p == 0 else torch.nn.functional.pad(x, (0, p, 0, p))


def set_precision(name: str) -> None:
    """'tf32' (bf16x3 split MFMA on gfx950) or 'ieee' (fp32 MFMA)."""
    if name not in ("tf32", "ieee"):
        raise ValueError(f"precision must be 'tf32' or 'ieee', got {name!r}")
    _state["precision"] = name


def get_precision() -> str:
    return _state["precision"]


def _prec_code() -> int:
    return _prec_code_of(_state["precision"])


def _prec_code_of(precision: str) -> int:
    if precision not in ("tf32", "ieee"):
        raise ValueError(f"precision must be 'tf32' or 'ieee', got {precision!r}")
    return nat.PREC_TF32 if precision == "tf32" else nat.PREC_IEEE


def _effective_prec(rule: int, save: bool, prec: int) -> int:
    """The product precision a forward actually runs in: adam keeping its
    moments for a backward runs in exact float32 ('ieee') whatever the
    setting, since its backward amplifies the rounding of the saved moments
    (split-bf16 products there put dK 0.29 from float64, in Frobenius norm,
    at BH = 64, N = 64, dh = 128, where float32 gives 3e-3).  The library
    applies the same rule (gmdn_scan_fwd); stating it here makes the choice
    visible at the Python boundary."""
    return nat.PREC_IEEE if (rule == 2 and save) else prec


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
    return t.to(torch.float32).contiguous()


def hip_state_scan(U, K, a, b, m, n, rule: int, ns: int, precision: str | None = None):
    """The scan through ``torch.ops.gmdn.state_scan`` and its registered
    autograd: float32 contiguous copies of the inputs (differentiable casts),
    the pre-update states in U's dtype.  Traceable by ``torch.compile``.
    ``precision`` ('tf32' or 'ieee') overrides the process-wide setting."""
    _check_inputs(U, K, a, b, m, n, rule, ns)
    dh = U.shape[-1]
    kd = _padded_dh(dh)
    ins = [_f32(t) for t in (_pad_sq(U, kd), _pad_sq(K, kd), a, b, m, n)]
    save = torch.is_grad_enabled() and any(t.requires_grad for t in (U, K, a, b, m, n))
    prec = _effective_prec(rule, save, _prec_code() if precision is None else _prec_code_of(precision))
    S_all, _, _ = torch.ops.gmdn.state_scan(*ins, rule, ns, prec, save)
    if kd != dh:
        S_all = S_all[..., :dh, :dh]
    return S_all if U.dtype == torch.float32 else S_all.to(U.dtype)


class HipScan(torch.autograd.Function):
    """``_TritonScan``'s interface over the same two operators."""

    @staticmethod
    def forward(ctx, U, K, a, b, m, n, rule, ns):
        _check_inputs(U, K, a, b, m, n, rule, ns)
        dh = U.shape[-1]
        kd = _padded_dh(dh)
        ins = [_f32(t.detach()) for t in (_pad_sq(U, kd), _pad_sq(K, kd), a, b, m, n)]
        save = any(ctx.needs_input_grad[:6])
        prec = _effective_prec(rule, save, _prec_code())
        S_all, M_all, V_all = torch.ops.gmdn.state_scan(*ins, rule, ns, prec, save)
        ctx.save_for_backward(*ins, S_all, M_all, V_all)
        ctx.rule, ctx.ns, ctx.prec, ctx.dh = rule, ns, prec, dh
        ctx.dtypes = tuple(t.dtype for t in (U, K, a, b, m, n))
        if kd != dh:
            S_all = S_all[..., :dh, :dh]
        return S_all if U.dtype == torch.float32 else S_all.to(U.dtype)

    @staticmethod
    def backward(ctx, gS):
        kd = ctx.saved_tensors[0].shape[-1]
        grads = torch.ops.gmdn.state_scan_bwd(*ctx.saved_tensors, _pad_sq(gS.float(), kd), ctx.rule, ctx.ns,
                                              ctx.prec)
        dh = ctx.dh
        grads = [g[..., :dh, :dh] if i < 2 and kd != dh else g for i, g in enumerate(grads)]
        grads = [g if g.dtype == dt else g.to(dt) for g, dt in zip(grads, ctx.dtypes)]
        return (*grads, None, None)
