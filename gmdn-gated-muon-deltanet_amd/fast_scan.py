"""Drop-in replacement of the reference's ``fast_scan`` module for MI355X.

Put this directory on ``sys.path`` and ``import fast_scan`` exactly as the
reference's ``train_ablation.py`` and ``test.py`` do.  The public surface
mirrors reference ``fast_scan.py``:

* ``fast_state_scan(U, K, a, b, m, n, rule, ns)`` -- the dispatcher
  (reference :403-414).  GPU tensors run the hand-written gfx950 kernels of
  ``libgmdn_scan.so``; CPU tensors (or ``set_backend('eager')``) run
  ``scan_eager``.
* ``set_backend('auto' | 'triton' | 'eager')`` and
  ``set_precision('tf32' | 'ieee')`` (reference :47-56); 'triton' is kept as
  the name of the native (HIP) backend so existing ``--scan triton`` flags
  work, and 'hip' is accepted as an alias.
* ``HAS_TRITON`` -- True when the native library is loadable (the flag
  callers test before requesting the kernel backend, reference :36-41).
* ``_TritonScan`` -- the autograd op, here the HIP one (reference :334-396).
* ``scan_eager``, ``manual_backward``, ``NS_A/NS_B/NS_C``, ``_EPS_NORM``,
  ``_EPS_ADAM`` (reference :32-34, :59-186).

Differences from the reference, on purpose:

* A GPU tensor never silently takes the eager path: if the native library
  is missing, or dh is not one of the built sizes (32, 64, 128), the call
  raises ``RuntimeError`` unless the backend was set to 'eager' explicitly.
* gfx950 has no TF32 MFMA; 'tf32' maps to bf16x3 split products (more
  accurate than TF32) and 'ieee' to fp32 MFMA.
* Gradients of gates the rule does not use are zeros (the reference's Triton
  backward leaves them uninitialised, reference :387-389).
"""
from __future__ import annotations

import torch

from gmdn_amd import _native
from gmdn_amd.scan import HipScan, SUPPORTED_DH, hip_state_scan
from gmdn_amd import scan as _scan_mod

NS_A, NS_B, NS_C = 3.4445, -4.7750, 2.0315
_EPS_NORM = 1e-7
_EPS_ADAM = 1e-6

HAS_NATIVE = _native.available()
HAS_TRITON = HAS_NATIVE  # compat name: "the kernel backend is available"

_BACKEND = "auto"     # 'auto' | 'triton' (native) | 'eager'
_PRECISION = "tf32"   # 'tf32' | 'ieee'

_TritonScan = HipScan


def set_precision(name: str):
    global _PRECISION
    assert name in ("tf32", "ieee")
    _PRECISION = name
    _scan_mod.set_precision(name)


def set_backend(name: str):
    global _BACKEND
    if name == "hip":
        name = "triton"
    assert name in ("auto", "triton", "eager")
    _BACKEND = name


# ---------------------------------------------------------------------------
# Eager implementation (CPU tensors, or backend 'eager')
# ---------------------------------------------------------------------------

def _ns_step(X):
    P = X @ X.mT
    return NS_A * X + (NS_B * P + NS_C * (P @ P)) @ X


def _msign_sq(M: torch.Tensor, ns: int) -> torch.Tensor:
    """Frobenius-normalised quintic Newton-Schulz for square matrices."""
    X = M / (M.norm(dim=(-2, -1), keepdim=True) + _EPS_NORM)
    for _ in range(ns):
        X = _ns_step(X)
    return X


def scan_eager(U, K, a, b, m, n, rule: int, ns: int) -> torch.Tensor:
    """Pre-update state stack by a Python loop over chunks; autograd
    differentiates it.  U, K: (B, H, N, dh, dh); a, b, m, n: (B, H, N)."""
    B, H, N, dh, _ = U.shape
    S = U.new_zeros(B, H, dh, dh)
    M = torch.zeros_like(S)
    V = torch.zeros_like(S)
    out = []
    for i in range(N):
        out.append(S)
        G = U[:, :, i] - S @ K[:, :, i]
        ai = a[:, :, i, None, None]
        if rule == 0:
            S = ai * S + G
        elif rule == 1:
            M = m[:, :, i, None, None] * M + G
            S = ai * S + b[:, :, i, None, None] * _msign_sq(M, ns)
        else:
            mi, ni = m[:, :, i, None, None], n[:, :, i, None, None]
            M = mi * M + (1 - mi) * G
            V = ni * V + (1 - ni) * G * G
            S = ai * S + b[:, :, i, None, None] * M / (V.sqrt() + _EPS_ADAM)
    return torch.stack(out, dim=2)


def _msign_vjp(Mi, Ybar, ns: int):
    """VJP of msign with the iterates kept from one forward pass."""
    nf = Mi.norm(dim=(-2, -1), keepdim=True)
    nrm = nf + _EPS_NORM
    X = Mi / nrm
    its = []
    for _ in range(ns):
        its.append(X)
        X = _ns_step(X)
    Xbar = Ybar
    for Xk in reversed(its):
        P = Xk @ Xk.mT
        Bm = NS_B * P + NS_C * (P @ P)
        Bbar = Xbar @ Xk.mT
        Abar = NS_B * Bbar + NS_C * (Bbar @ P + P @ Bbar)
        Xbar = NS_A * Xbar + Bm @ Xbar + (Abar + Abar.mT) @ Xk
    dot = (Xbar * Mi).sum(dim=(-2, -1), keepdim=True)
    return Xbar / nrm - dot / nrm.square() * (Mi / nf.clamp_min(1e-12))


def manual_backward(U, K, a, b, m, n, S_all, M_all, V_all, gS, rule: int, ns: int):
    """Hand-derived reverse scan in PyTorch; returns dU, dK, da, db, dm, dn."""
    B, H, N, dh, _ = U.shape
    dU, dK = torch.zeros_like(U), torch.zeros_like(K)
    da, db, dm, dn = (torch.zeros_like(t) for t in (a, b, m, n))
    Sb = U.new_zeros(B, H, dh, dh)
    Mb, Vb = torch.zeros_like(Sb), torch.zeros_like(Sb)
    for i in reversed(range(N)):
        S, Ki = S_all[:, :, i], K[:, :, i]
        ai, bi, mi = (t[:, :, i, None, None] for t in (a, b, m))
        G = U[:, :, i] - S @ Ki
        da[:, :, i] = (Sb * S).sum(dim=(-2, -1))
        if rule == 0:
            Gb = Sb
        elif rule == 1:
            Mp = M_all[:, :, i]
            Mi = mi * Mp + G
            db[:, :, i] = (Sb * _msign_sq(Mi, ns)).sum(dim=(-2, -1))
            Mtot = Mb + _msign_vjp(Mi, bi * Sb, ns)
            dm[:, :, i] = (Mtot * Mp).sum(dim=(-2, -1))
            Mb = mi * Mtot
            Gb = Mtot
        else:
            ni = n[:, :, i, None, None]
            Mp, Vp = M_all[:, :, i], V_all[:, :, i]
            Mi = mi * Mp + (1 - mi) * G
            Vi = ni * Vp + (1 - ni) * G * G
            root = Vi.sqrt()
            den = root + _EPS_ADAM
            db[:, :, i] = (Sb * Mi / den).sum(dim=(-2, -1))
            ub = bi * Sb
            Mtot = Mb + ub / den
            Vtot = Vb - ub * Mi / den.square() / (2 * root.clamp_min(1e-12))
            dm[:, :, i] = (Mtot * (Mp - G)).sum(dim=(-2, -1))
            dn[:, :, i] = (Vtot * (Vp - G * G)).sum(dim=(-2, -1))
            Mb, Vb = mi * Mtot, ni * Vtot
            Gb = (1 - mi) * Mtot + (1 - ni) * 2 * G * Vtot
        dU[:, :, i] = Gb
        dK[:, :, i] = -S.mT @ Gb
        Sb = ai * Sb - Gb @ Ki.mT + gS[:, :, i]
    return dU, dK, da, db, dm, dn


# ---------------------------------------------------------------------------
# Dispatcher
# ---------------------------------------------------------------------------

def fast_state_scan(U, K, a, b, m, n, rule: int, ns: int) -> torch.Tensor:
    """Pre-update state stack (B, H, N, dh, dh).  GPU tensors run the HIP
    kernels (backend 'auto' or 'triton'); CPU tensors run scan_eager unless
    the native backend was forced, which raises."""
    if _BACKEND == "eager":
        return scan_eager(U, K, a, b, m, n, rule, ns)
    if U.is_cuda:
        if not HAS_NATIVE:
            raise RuntimeError("GPU tensors need the native gmdn kernels, but libgmdn_scan.so "
                               "is not built; build it or set_backend('eager') explicitly")
        if U.shape[-1] not in SUPPORTED_DH:
            raise RuntimeError(f"native scan supports head dims {SUPPORTED_DH}, got {U.shape[-1]}; "
                               "set_backend('eager') to run this size eagerly")
        return hip_state_scan(U, K, a, b, m, n, rule, ns)
    if _BACKEND == "triton":
        raise RuntimeError("native backend requested but unavailable for CPU tensors "
                           "(needs GPU tensors and libgmdn_scan.so)")
    return scan_eager(U, K, a, b, m, n, rule, ns)
