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
* ``scan_eager``, ``manual_backward``, ``_msign_sq``, ``_msign_vjp``,
  ``_ns_step``, ``NS_A/NS_B/NS_C``, ``_EPS_NORM``, ``_EPS_ADAM`` (reference
  :32-34, :59-186), written here around a carried state tuple per rule.

Differences from the reference, on purpose:

* A GPU tensor never silently takes the eager path because the native
  library is missing: that raises ``RuntimeError`` unless the backend was
  set to 'eager' explicitly.  Head dims without kernels run eagerly under
  'auto' and raise under 'triton', as the reference dispatches (:403-414);
  the kernels cover 32, 64 and 128, and 16 by zero-padding to 32.
* gfx950 has no TF32 MFMA; 'tf32' maps to bf16x3 split products (more
  accurate than TF32) and 'ieee' to fp32 MFMA.
* Adam (rule 2) run with gradients enabled takes 'ieee' for its forward
  whatever ``set_precision`` says: its backward amplifies the rounding of
  the saved moments past the gradient tolerance under split products.  So
  under 'tf32' its S_all with grad enabled can differ in the last bits from
  the same call without grad.
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
# Eager implementation (CPU tensors, backend 'eager', head dims without kernels)
#
# The scan carries per (b, h) a state tuple through the chunks: (S,) for
# delta, (S, M) for muon, (S, M, V) for adam.  ``_advance`` applies one
# chunk's update to the tuple; ``manual_backward`` walks the chunks in
# reverse, carrying the cotangents of the same tuple, with ``_retreat`` the
# VJP of one chunk's update.  Gates are viewed once as (B, H, N, 1, 1).
# ---------------------------------------------------------------------------

def _gate_views(*gates):
    return [g[..., None, None] for g in gates]


def _ns_step(X):
    """One quintic Newton-Schulz step X -> a X + b (P X) + c P (P X), P = X X^T."""
    PX = (X @ X.mT) @ X
    return NS_A * X + NS_B * PX + NS_C * ((X @ X.mT) @ PX)


def _normalise(M):
    """M / (||M||_F + eps) and the norm itself."""
    nf = torch.linalg.matrix_norm(M)[..., None, None]
    return M / (nf + _EPS_NORM), nf


def _msign_sq(M: torch.Tensor, ns: int) -> torch.Tensor:
    """Frobenius-normalised quintic Newton-Schulz of square matrices."""
    X, _ = _normalise(M)
    for _ in range(ns):
        X = _ns_step(X)
    return X


def _advance(rule, ns, carry, G, ai, bi, mi, ni):
    """One chunk's update of the carried (S[, M[, V]]) given G = U - S K."""
    S = carry[0]
    if rule == 0:
        return (ai * S + G,)
    if rule == 1:
        M = mi * carry[1] + G
        return (ai * S + bi * _msign_sq(M, ns), M)
    M = torch.lerp(G, carry[1], mi)            # m M + (1 - m) G
    V = torch.lerp(G * G, carry[2], ni)        # n V + (1 - n) G^2
    return (ai * S + bi * (M / (V.sqrt() + _EPS_ADAM)), M, V)


def scan_eager(U, K, a, b, m, n, rule: int, ns: int) -> torch.Tensor:
    """Stack of pre-update states (B, H, N, dh, dh) by a loop over chunks;
    autograd differentiates it.  U, K: (B, H, N, dh, dh); a, b, m, n: (B, H, N)."""
    Bn, Hn, N, dh, _ = U.shape
    zero = U.new_zeros(Bn, Hn, dh, dh)
    carry = (zero,) if rule == 0 else (zero, zero) if rule == 1 else (zero, zero, zero)
    av, bv, mv, nv = _gate_views(a, b, m, n)
    pre = []
    for i in range(N):
        pre.append(carry[0])
        G = U.select(2, i) - carry[0] @ K.select(2, i)
        carry = _advance(rule, ns, carry, G, av.select(2, i), bv.select(2, i), mv.select(2, i),
                         nv.select(2, i))
    if N == 0:
        return U.new_zeros(U.shape)
    return torch.stack(pre, dim=2)


def _msign_vjp(Mi, Ybar, ns: int):
    """Cotangent of M for Y = msign(M), given Ybar.  The iterates X_0..X_{ns-1}
    are kept from one forward pass.  Per step, with P = X X^T and
    Z = b P + c P^2, the cotangent Xbar of X' = a X + Z X becomes
        Bs = Xbar X^T + X Xbar^T,  Y = P Bs,
        Xbar <- a Xbar + Z Xbar + (b Bs + c (Y + Y^T)) X.
    Normalisation X_0 = M / n, n = ||M|| + eps:
        Mbar = (Xbar_0 - <Xbar_0, X_0> M / ||M||) / n."""
    X, nf = _normalise(Mi)
    iterates = [X]
    for _ in range(ns - 1):
        iterates.append(_ns_step(iterates[-1]))
    Xbar = Ybar
    for Xk in (reversed(iterates) if ns > 0 else ()):
        P = Xk @ Xk.mT
        Z = NS_B * P + NS_C * (P @ P)
        Bs = Xbar @ Xk.mT
        Bs = Bs + Bs.mT
        Y = P @ Bs
        Xbar = NS_A * Xbar + Z @ Xbar + (NS_B * Bs + NS_C * (Y + Y.mT)) @ Xk
    X0 = iterates[0]
    proj = (Xbar * X0).sum(dim=(-2, -1), keepdim=True)
    return (Xbar - proj * Mi / nf.clamp_min(1e-12)) / (nf + _EPS_NORM)


def _retreat(rule, ns, Sbar, carry_bar, G, M_prev, V_prev, bi, mi, ni):
    """VJP of one chunk's update except the a S term: from the cotangent
    Sbar of S_{i+1} and the carried cotangents of M_{i+1} (and V_{i+1}),
    returns (Gbar, dbeta, dmu, dnu, cotangents of M_i[, V_i])."""
    zero = Sbar.new_zeros(Sbar.shape[:-2])
    if rule == 0:
        return Sbar, zero, zero, zero, ()
    if rule == 1:
        M = mi * M_prev + G
        Y = _msign_sq(M, ns)
        Mtot = carry_bar[0] + _msign_vjp(M, bi * Sbar, ns)
        return (Mtot, (Sbar * Y).sum(dim=(-2, -1)), (Mtot * M_prev).sum(dim=(-2, -1)), zero,
                (mi * Mtot,))
    M = torch.lerp(G, M_prev, mi)
    V = torch.lerp(G * G, V_prev, ni)
    root = V.sqrt()
    inv = 1.0 / (root + _EPS_ADAM)
    ubar = bi * Sbar
    Mtot = carry_bar[0] + ubar * inv
    Vtot = carry_bar[1] - 0.5 * ubar * M * inv * inv / root.clamp_min(1e-12)
    Gbar = (1 - mi) * Mtot + 2 * (1 - ni) * G * Vtot
    return (Gbar, (Sbar * M * inv).sum(dim=(-2, -1)), (Mtot * (M_prev - G)).sum(dim=(-2, -1)),
            (Vtot * (V_prev - G * G)).sum(dim=(-2, -1)), (mi * Mtot, ni * Vtot))


def manual_backward(U, K, a, b, m, n, S_all, M_all, V_all, gS, rule: int, ns: int):
    """Hand-derived reverse scan: returns dU, dK, da, db, dm, dn.  S_all,
    M_all, V_all hold the pre-update values of every chunk."""
    N = U.shape[2]
    grads = {name: torch.zeros_like(t) for name, t in (("U", U), ("K", K), ("a", a), ("b", b), ("m", m),
                                                       ("n", n))}
    if N == 0:
        return tuple(grads[k] for k in ("U", "K", "a", "b", "m", "n"))
    av, bv, mv, nv = _gate_views(a, b, m, n)
    Sbar = torch.zeros_like(U.select(2, 0))
    carry_bar = () if rule == 0 else (torch.zeros_like(Sbar),) if rule == 1 else (torch.zeros_like(Sbar),) * 2
    for i in range(N - 1, -1, -1):
        S, Ki = S_all.select(2, i), K.select(2, i)
        G = U.select(2, i) - S @ Ki
        M_prev = M_all.select(2, i) if rule else None
        V_prev = V_all.select(2, i) if rule == 2 else None
        Gbar, dbi, dmi, dni, carry_bar = _retreat(rule, ns, Sbar, carry_bar, G, M_prev, V_prev, bv.select(2, i),
                                                  mv.select(2, i), nv.select(2, i))
        grads["a"][:, :, i] = (Sbar * S).sum(dim=(-2, -1))
        grads["b"][:, :, i], grads["m"][:, :, i], grads["n"][:, :, i] = dbi, dmi, dni
        grads["U"][:, :, i] = Gbar
        grads["K"][:, :, i] = -(S.mT @ Gbar)
        Sbar = av.select(2, i) * Sbar - Gbar @ Ki.mT + gS.select(2, i)
    return tuple(grads[k] for k in ("U", "K", "a", "b", "m", "n"))


# ---------------------------------------------------------------------------
# Dispatcher (reference fast_scan.py:403-414)
# ---------------------------------------------------------------------------

def fast_state_scan(U, K, a, b, m, n, rule: int, ns: int) -> torch.Tensor:
    """Pre-update state stack (B, H, N, dh, dh).

    * backend 'eager': ``scan_eager``.
    * GPU tensors whose head dim has kernels (16, 32, 64, 128): the HIP
      kernels.  A GPU tensor never runs eagerly because the native library
      is missing: that raises.
    * otherwise (CPU tensors, other head dims): ``scan_eager`` under 'auto';
      under 'triton' (the native backend forced) a ``RuntimeError``, as the
      reference raises when its kernel cannot run.
    """
    if _BACKEND == "eager":
        return scan_eager(U, K, a, b, m, n, rule, ns)
    if U.is_cuda and not HAS_NATIVE:
        raise RuntimeError("GPU tensors need the native gmdn kernels, but libgmdn_scan.so "
                           "is not built; build it or set_backend('eager') explicitly")
    if U.is_cuda and U.shape[-1] in SUPPORTED_DH:
        return hip_state_scan(U, K, a, b, m, n, rule, ns)
    if _BACKEND == "triton":
        raise RuntimeError("native backend requested but unavailable (needs GPU tensors, libgmdn_scan.so "
                           f"and a head dim in {SUPPORTED_DH}; got dh={U.shape[-1]}, "
                           f"device {U.device})")
    return scan_eager(U, K, a, b, m, n, rule, ns)
