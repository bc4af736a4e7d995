"""The reference's outer Muon optimizer on the HIP msign kernels.

``msign`` restates train_ablation.py:60-73 (Frobenius normalisation, then
``steps`` quintic Newton-Schulz steps on the wide orientation of each
matrix, the result cast back to the input dtype) as one call of
``torch.ops.gmdn.msign`` for a whole batch of matrices.

``Muon`` restates the optimizer of train_ablation.py:264-288 with the same
constructor arguments, defaults, state (``buf``) and update
``p <- p (1 - lr wd) - lr max(1, rows/cols)^0.5 msign(u)`` with
``u = g + mom buf`` (Nesterov) or ``buf``.  The only change is scheduling:
the reference runs msign one parameter at a time; here the updates of every
parameter of one shape are stacked and orthogonalised in one batched call
(msign acts on each matrix independently, so the result is the same).

``build_optimizers`` restates train_ablation.py:291-307: 2-D weights other
than the embedding go to Muon when ``outer == "muon"``, everything else to
AdamW(betas (0.9, 0.95)).
"""
from __future__ import annotations

from collections import defaultdict

import torch
from torch import Tensor

from . import ops  # noqa: F401  -- registers torch.ops.gmdn.*

NS_STEPS = 5
EPS = 1e-7


def msign(M: Tensor, steps: int = NS_STEPS, eps: float = EPS) -> Tensor:
    """msign of a matrix or of each matrix of a batch (..., rows, cols) on the
    HIP kernels.  float32 and bfloat16 run as they are; other dtypes go
    through float32 (the reference computes in float32 whatever the input,
    train_ablation.py:61-62) and come back in their own dtype."""
    if not M.is_cuda:
        raise RuntimeError("gmdn_amd.muon.msign runs on the GPU kernels only; got a CPU tensor")
    if M.dtype in (torch.float32, torch.bfloat16):
        return torch.ops.gmdn.msign(M, int(steps), float(eps))
    return torch.ops.gmdn.msign(M.float(), int(steps), float(eps)).to(M.dtype)


class Muon(torch.optim.Optimizer):
    """Momentum + Nesterov + msign for 2-D weights (train_ablation.py:264-288)."""

    def __init__(self, params, lr=0.02, momentum=0.95, nesterov=True, weight_decay=0.0, ns_steps=5):
        super().__init__(params, dict(lr=lr, momentum=momentum, nesterov=nesterov, weight_decay=weight_decay,
                                      ns_steps=ns_steps))

    @torch.no_grad()
    def step(self):
        for group in self.param_groups:
            lr, mom = group["lr"], group["momentum"]
            live, updates = [], []
            for p in group["params"]:
                if p.grad is None:
                    continue
                g = p.grad
                st = self.state[p]
                if "buf" not in st:
                    st["buf"] = torch.zeros_like(g)
                buf = st["buf"]
                buf.mul_(mom).add_(g)
                live.append(p)
                updates.append(g.add(buf, alpha=mom) if group["nesterov"] else buf)
            # one batched msign per (shape, dtype, device)
            by_key = defaultdict(list)
            for i, u in enumerate(updates):
                by_key[(tuple(u.shape), u.dtype, u.device)].append(i)
            ortho = [None] * len(updates)
            for idx in by_key.values():
                stacked = torch.stack([updates[i] for i in idx]) if len(idx) > 1 else updates[idx[0]].unsqueeze(0)
                out = msign(stacked, group["ns_steps"])
                for j, i in enumerate(idx):
                    ortho[i] = out[j]
            for p, u in zip(live, ortho):
                scale = max(1.0, p.shape[0] / p.shape[1]) ** 0.5
                if group["weight_decay"]:
                    p.mul_(1 - lr * group["weight_decay"])
                p.add_(u, alpha=-lr * scale)


def build_optimizers(model, outer: str, args):
    """Outer optimizers of the LM stack (train_ablation.py:291-307); ``args``
    carries ``muon_lr``, ``adam_lr`` and ``weight_decay`` (the trainer's
    --muon-lr 0.02, --adam-lr 4e-4, --weight-decay 0.1 flags,
    train_ablation.py:567-569)."""
    hidden2d, other = [], []
    emb_ids = {id(model.emb.weight)}
    for p in model.parameters():
        if not p.requires_grad:
            continue
        if p.ndim == 2 and id(p) not in emb_ids:
            hidden2d.append(p)
        else:
            other.append(p)
    adamw_kw = dict(lr=args.adam_lr, betas=(0.9, 0.95), weight_decay=args.weight_decay)
    if outer == "muon":
        return [Muon(hidden2d, lr=args.muon_lr, weight_decay=args.weight_decay),
                torch.optim.AdamW(other, **adamw_kw)]
    return [torch.optim.AdamW(hidden2d, **adamw_kw), torch.optim.AdamW(other, **adamw_kw)]
