"""Synthetic workloads of the benchmark configurations.

Inputs are drawn on the CPU from one ``torch.Generator().manual_seed(seed)``
in a fixed order (q, k, v, beta, g, dO), in float32, then cast and moved, so
a CPU checker and the GPU see identical values:

* q, k ~ N(0, 1) over (B, H, T, d), L2-normalised per head
  (the mixer front-end normalises them, reference train_ablation.py:127-128)
* v ~ N(0, 1); beta = sigmoid(N(0, 1)); g = logsigmoid(N(0, 1) + 3)
* muon: log mu = log(0.9) / 64 per token, so each chunk's momentum product is
  0.9; adam: log mu = log(0.9) / 64, log nu = log(0.999) / 64
* dO ~ N(0, 1) (the cotangent of o)
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    rule: str
    B: int
    H: int
    T: int
    d: int
    ns: int = 5
    chunk: int = 64

    @property
    def tokens(self) -> int:
        return self.B * self.T


# The benchmark configurations (B, H, T, d, chunk 64 throughout).
WORKLOADS = {
    "delta_fp32_small": Workload("delta_fp32_small", "delta", 1, 2, 256, 64),
    "gated_delta_b4_h16_t4096_d128": Workload("gated_delta_b4_h16_t4096_d128", "delta", 4, 16, 4096, 128),
    "muon_b2_h16_t8192_d128": Workload("muon_b2_h16_t8192_d128", "muon", 2, 16, 8192, 128, ns=5),
    "adam_b2_h8_t4096_d64": Workload("adam_b2_h8_t4096_d64", "adam", 2, 8, 4096, 64),
}


def make_inputs(w: Workload, seed: int = 0, device=None, dtype=torch.bfloat16, with_grad_out: bool = True):
    """Return dict(q, k, v, beta, g, gmu, gnu, dO) for workload ``w``."""
    gen = torch.Generator().manual_seed(seed)
    shape = (w.B, w.H, w.T, w.d)
    q = torch.randn(shape, generator=gen)
    q = q / torch.clamp(q.norm(dim=-1, keepdim=True), min=1e-12)
    k = torch.randn(shape, generator=gen)
    k = k / torch.clamp(k.norm(dim=-1, keepdim=True), min=1e-12)
    v = torch.randn(shape, generator=gen)
    beta = torch.sigmoid(torch.randn(w.B, w.H, w.T, generator=gen))
    g = torch.nn.functional.logsigmoid(torch.randn(w.B, w.H, w.T, generator=gen) + 3.0)
    dO = torch.randn(shape, generator=gen) if with_grad_out else None
    gmu = gnu = None
    if w.rule in ("muon", "adam"):
        gmu = torch.full((w.B, w.H, w.T), math.log(0.9) / w.chunk)
    if w.rule == "adam":
        gnu = torch.full((w.B, w.H, w.T), math.log(0.999) / w.chunk)
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), beta=beta, g=g, gmu=gmu, gnu=gnu,
               dO=None if dO is None else dO.to(dtype))
    if device is not None:
        out = {key: (None if t is None else t.to(device)) for key, t in out.items()}
    return out
