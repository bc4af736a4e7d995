"""The reference's fast-weight mixer layer and LM stack around the fused core.

``FastWeightMixer``, ``Block`` and ``LM`` restate train_ablation.py:80-257
with the same constructor arguments, parameter names and shapes (so a
reference ``state_dict`` loads unchanged), the same front-end (qkv
projection, causal depthwise conv, SiLU, per-head L2 norm, gate sigmoids),
tail (per-head RMSNorm, output projection) and initialisation.  The conv,
SiLU and norms run as one HIP kernel per direction
(``torch.ops.gmdn.front_fwd``), the gate activations as another
(``gates_fwd``); phases 1-3 of the mixer (train_ablation.py:142-187: gate
reductions, the intra-chunk products, the state scan and the output) are one
call of ``chunk_scan`` -- the fused HIP core at chunk length 64, the
reference's schedule around the drop-in HIP scan at other lengths -- whose
output lands in the
(B, T, H, dh) layout that the per-head RMSNorm kernel (``head_norm_fwd``)
and the output projection read.

The stack is the end-to-end harness for the 12-layer, d_model 1024, 8-head,
muon configuration: it measures the whole training step around the core.
The trainer, its data pipeline and the outer optimisers are not restated.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops  # noqa: F401  -- registers torch.ops.gmdn.*
from .chunk import chunk_scan


class FastWeightMixer(nn.Module):
    """Token mixing via per-head fast weights (train_ablation.py:80-108)."""

    def __init__(self, d_model: int, n_heads: int, inner: str, chunk: int = 64, ns_steps: int = 3,
                 conv_kernel: int = 4):
        super().__init__()
        assert inner in ("delta", "muon", "adam")
        assert d_model % n_heads == 0
        self.h, self.dh = n_heads, d_model // n_heads
        self.inner, self.chunk, self.ns_steps = inner, chunk, ns_steps
        self.qkv = nn.Linear(d_model, 3 * d_model, bias=False)
        self.conv = nn.Conv1d(3 * d_model, 3 * d_model, conv_kernel, groups=3 * d_model,
                              padding=conv_kernel - 1)
        self.n_gates = 4 if inner == "adam" else 3  # alpha, beta, mu (, nu)
        self.gates = nn.Linear(d_model, self.n_gates * n_heads, bias=True)
        self.norm = nn.RMSNorm(self.dh)
        self.out = nn.Linear(d_model, d_model, bias=False)
        self.reset_gate_bias()

    def reset_gate_bias(self):
        """Gate priors alpha ~ 0.95, beta ~ 0.27, mu ~ 0.73, nu ~ 0.88
        (train_ablation.py:101-108)."""
        with torch.no_grad():
            bias = self.gates.bias.view(self.n_gates, self.h)
            bias[0].fill_(3.0)
            bias[1].fill_(-1.0)
            bias[2].fill_(1.0)
            if self.n_gates == 4:
                bias[3].fill_(2.0)

    def front_end(self, x: torch.Tensor):
        """q, k, v (B, H, T, dh) views and the gate streams (B, H, T): beta and
        the log gates clamped at log 1e-6 (train_ablation.py:124-134, 155, 170-175)."""
        B, T, D = x.shape
        H, dh = self.h, self.dh
        # conv, SiLU and the q / k norms in one HIP kernel per direction
        q, k, v = torch.ops.gmdn.front_fwd(self.qkv(x), self.conv.weight, self.conv.bias, dh)
        q, k, v = (t.view(B, T, H, dh).transpose(1, 2) for t in (q, k, v))
        # beta = sigmoid and the other gates' logs (log sigmoid, the reference's
        # 1e-6 floor) as (B, H, T) float32 rows, in one HIP pass per direction
        gs = torch.ops.gmdn.gates_fwd(self.gates(x), H, self.n_gates)  # (nG, B, H, T)
        log_nu = gs[3] if self.n_gates == 4 else None
        return q, k, v, gs[1], gs[0], gs[2], log_nu

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, D = x.shape
        if T % self.chunk:
            raise ValueError("seq_len must be a multiple of chunk size")
        q, k, v, beta, log_alpha, log_mu, log_nu = self.front_end(x)
        # float32 activations (autocast off: the reference's precision there,
        # train_ablation.py:424, 465) stay float32; others run in bfloat16
        dt = torch.float32 if q.dtype == torch.float32 else torch.bfloat16
        o = chunk_scan(q.to(dt), k.to(dt), v.to(dt), beta, log_alpha, log_mu, log_nu, rule=self.inner,
                       ns=self.ns_steps, chunk=self.chunk)
        # per-head RMSNorm (HIP) on o's (B, T, H, dh) storage: the output is
        # already the (B, T, D) input of the projection.  The reference norms
        # in float32 (autocast runs RMSNorm in float32) and autocast rounds the
        # result to bfloat16 for the projection; under bfloat16 autocast the
        # kernel reads the bfloat16 o and writes that rounding itself (it
        # computes in float32 either way), so no float32 copy is made.
        ot = o.transpose(1, 2)
        bf16_autocast = (ot.dtype == torch.bfloat16 and torch.is_autocast_enabled(ot.device.type)
                         and torch.get_autocast_dtype(ot.device.type) == torch.bfloat16)
        if not bf16_autocast:
            ot = ot.to(self.norm.weight.dtype)
        # (nn.RMSNorm's default eps is its input dtype's: float32 under autocast)
        eps = self.norm.eps if self.norm.eps is not None else torch.finfo(
            torch.float32 if bf16_autocast else ot.dtype).eps
        y, _ = torch.ops.gmdn.head_norm_fwd(ot, self.norm.weight.float(), eps)
        y = y.view(B, T, D)
        return self.out(y if bf16_autocast else y.to(x.dtype))


class Block(nn.Module):
    """Pre-norm residual block: mixer, then a 4x GELU MLP (train_ablation.py:197-210)."""

    def __init__(self, d_model, n_heads, inner, chunk, ns_steps=3):
        super().__init__()
        self.n1 = nn.RMSNorm(d_model)
        self.mixer = FastWeightMixer(d_model, n_heads, inner, chunk, ns_steps)
        self.n2 = nn.RMSNorm(d_model)
        self.mlp = nn.Sequential(nn.Linear(d_model, 4 * d_model, bias=False), nn.GELU(),
                                 nn.Linear(4 * d_model, d_model, bias=False))

    def forward(self, x):
        x = x + self.mixer(self.n1(x))
        return x + self.mlp(self.n2(x))


class LM(nn.Module):
    """Embedding, blocks, final RMSNorm and a tied head; next-token cross
    entropy in float32 (train_ablation.py:213-243)."""

    def __init__(self, vocab, d_model, n_layers, n_heads, inner, chunk=64, ns_steps=3):
        super().__init__()
        self.emb = nn.Embedding(vocab, d_model)
        self.blocks = nn.ModuleList(Block(d_model, n_heads, inner, chunk, ns_steps) for _ in range(n_layers))
        self.norm_f = nn.RMSNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab, bias=False)
        self.lm_head.weight = self.emb.weight  # tied
        self.apply(self._init)
        for blk in self.blocks:  # scaled residual init
            for w in (blk.mixer.out.weight, blk.mlp[2].weight):
                nn.init.normal_(w, std=0.02 / math.sqrt(2 * n_layers))
            blk.mixer.reset_gate_bias()

    @staticmethod
    def _init(m):
        if isinstance(m, nn.Linear):
            nn.init.normal_(m.weight, std=0.02)
            if m.bias is not None:
                nn.init.zeros_(m.bias)
        elif isinstance(m, nn.Embedding):
            nn.init.normal_(m.weight, std=0.02)

    def forward(self, idx, targets=None):
        x = self.emb(idx)
        for blk in self.blocks:
            x = blk(x)
        logits = self.lm_head(self.norm_f(x))
        if targets is None:
            return logits, None
        loss = F.cross_entropy(logits.view(-1, logits.size(-1)).float(), targets.reshape(-1))
        return logits, loss
