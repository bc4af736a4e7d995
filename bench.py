#!/usr/bin/env python3
"""Throughput of the fused chunkwise mixer core on one MI355X.

One step is one pass of the hot path over one batch of synthetic input: the
fused mixer core (reference train_ablation.py:142-187 with the state scan of
fast_scan.py:72-95) over B=4, H=16, T=4096, d=128, chunk 64, gated delta rule,
bf16 q/k/v/o with fp32 state, forward and (where built) backward.  Inputs are
resident in HBM before the timed region starts.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

prints one JSON line.  ``value`` is tokens/s (B*T per step) of the forward +
backward step when the backward of the rule is built, else of the forward.
For the delta and adam rules the training step (forward + backward) is
captured into one HIP graph (its first replay checked bit for bit against an
eager step) and ``value`` times K graph replays bracketed by
synchronisations; the inference forward (one kernel) is timed over K eager
launches.  ``step_us`` keeps both kinds of time (``train_step_eager``: K eager
steps, whose host launch work is in the timed region;
``fwd_inference_graph``) and the per-pass times (HIP events around the eager
launches).
``roofline`` prices the dominant part of the step -- the backward pass (its
two kernels) -- and ``roofline_fwd`` the inference forward kernel: average
durations measured with HIP events on the launch stream inside the timed
regions, algorithmic bytes of the op's own inputs and outputs, against
MI355X's HBM bandwidth (8 TB/s); ``traffic`` is read from the committed
FETCH_SIZE/WRITE_SIZE summaries of the same kernels and workload.
``drop_in`` times the drop-in scan ``fast_state_scan`` on the same chunk
grid (fp32 d x d inputs per chunk), forward and forward + backward, with its
own roofline.  ``cpu_baseline`` times the CPU restatement of the reference matrix form
(float32, torch on the host cores) on the same workload.

``configs`` (default workload only; ``--no-configs`` skips it) holds one
sub-object per other configuration: the muon rule at B=2, H=16, T=8192,
d=128, ns=5 and the adam rule at B=2, H=8, T=4096, d=64 (inference forward
and forward + backward, their rooflines and a CPU baseline on a bounded
sample), the exact WY/UT mode at the default workload's shape (inference
forward and forward + backward, eager), and the 12-layer LM's training step
(tokens/s only).  The CPU
baselines use every CPU of the process's affinity, capped by
OMP_NUM_THREADS when set, and report the host (lscpu model, sockets,
physical cores, torch threads).

``measured_peaks`` (default workload, with ``configs``) gives what the GPU
sustains beside the datasheet peaks the rooflines are priced on: the HBM
bandwidth of a 2 GiB device copy and the bf16 throughput of an 8192^3
torch.matmul.

``--workload lm_b8_t2048_muon`` times the 12-layer LM stack around the
fused core end to end (forward + backward, tokens/s only).
``--workload outer_muon_lm12_d1024`` times one outer Muon optimizer step
(msign of the LM's 60 hidden weights) in fp32-equivalent TFLOP/s.

``--fwd-only`` times the inference forward alone; ``--copy-calibration
BYTES`` only runs a device copy of BYTES bytes a few times (the calibration
kernel for the HBM byte counters).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "gmdn-gated-muon-deltanet_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "scan tokens/s at H16 d128 T4096 bf16 (fwd, fwd+bwd); % of MFMA/HBM peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
DEFAULT_WORKLOAD = "gated_delta_b4_h16_t4096_d128"
GATES = {"delta": 2, "muon": 3, "adam": 4}


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    # the GPU's clocks settle after ~30 ms of continuous work (a kernel-trace
    # of back-to-back steps: the pair kernel goes 316 -> 338 -> 289 us over
    # the first ~50 launches), so the sub-millisecond steps warm up for 50
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--workload", default=DEFAULT_WORKLOAD)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-drop-in", action="store_true", help="skip the drop-in scan (fast_state_scan) leg")
    p.add_argument("--fwd-only", action="store_true", help="time the inference forward only")
    p.add_argument("--no-configs", action="store_true",
                   help="skip the other configurations' sub-objects (muon, adam, LM) of the default line")
    p.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work (about)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES")
    return p.parse_args(argv)


def fwd_bytes_per_token_head(w) -> int:
    """q, k, v read and o written in bf16, plus the fp32 gate streams."""
    return 3 * 2 * w.d + 2 * w.d + 4 * GATES[w.rule]


def bwd_bytes_per_token_head(w) -> int:
    """Reads dO, q, k, v and the gates; writes dq, dk, dv and the gate gradients."""
    return 4 * 2 * w.d + 3 * 2 * w.d + 2 * 4 * GATES[w.rule]


def fwd_flops_per_chunk_head(w) -> int:
    """E-form: A = QK^T, E = V - K S^T, o = QS^T + AE, G = E^T diag(w) K."""
    C, d = w.chunk, w.d
    f = 4 * C * C * d + 6 * C * d * d
    if w.rule == "muon":
        f += 6 * w.ns * d ** 3
    return f


def drop_in_bytes_per_chunk(d: int):
    """The drop-in scan's own I/O per chunk: forward reads U, K and the four
    gate scalars and writes S (3 d^2 fp32 + 16 B); the backward reads gS and
    writes dU, dK and the four scalar gradients, besides reading U, K, S and
    the gates again (5 d^2 fp32 + 32 B)."""
    return 3 * d * d * 4 + 16, 8 * d * d * 4 + 48


def drop_in_flops_per_chunk(rule: str, d: int, ns: int):
    """Minimal flops per chunk, forward and backward: delta 2 d^3 and 4 d^3,
    adam 2 d^3 and 6 d^3, muon (2 + 6 ns) d^3 and (6 + 16 ns) d^3."""
    fwd = {"delta": 2, "adam": 2, "muon": 2 + 6 * ns}[rule]
    bwd = {"delta": 4, "adam": 6, "muon": 6 + 16 * ns}[rule]
    return fwd * d ** 3, bwd * d ** 3


def drop_in_cpu_baseline(w, budget_s: float) -> dict:
    """The restated reference scan (scan_eager: fast_scan.py:72-95, float32
    torch on the host cores, autograd for the backward) on a bounded sample
    of the drop-in workload's heads; per-head time scaled to all B * H heads."""
    import torch
    from oracle import scan as osc

    threads = cpu_threads()
    torch.set_num_threads(threads)
    rid = {"delta": 0, "muon": 1, "adam": 2}[w.rule]
    N, d = w.T // w.chunk, w.d
    gen = torch.Generator().manual_seed(0)

    def sample(nh):
        X = torch.randn(nh, 1, N, d, d, generator=gen)
        K = (X @ X.transpose(-1, -2)) / (2 * d)
        U = torch.randn(nh, 1, N, d, d, generator=gen)
        gates = [0.9 + 0.1 * torch.rand(nh, 1, N, generator=gen) for _ in range(4)]
        xs = [t.requires_grad_(True) for t in [U, K] + gates]
        gS = torch.randn(nh, 1, N, d, d, generator=gen)
        t0 = time.perf_counter()
        S = osc.scan_forward(*xs, rid, w.ns)
        torch.autograd.grad(S, xs, gS, allow_unused=True)  # (the rule's unused gates)
        return time.perf_counter() - t0

    t1 = sample(1)  # warm-up and size the sample
    nh = max(1, min(w.B * w.H, int(budget_s / max(t1, 1e-3))))
    t = sample(nh) / nh
    total = t * w.B * w.H
    return {"value": w.B * w.T / total, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{nh} of {w.B * w.H} heads of the drop-in workload (N={N}, d={d}, rule {w.rule}), "
                      f"fwd+bwd, float32 scan_eager restatement with autograd; {t * 1e3:.0f} ms per head, "
                      f"scaled to all heads"}


def drop_in_leg(w, steps: int, warmup: int) -> dict:
    """The drop-in scan ``fast_state_scan(U, K, a, b, m, n, rule, ns)``
    (reference fast_scan.py:403-414) on the workload's chunk grid: B*H scans of
    T/chunk chunks of d x d fp32 ``U``, ``K`` (K = X X^T / 2d, X ~ N(0, 1)) and
    gate scalars in (0.9, 1), forward and forward + backward against a
    N(0, 1) state cotangent, timed with HIP events on the launch stream.
    Priced per chunk on the op's own I/O (3 d^2 fp32 + 4 scalars forward,
    5 d^2 + 8 scalars backward) against HBM, or for muon on its minimal flops
    ((2 + 6 ns) d^3 forward, (6 + 16 ns) d^3 backward) against bf16 MFMA."""
    import torch
    import fast_scan

    B, H, N, d = w.B, w.H, w.T // w.chunk, w.d
    rid = {"delta": 0, "muon": 1, "adam": 2}[w.rule]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    X = torch.randn(B * H * N, d, d, device=dev, generator=gen)
    K = torch.bmm(X, X.transpose(1, 2).contiguous()).div_(2 * d).view(B, H, N, d, d)
    del X
    U = torch.randn(B, H, N, d, d, device=dev, generator=gen)
    gates = [0.9 + 0.1 * torch.rand(B, H, N, device=dev, generator=gen) for _ in range(4)]
    gS = torch.randn(B, H, N, d, d, device=dev, generator=gen)
    xs = [t.requires_grad_(True) for t in [U, K] + gates]
    fast_scan.set_backend("triton")  # the native path, never eager
    fast_scan.set_precision("tf32")
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for e in evs:
            e[0].record(stream)
            fn()
            e[1].record(stream)
        torch.cuda.synchronize()
        return statistics.mean(e[0].elapsed_time(e[1]) for e in evs)

    try:
        with torch.no_grad():
            fwd_ms = timed(lambda: fast_scan.fast_state_scan(*xs, rid, w.ns))
        fb_ms = timed(lambda: torch.autograd.grad(fast_scan.fast_state_scan(*xs, rid, w.ns), xs, gS))
    finally:
        fast_scan.set_backend("auto")
    chunks = B * H * N

    def roof(ms, nbytes, flops):
        if w.rule == "muon":
            ach, peak, unit, bound = flops / (ms * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s", "mfma"
        else:
            ach, peak, unit, bound = nbytes / (ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", "hbm"
        return {"bound": bound, "achieved": ach, "peak": peak, "unit": unit, "frac": ach / peak,
                "alg_bytes": nbytes, "alg_flops": flops, "avg_us": ms * 1e3}

    fwd_b, fb_b = drop_in_bytes_per_chunk(d)
    fwd_f, bwd_f = drop_in_flops_per_chunk(w.rule, d, w.ns)
    fwd_flops, bwd_flops = fwd_f * chunks, bwd_f * chunks
    return {"op": "fast_state_scan", "shape": {"B": B, "H": H, "N": N, "d": d, "rule": w.rule, "ns": w.ns},
            "precision": ("tf32 (bf16x3 split products); fwd+bwd in exact float32 (adam keeps its moments)"
                          if w.rule == "adam" else "tf32 (bf16x3 split products)"),
            "fwd_tokens_per_s": B * N * w.chunk / (fwd_ms * 1e-3),
            "fwd_bwd_tokens_per_s": B * N * w.chunk / (fb_ms * 1e-3),
            "roofline_fwd": roof(fwd_ms, fwd_b * chunks, fwd_flops),
            "roofline_fwd_bwd": roof(fb_ms, fb_b * chunks, fwd_flops + bwd_flops)}


def bwd_flops_per_chunk_head(w) -> int:
    """Twice the forward's GEMMs; for muon the msign VJP adds (2 + 16 ns) d^3
    (in place of twice the forward Newton-Schulz)."""
    C, d = w.chunk, w.d
    f = 2 * (4 * C * C * d + 6 * C * d * d)
    if w.rule == "muon":
        f += (2 + 16 * w.ns) * d ** 3
    return f


LM_WORKLOAD = "lm_b8_t2048_muon"


def lm_line(args) -> dict:
    """The 12-layer GMDN stack (d_model 1024, 8 heads x 128, muon inner rule,
    ns = 3 -- the trainer's default, train_ablation.py:556-558), vocab 32000,
    B = 8, T = 2048, bf16 weights from the reference's N(0, 0.02) init,
    token ids uniform over the vocabulary, next-token cross entropy.  One
    step is the trainer's (train_ablation.py:458-474): forward, backward,
    gradient clipping at norm 1, then the outer Muon step on the hidden 2-D
    weights and AdamW on the rest (build_optimizers, :291-307, with the
    trainer's default rates).  The forward + backward alone and the
    inference forward are reported beside it.  End-to-end tokens/s only: the
    step is mostly library GEMMs, the muon core and the outer msign, so no
    single roofline applies."""
    import types

    import torch
    from gmdn_amd.mixer import LM
    from gmdn_amd.muon import build_optimizers

    B, T, vocab, d_model, layers, heads, ns = 8, 2048, 32000, 1024, 12, 8, 3
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = LM(vocab, d_model, layers, heads, "muon", ns_steps=ns).to(dev, torch.bfloat16)
    opts = build_optimizers(model, "muon", types.SimpleNamespace(muon_lr=0.02, adam_lr=4e-4, weight_decay=0.1))
    gen = torch.Generator(device=dev).manual_seed(0)
    idx = torch.randint(0, vocab, (B, T + 1), device=dev, generator=gen)
    stream = torch.cuda.current_stream(dev)

    def fwd_bwd():
        _, loss = model(idx[:, :-1], idx[:, 1:])
        loss.backward()
        for p in model.parameters():
            p.grad = None
        return loss

    def train_step():
        for opt in opts:
            opt.zero_grad(set_to_none=True)
        _, loss = model(idx[:, :-1], idx[:, 1:])
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        for opt in opts:
            opt.step()
        return loss

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        t0 = time.perf_counter()
        for e in evs:
            e[0].record(stream)
            fn()
            e[1].record(stream)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps, statistics.mean(e[0].elapsed_time(e[1]) for e in evs) / 1e3

    # steps of ~0.1 s: a few warm-up steps reach settled clocks
    steps, warmup = min(args.steps, 10), min(max(args.warmup, 1), 5)
    wall, ev = timed(train_step, steps, warmup)
    _, fb_ev = timed(fwd_bwd, steps, warmup)
    with torch.no_grad():
        _, fwd_ev = timed(lambda: model(idx[:, :-1]), steps, warmup)
    tokens = B * T
    return {
        "metric": METRIC, "value": tokens / wall, "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": wall * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": LM_WORKLOAD, "layers": layers, "d_model": d_model, "heads": heads,
                   "head_dim": d_model // heads, "rule": "muon", "ns": ns, "B": B, "T": T, "vocab": vocab,
                   "pass": "fwd+bwd+clip+optimizer (Muon + AdamW)", "global_batch": B, "seq_len": T,
                   "parallelism": "none"},
        "train_step_tokens_per_s": tokens / ev, "fwd_tokens_per_s": tokens / fwd_ev,
        "fwd_bwd_tokens_per_s": tokens / fb_ev,
        "step_us": {"train_step": ev * 1e6, "fwd_bwd": fb_ev * 1e6, "fwd_inference": fwd_ev * 1e6},
        "roofline": None, "roofline_note": "end-to-end stack: tokens/s only",
        "cpu_baseline": None,
    }


MSIGN_WORKLOAD = "outer_muon_lm12_d1024"


def msign_flops(rows: int, cols: int, steps: int) -> int:
    """Algorithmic flops of msign on one rows x cols matrix: per NS step
    X X^T (2 m^2 n), A A (2 m^3) and B X (2 m^2 n), m = min, n = max."""
    m, n = min(rows, cols), max(rows, cols)
    return steps * (4 * m * m * n + 2 * m ** 3)


def lm_hidden_shapes(layers=12, d_model=1024, heads=8, gates=3):
    """The 2-D weights the reference hands to Muon in the LM stack
    (train_ablation.py:291-300): per layer the qkv, gate, out and the two MLP
    projections (the embedding and the tied head go to AdamW)."""
    per = [(3 * d_model, d_model), (gates * heads, d_model), (d_model, d_model), (4 * d_model, d_model),
           (d_model, 4 * d_model)]
    return [s for _ in range(layers) for s in per]


def msign_line(args) -> dict:
    """One outer Muon step (train_ablation.py:271-288, ns_steps 5) over the
    LM's 60 hidden weights, fp32 parameters and N(0, 1) gradients; the
    updates of each shape are orthogonalised in one batched msign call."""
    import torch
    from gmdn_amd.muon import Muon

    dev = torch.device("cuda:0")
    shapes = lm_hidden_shapes()
    gen = torch.Generator(device=dev).manual_seed(0)
    params = [torch.nn.Parameter(torch.randn(s, device=dev, generator=gen) * 0.02) for s in shapes]
    for p in params:
        p.grad = torch.randn(p.shape, device=dev, generator=gen)
    opt = Muon(params, lr=0.02, momentum=0.95, nesterov=True, weight_decay=0.1, ns_steps=5)
    flops = sum(msign_flops(*s, 5) for s in shapes)
    stream = torch.cuda.current_stream(dev)
    for _ in range(min(max(args.warmup, 1), 5)):
        opt.step()
    torch.cuda.synchronize()
    steps = min(args.steps, 20)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for e in evs:
        e[0].record(stream)
        opt.step()
        e[1].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    ev = statistics.mean(e[0].elapsed_time(e[1]) for e in evs) / 1e3
    achieved = flops / ev / 1e12
    line = {
        "metric": METRIC, "value": flops / wall / 1e12, "unit": "TFLOP/s (msign, fp32-equivalent)", "n_gpus": 1,
        "steps": steps, "warmup": min(max(args.warmup, 1), 5), "ms_per_step": wall * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (split bf16 products)", "data": "synthetic",
        "config": {"workload": MSIGN_WORKLOAD, "matrices": len(shapes), "ns_steps": 5,
                   "shapes": sorted({f"{r}x{c}" for r, c in shapes}), "parallelism": "none"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / BF16_PEAK_TFLOPS, "traffic": None},
        "roofline_note": "algorithmic fp32-equivalent flops of the whole optimizer step (HIP events) against the "
                         "bf16 MFMA peak; three split products per multiply cap frac at 1/3",
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = msign_cpu_baseline(shapes, args.cpu_budget)
    return line


def msign_cpu_baseline(shapes, budget_s: float) -> dict:
    """The oracle's float32 msign (train_ablation.py:60-73 restated, torch on
    the host cores) on one layer's five weights, scaled to all layers."""
    import torch
    from oracle import muon as om

    torch.set_num_threads(cpu_threads())
    layer = shapes[:5]
    flops = sum(msign_flops(*s, 5) for s in layer)
    gen = torch.Generator().manual_seed(0)
    mats = [torch.randn(s, generator=gen) for s in layer]
    t0 = time.perf_counter()
    reps = 0
    while True:
        for M in mats:
            om.msign(M, 5)
        reps += 1
        if time.perf_counter() - t0 > min(budget_s, 30.0) or reps >= 3:
            break
    dt = (time.perf_counter() - t0) / reps
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s (msign, fp32-equivalent)",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"one layer's 5 hidden weights, float32 torch matmuls, {reps} repetition(s); "
                      f"a full optimizer step would take {dt * len(shapes) / len(layer) * 1e3:.0f} ms"}


def copy_calibration(nbytes: int) -> None:
    import torch
    # an elementwise kernel (MulFunctor) that reads nbytes and writes nbytes
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes}))


def measured_peaks(steps: int = 10) -> dict:
    """What this GPU sustains beside the datasheet peaks the rooflines use:
    HBM bandwidth of a device copy of 2 GiB (torch's elementwise copy: 2 GiB
    read + 2 GiB written per call) and dense bf16 MFMA throughput of an
    8192 x 8192 x 8192 torch.matmul (hipBLASLt), HIP events around each."""
    import torch
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(2)) for _ in range(steps)]
        for e in evs:
            e[0].record(stream)
            fn()
            e[1].record(stream)
        torch.cuda.synchronize()
        return statistics.median(e[0].elapsed_time(e[1]) for e in evs)

    n = 1 << 29  # float32 elements: 2 GiB
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    ms_copy = timed(lambda: dst.copy_(src))
    del src, dst
    m = 8192
    a = torch.randn(m, m, device=dev, dtype=torch.bfloat16)
    b = torch.randn(m, m, device=dev, dtype=torch.bfloat16)
    ms_mm = timed(lambda: torch.matmul(a, b))
    del a, b
    hbm = 2 * n * 4 / (ms_copy * 1e-3) / 1e9
    tf = 2 * m ** 3 / (ms_mm * 1e-3) / 1e12
    return {"hbm_copy_GBs": hbm, "hbm_datasheet_GBs": HBM_PEAK_GBS, "hbm_measured_frac": hbm / HBM_PEAK_GBS,
            "bf16_matmul_TFLOPs": tf, "bf16_datasheet_TFLOPs": BF16_PEAK_TFLOPS,
            "bf16_measured_frac": tf / BF16_PEAK_TFLOPS,
            "how": "2 GiB device copy (read + write) and an 8192^3 bf16 torch.matmul, medians of HIP events"}


def cpu_info() -> dict:
    """The host the CPU baseline ran on: lscpu model, sockets, physical
    cores, the process's CPU affinity and torch's thread count."""
    import subprocess

    import torch
    info = {"affinity_cpus": len(os.sched_getaffinity(0)), "torch_threads": torch.get_num_threads()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                kv[k.strip()] = v.strip()
        info["model"] = kv.get("Model name")
        sockets = int(kv.get("Socket(s)", "0") or 0)
        per = int(kv.get("Core(s) per socket", "0") or 0)
        info["sockets"] = sockets
        info["physical_cores"] = sockets * per if sockets and per else None
    except (OSError, ValueError, subprocess.SubprocessError):
        info["model"] = None
    return info


def cpu_threads() -> int:
    """Threads for the CPU baseline: every CPU of the process's affinity,
    capped by OMP_NUM_THREADS when the environment sets it (the host's CPU
    share per GPU)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(w, budget_s: float, with_bwd: bool, max_heads: int | None = None):
    """The CPU restatement of the reference matrix form in float32 (reference
    train_ablation.py:142-187 and fast_scan.py:72-95, autograd for backward),
    timed on this host's cores over the whole workload, or over its first
    ``max_heads`` heads of one batch row scaled to all B * H heads."""
    import dataclasses

    import torch
    from oracle import chunk as oc
    from gmdn_amd.workloads import make_inputs

    threads = cpu_threads()
    torch.set_num_threads(threads)
    ws = w if max_heads is None else dataclasses.replace(w, B=1, H=min(max_heads, w.H))
    scale = (w.B * w.H) / (ws.B * ws.H)
    inp = make_inputs(ws, seed=0, dtype=torch.float32, with_grad_out=True)
    rule = {"delta": 0, "muon": 1, "adam": 2}[w.rule]
    names = ("q", "k", "v", "beta", "g", "gmu", "gnu")

    def step():
        xs = [None if inp[n] is None else inp[n].clone().requires_grad_(with_bwd) for n in names]
        o = oc.mixer_core(*xs, rule=rule, ns=w.ns, C=w.chunk)
        if with_bwd:
            torch.autograd.grad(o, [x for x in xs if x is not None], inp["dO"])

    step()  # warm-up
    times, t_all = [], time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_all < budget_s and len(times) < 500):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > 3 * budget_s:
            break
    t = statistics.median(times) * scale
    what = (f"whole workload {w.name}" if max_heads is None else
            f"{ws.H} of {w.B * w.H} heads of {w.name}, scaled to all heads")
    return {"value": w.tokens / t, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{what} ({'fwd+bwd' if with_bwd else 'fwd'}), float32 matrix form, "
                      f"median of {len(times)} runs ({t * 1e3:.0f} ms for the workload)",
            "host": cpu_info()}


def chunk_leg(w, steps: int, warmup: int, with_bwd: bool) -> dict:
    """Time the fused mixer core ``chunk_scan`` on workload ``w``: the
    training step (forward with the state checkpoint, then the backward)
    when ``with_bwd``, and the inference forward, with HIP events on the
    launch stream inside the timed regions.  Returns the timings and the
    roofline objects of the backward (the dominant part of a step) and of
    the inference forward."""
    import torch
    from gmdn_amd import chunk, profiling
    from gmdn_amd.workloads import make_inputs

    dev = torch.device("cuda:0")
    inp = make_inputs(w, seed=0, device=dev, with_grad_out=True)
    names = ("q", "k", "v", "beta", "g", "gmu", "gnu")
    xs = [inp[n] if inp[n] is None else inp[n].detach().requires_grad_(with_bwd) for n in names]
    grads_of = [x for x in xs if x is not None]
    dO = inp["dO"]
    stream = torch.cuda.current_stream(dev)

    def fwd():
        return chunk.chunk_scan(*xs, rule=w.rule, ns=w.ns)

    out = {}
    if with_bwd:
        def step(ev=None):
            if ev is not None:
                ev[0].record(stream)
            o = fwd()
            if ev is not None:
                ev[1].record(stream)
            torch.autograd.grad(o, grads_of, dO)
            if ev is not None:
                ev[2].record(stream)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            step(evs[i])
        torch.cuda.synchronize()
        out["ms_step"] = (time.perf_counter() - t0) * 1e3 / steps
        # the forward launch (which also writes the state checkpoint) and the backward
        out["fwd_train_ms"] = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
        out["bwd_ms"] = statistics.mean(e[1].elapsed_time(e[2]) for e in evs)

    # inference forward (no state checkpoint), timed the same way
    fwd_evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(2)) for _ in range(steps)]
    with torch.no_grad():
        for _ in range(warmup):
            fwd()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for e in fwd_evs:
            e[0].record(stream)
            fwd()
            e[1].record(stream)
        torch.cuda.synchronize()
        out["fwd_ms"] = (time.perf_counter() - t1) * 1e3 / steps
    out["fwd_kernel_ms"] = statistics.mean(e[0].elapsed_time(e[1]) for e in fwd_evs)

    # The same step captured into one HIP graph and replayed: the launches
    # cost no host time per step.  Delta and adam only (their capture is
    # tested; the muon path is timed eagerly).  The capture's first replay
    # must reproduce an eager step bit for bit; if it does not, the line says
    # so in ``graph_check`` and keeps the eager times.
    if w.rule in ("delta", "adam"):
        def graph_of(fn):
            side = torch.cuda.Stream()
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                for _ in range(2):
                    fn()
            stream.wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                outs = fn()
            torch.cuda.synchronize()
            ref = fn()
            g.replay()
            torch.cuda.synchronize()
            if not all(torch.equal(a, b) for a, b in zip(outs, ref)):
                print(f"bench.py: {w.name}: a graph replay differs from the eager step; eager times kept",
                      file=sys.stderr)
                out["graph_check"] = "replay differs from the eager step"
                return None
            out.setdefault("graph_check", "replays equal the eager step bit for bit")
            return g

        def replay_ms(g):
            if g is None:
                return None
            for _ in range(warmup):
                g.replay()
            torch.cuda.synchronize()
            t = time.perf_counter()
            for _ in range(steps):
                g.replay()
            torch.cuda.synchronize()
            return (time.perf_counter() - t) * 1e3 / steps

        def inference():
            with torch.no_grad():
                return (fwd(),)

        gf = replay_ms(graph_of(inference))
        if gf is not None:
            out["graph_fwd_ms"] = gf
        if with_bwd:
            # fresh leaves: the eager steps above ran on another stream, and
            # leaves with that autograd history make the capture add
            # cross-stream waits
            gxs = [None if x is None else x.detach().clone().requires_grad_(True) for x in xs]
            gwrt = [x for x in gxs if x is not None]

            def train():
                o = chunk.chunk_scan(*gxs, rule=w.rule, ns=w.ns)
                return (o,) + tuple(torch.autograd.grad(o, gwrt, dO))

            gs = replay_ms(graph_of(train))
            if gs is not None:
                out["graph_ms_step"] = gs

    units = w.B * w.H * w.T
    rid = {"delta": 0, "muon": 1, "adam": 2}[w.rule]

    def roof(kernel, alg_bytes, alg_flops, ms, traffic_file):
        if w.rule == "muon":
            bound, ach, peak, unit = "mfma", alg_flops / (ms * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
        else:
            bound, ach, peak, unit = "hbm", alg_bytes / (ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        traffic = profiling.read_traffic(os.path.join(ROOT, "profiles", traffic_file))
        return {"kernel": kernel, "bound": bound, "achieved": ach, "peak": peak, "unit": unit,
                "frac": ach / peak, "traffic": traffic, "avg_launch_us": ms * 1e3,
                "alg_bytes": alg_bytes, "alg_flops": alg_flops}

    chunks = w.B * w.H * (w.T // w.chunk)
    fwd_name = (f"chunk_fwd_muon<{w.d}> + chunk_out<{w.d}>" if rid == 1
                else f"chunk_fwd_rows<{w.d},0>" if rid == 0
                else f"chunk_fwd_adam16<{w.d}>" if w.d == 64 else f"chunk_fwd<{w.d},{rid}>")
    out["roofline_fwd"] = roof(fwd_name, fwd_bytes_per_token_head(w) * units,
                               fwd_flops_per_chunk_head(w) * chunks, out["fwd_kernel_ms"],
                               f"chunk_fwd_{w.name}_traffic.md")
    if with_bwd:
        if rid == 1:
            bwd_name = f"chunk_bwd_muon_pipe<{w.d}> (chunk_prep, muon_pre/x3, chunk_bwd_tok stages)"
        elif rid == 0:
            bwd_name = f"chunk_bwd_dscan<{w.d}> + chunk_bwd_pair<{w.d}>"
        elif w.d == 128:
            bwd_name = "chunk_prep<128,2> + scan_bwd_rows<128,2> (fp32) + chunk_bwd_tok<128,2>"
        else:
            bwd_name = f"chunk_bwd_ascan<{w.d}> + chunk_bwd_tok_range<{w.d},{rid}> (2 segments, two streams)"
        out["roofline"] = roof(bwd_name, bwd_bytes_per_token_head(w) * units,
                               bwd_flops_per_chunk_head(w) * chunks, out["bwd_ms"],
                               f"chunk_bwd_{w.name}_traffic.md")
    return out


def config_leg(name: str, steps: int, warmup: int, cpu_budget: float | None, with_bwd: bool,
               max_heads: int | None = None) -> dict:
    """One sub-object of the default line: another configuration of the
    fused core, its tokens/s, rooflines and (when a budget is given) a CPU
    baseline on a bounded sample."""
    from gmdn_amd.workloads import WORKLOADS

    w = WORKLOADS[name]
    r = chunk_leg(w, steps, warmup, with_bwd)
    leg = {"workload": name, "rule": w.rule, "B": w.B, "H": w.H, "T": w.T, "d": w.d, "ns": w.ns if w.rule == "muon" else None,
           "fwd_tokens_per_s": w.tokens / (r["fwd_ms"] * 1e-3),
           "step_us": {"fwd_inference": r["fwd_kernel_ms"] * 1e3},
           "roofline_fwd": r["roofline_fwd"]}
    if "graph_fwd_ms" in r:
        leg["step_us"]["fwd_inference_graph"] = r["graph_fwd_ms"] * 1e3
    if "graph_check" in r:
        leg["graph_check"] = r["graph_check"]
    if with_bwd:
        leg["fwd_bwd_tokens_per_s"] = w.tokens / (r.get("graph_ms_step", r["ms_step"]) * 1e-3)
        leg["step_us"].update(fwd_with_checkpoint=r["fwd_train_ms"] * 1e3, bwd=r["bwd_ms"] * 1e3,
                              train_step_eager=r["ms_step"] * 1e3)
        if "graph_ms_step" in r:
            leg["step_us"]["train_step_graph"] = r["graph_ms_step"] * 1e3
        leg["roofline"] = r["roofline"]
    if cpu_budget:
        leg["cpu_baseline"] = cpu_baseline(w, cpu_budget, with_bwd, max_heads)
    return leg


def wy_leg(steps: int, warmup: int) -> dict:
    """The exact WY/UT mode (``wy_scan``) at the headline shape B=4, H=16,
    T=4096, d=128 (bf16 q, k, v): inference forward and forward + backward,
    eager launches, HIP events on the launch stream.  Priced on the same
    algorithmic bytes as the fused core (the op's inputs and outputs)."""
    import torch
    from gmdn_amd import wy
    from gmdn_amd.workloads import WORKLOADS, make_inputs

    w = WORKLOADS[DEFAULT_WORKLOAD]
    dev = torch.device("cuda:0")
    inp = make_inputs(w, seed=0, device=dev, with_grad_out=True)
    xs = [inp[n].detach().requires_grad_(True) for n in ("q", "k", "v", "beta", "g")]
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(2)) for _ in range(steps)]
        for e in evs:
            e[0].record(stream)
            fn()
            e[1].record(stream)
        torch.cuda.synchronize()
        return statistics.mean(e[0].elapsed_time(e[1]) for e in evs)

    def fwd():
        with torch.no_grad():
            wy.wy_scan(*xs)

    def fwd_bwd():
        o = wy.wy_scan(*xs)
        torch.autograd.grad(o, xs, inp["dO"])

    ms_f, ms_fb = timed(fwd), timed(fwd_bwd)
    units = w.B * w.H * w.T
    bf, bb = fwd_bytes_per_token_head(w) * units, (fwd_bytes_per_token_head(w) + bwd_bytes_per_token_head(w)) * units
    return {"workload": "wy_" + DEFAULT_WORKLOAD, "B": w.B, "H": w.H, "T": w.T, "d": w.d,
            "fwd_tokens_per_s": w.tokens / (ms_f * 1e-3), "fwd_bwd_tokens_per_s": w.tokens / (ms_fb * 1e-3),
            "step_us": {"fwd_inference": ms_f * 1e3, "fwd_bwd": ms_fb * 1e3},
            "hbm_frac_fwd": bf / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "hbm_frac_fwd_bwd": bb / (ms_fb * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "kernels": "wy_prep + scan_fwd_rows8<128,0> + wy_out; bwd: wy_gs + scan_bwd_rows8<128,0> + "
                       "wy_ka + wy_kb + wy_kc1 + wy_kc2 (split-bf16 MFMA throughout; T by float32 "
                       "forward substitution)"}


def main(argv=None):
    args = parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py measures one GPU only; --gpus {max(args.gpus, world)} is not supported. "
              f"The scan shards over (batch, head) with no exchange between GPUs, so the job's "
              f"throughput is the one-GPU figure times the GPU count.", file=sys.stderr)
        return 2

    import torch
    from gmdn_amd import _native, chunk, profiling
    from gmdn_amd.workloads import WORKLOADS, make_inputs

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU (no HIP device visible)")
    _native.load()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return 0

    if args.workload == LM_WORKLOAD:
        print(json.dumps(lm_line(args)), flush=True)
        return 0
    if args.workload == MSIGN_WORKLOAD:
        print(json.dumps(msign_line(args)), flush=True)
        return 0
    w = WORKLOADS[args.workload]
    with_bwd = chunk.backward_supported(w.rule, w.d) and not args.fwd_only
    r = chunk_leg(w, args.steps, args.warmup, with_bwd)
    # the graph-replayed training step where the rule's capture is built,
    # else eager; the inference forward eager (one kernel: a graph replay
    # adds more than the launch it saves)
    ms_fwd = r["fwd_ms"]
    ms_fb = r.get("graph_ms_step", r["ms_step"]) if with_bwd else None
    ms_step = ms_fb if with_bwd else ms_fwd
    line = {
        "metric": METRIC,
        "value": w.tokens / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": w.name, "rule": w.rule, "B": w.B, "H": w.H, "T": w.T, "d": w.d,
                   "chunk": w.chunk, "pass": "fwd+bwd" if with_bwd else "fwd",
                   "state": "fp32", "global_batch": w.B, "seq_len": w.T, "parallelism": "none"},
        "fwd_tokens_per_s": w.tokens / (ms_fwd * 1e-3),
        "fwd_bwd_tokens_per_s": w.tokens / (ms_fb * 1e-3) if with_bwd else None,
        "timing": ("fwd+bwd: HIP graph replays, fwd: eager launches" if with_bwd and "graph_ms_step" in r
                   else "eager launches"),
        "graph_check": r.get("graph_check"),
        "step_us": {"fwd_with_checkpoint": r["fwd_train_ms"] * 1e3 if with_bwd else None,
                    "bwd": r["bwd_ms"] * 1e3 if with_bwd else None,
                    "fwd_inference": r["fwd_kernel_ms"] * 1e3,
                    "train_step_eager": r["ms_step"] * 1e3 if with_bwd else None,
                    "train_step_graph": r["graph_ms_step"] * 1e3 if "graph_ms_step" in r else None,
                    "fwd_inference_eager": r["fwd_ms"] * 1e3,
                    "fwd_inference_graph": r["graph_fwd_ms"] * 1e3 if "graph_fwd_ms" in r else None},
        "roofline": r["roofline"] if with_bwd else r["roofline_fwd"],
        "roofline_fwd": r["roofline_fwd"],
    }
    if not (args.no_drop_in or args.fwd_only):
        line["drop_in"] = drop_in_leg(w, min(args.steps, 20), max(args.warmup, 1))
        if not args.no_cpu_baseline:
            line["drop_in"]["cpu_baseline"] = drop_in_cpu_baseline(w, args.cpu_budget / 2)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_budget, with_bwd)
    if args.workload == DEFAULT_WORKLOAD and not (args.fwd_only or args.no_configs):
        # the other configurations: muon (forward, and forward + backward),
        # adam (forward, forward + backward) and the 12-layer LM's training step
        budget = None if args.no_cpu_baseline else args.cpu_budget / 2
        steps = min(args.steps, 10)
        line["configs"] = {
            "muon_b2_h16_t8192_d128": config_leg("muon_b2_h16_t8192_d128", steps, min(max(args.warmup, 1), 5), budget,
                                                 True, max_heads=2),
            "adam_b2_h8_t4096_d64": config_leg("adam_b2_h8_t4096_d64", args.steps, args.warmup, budget, True),
        }
        line["configs"]["wy_" + DEFAULT_WORKLOAD] = wy_leg(min(args.steps, 10), min(max(args.warmup, 1), 5))
        line["measured_peaks"] = measured_peaks()
        lm = lm_line(args)
        line["configs"][LM_WORKLOAD] = {k: lm[k] for k in ("value", "unit", "ms_per_step", "config",
                                                           "train_step_tokens_per_s", "fwd_tokens_per_s",
                                                           "fwd_bwd_tokens_per_s", "step_us", "roofline_note")}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
