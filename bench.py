#!/usr/bin/env python3
"""Benchmark: causal RACE layer forward+backward tokens/s on one MI355X.

Workload (the metric's "N=1M causal" case): one RACE
attention layer core, B=1, H=8, N=2^20 tokens, d=64, bf16 inputs/outputs with
fp32 accumulation, K=4 hash bits (16 buckets per table), L=8 tables, M=1,
temperature sqrt(d).  Inputs are synthetic: Q, K, V ~ N(0,1) row-normalised to
unit L2 norm, dO ~ N(0,1), hyperplanes ~ N(0,1) (seeds 0 and 1234), resident in
HBM before the timed region.

A step is one race_fwd + race_bwd through the C ABI (six kernels: forward
segment reduce, scan, output; backward reduce, scan, output).  Every kernel is
enqueued on torch's current stream with HIP events between them, so the
per-kernel average durations (and the roofline of the dominant kernel) come
from the timed region itself.  The CPU baseline times the reference's own CPU
path (aten + kernels/cpu/race_pref.cpp compiled from source) on a bounded
sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--seq N] [--no-cpu-baseline] [--no-max-n]
                    [--copy-calib MIB] [--workload c4|c5] [--mode f1|global]

--workload c5 times the attention core of BASELINE configs[4] instead (the
GPT-style decoder's layer: causal, K=8 so 256 buckets per table, L=4, M=2
estimators with independent hyperplanes over Q/K/V expanded with stride 0,
B=8, 12 heads, N=8192, d=64, bf16): 1024 buckets run as 8 bucket slices.
The default (c4) line is the headline metric.

--mode probs times the bucket probabilities as an output (race_probs +
race_probs_bwd of Q, fp32 P [H,T,L*2^K] per step): HBM-bound, so its line
reports GB/s of the compulsory bytes (read x, write P; read x and dP, write dx).

--mode global times the globally normalised causal mode (CausalRACEAttention,
misc/elsaa_causal_complete.py:438-586) on the same workload with beta = 1:
race_fwd_global + race_bwd_global (the backward's first phase also runs the
per-token prologue kernel).  Its CPU baseline is the fp64 C restatement under
oracle/ (the reference's F2 CPU path is aten einsums), on a bounded sample.

--workload c3-step / c5-step time one full training step of the models of
BASELINE configs[2] and configs[4] with RACE blocks (forward, backward,
AdamW; bf16 autocast over fp32 weights): the ViT encoder (6 layers, d=384,
6 heads, MLP 1536, non-causal K=2 L=5 M=1, batch 64 x 785 tokens of 28x28
images, 10 classes) and the GPT decoder (12 layers, d=768, 12 heads, MLP
3072, vocab 50257, causal K=8 L=4 M=2, batch 8 x 8192 token ids).  Value is
tokens/s of the step.

--copy-calib MIB ends the run with one device-to-device copy of MIB MiB, the
known-size kernel against which rocprofv3's FETCH_SIZE / WRITE_SIZE counters
are scaled when the HBM traffic of the operator's kernels is measured.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "RACE layer fwd+bwd tokens/s at N=1M causal; % of HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16

PHASES = (("fwd_reduce", "fwd", 1), ("fwd_scan", "fwd", 2), ("fwd_out", "fwd", 4),
          ("bwd_reduce", "bwd", 1), ("bwd_scan", "bwd", 2), ("bwd_out", "bwd", 4))


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seq", type=int, default=1 << 20, help="tokens per sequence (default 2^20)")
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=65536, help="tokens of one head per timed CPU run")
    ap.add_argument("--no-max-n", dest="max_n", action="store_false",
                    help="skip the bisection of the longest sequence that fits in HBM (run by default for c4 f1)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="finish with a device-to-device copy of MIB MiB (PMC calibration)")
    ap.add_argument("--workload", choices=("c4", "c5", "c3-step", "c5-step"), default="c4")
    ap.add_argument("--mode", choices=("f1", "global", "probs"), default="f1",
                    help="f1: per-bucket normalisation (headline); global: one normaliser per token; "
                         "probs: the bucket probabilities of Q as an output, forward + backward")
    return ap.parse_args()


def make_inputs(B, T, H, D, L, K, dev, seed=0, M=1):
    """Q, K, V [M,B,T,H,D] (one [B,T,H,D] tensor expanded over M with stride
    0, as the modules pass them), dO [M,B,T,H,D], planes [M,L,K,D] fp32."""
    import torch
    g = torch.Generator(device="cpu").manual_seed(seed)
    out = []
    for _ in range(3):  # Q, K, V generated in chunks to bound host memory
        x = torch.empty(B, T, H, D, dtype=torch.bfloat16, device=dev)
        step = 1 << 18
        for t0 in range(0, T, step):
            t1 = min(T, t0 + step)
            c = torch.randn(B, t1 - t0, H, D, generator=g)
            x[:, t0:t1] = torch.nn.functional.normalize(c, dim=-1).to(torch.bfloat16).to(dev)
        out.append(x.unsqueeze(0).expand(M, -1, -1, -1, -1))
    do = torch.empty(M, B, T, H, D, dtype=torch.bfloat16, device=dev)
    step = 1 << 18
    for m in range(M):
        for t0 in range(0, T, step):
            t1 = min(T, t0 + step)
            do[m, :, t0:t1] = torch.randn(B, t1 - t0, H, D, generator=g).to(torch.bfloat16).to(dev)
    gp = torch.Generator(device="cpu").manual_seed(1234)
    planes = torch.randn(M, L, K, D, generator=gp).to(dev)
    return out[0], out[1], out[2], do, planes


class Step:
    """Pre-allocated buffers and descriptors for one fwd+bwd through the C ABI."""

    def __init__(self, q, k, v, do, planes, L, K):
        import torch
        from race_attention_amd import _lib
        from race_attention_amd.functional import make_desc, _strides4
        self.lib = _lib.load()
        self.q, self.k, self.v, self.do, self.planes = q, k, v, do, planes.float().contiguous()
        self.d = make_desc(q, k, v, self.planes, L=L, K=K, causal=True, eps=1e-6, inv_temp=1.0 / math.sqrt(q.shape[-1]))
        new = lambda: torch.empty(q.shape, dtype=q.dtype, device=q.device)  # noqa: E731  (q may be an M-expand)
        self.out = new()
        self.dq, self.dk, self.dv = new(), new(), new()
        self.d.o_stride = _strides4(self.out)
        self.d.do_stride = _strides4(do)
        self.d.g_stride = _strides4(self.dq)
        ref = ctypes.byref(self.d)
        sb, fw, bw = (self.lib.race_state_bytes(ref), self.lib.race_fwd_workspace_bytes(ref),
                      self.lib.race_bwd_workspace_bytes(ref))
        if sb == 0:
            _lib.check(-1, "race_state_bytes")
        self.state = torch.empty(sb, dtype=torch.uint8, device=q.device)
        self.ws = torch.empty(max(fw, bw), dtype=torch.uint8, device=q.device)
        self.sizes = (sb, bw)  # state and backward-workspace bytes (scan_bytes)
        self.git = torch.empty((), dtype=torch.float32, device=q.device)
        self.check = _lib.check
        P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        self.fargs = (P(q), P(k), P(v), P(self.planes), P(self.out), P(self.state), P(self.ws),
                      ctypes.c_size_t(self.ws.numel()))
        self.bargs = (P(q), P(k), P(v), P(self.planes), P(do), P(self.state), P(self.dq), P(self.dk), P(self.dv),
                      P(self.git), P(self.ws), ctypes.c_size_t(self.ws.numel()))

    def run(self, phases=0, which="both"):
        import torch
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.d.phases = phases
        if which in ("both", "fwd"):
            self.check(self.lib.race_fwd(ctypes.byref(self.d), *self.fargs, st), "race_fwd")
        if which in ("both", "bwd"):
            self.check(self.lib.race_bwd(ctypes.byref(self.d), *self.bargs, st), "race_bwd")
        self.d.phases = 0


class GlobalStep(Step):
    """One race_fwd_global + race_bwd_global (beta = 1, no upstream den gradient)."""

    def __init__(self, q, k, v, do, planes, L, K):
        import torch
        super().__init__(q, k, v, do, planes, L, K)
        self.d.inv_temp = 1.0
        M, B, T, H, _ = q.shape
        self.den = torch.empty((M, B, H, T), dtype=torch.float32, device=q.device)
        ref = ctypes.byref(self.d)
        fw, bw = self.lib.race_fwd_global_workspace_bytes(ref), self.lib.race_bwd_global_workspace_bytes(ref)
        self.ws = torch.empty(max(fw, bw), dtype=torch.uint8, device=q.device)
        P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        self.fargs = (P(q), P(k), P(v), P(self.planes), P(self.out), P(self.den), P(self.state), P(self.ws),
                      ctypes.c_size_t(self.ws.numel()))
        self.bargs = (P(q), P(k), P(v), P(self.planes), P(self.out), P(self.den), P(do), None, P(self.state),
                      P(self.dq), P(self.dk), P(self.dv), P(self.git), P(self.ws), ctypes.c_size_t(self.ws.numel()))

    def run(self, phases=0, which="both"):
        import torch
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.d.phases = phases
        if which in ("both", "fwd"):
            self.check(self.lib.race_fwd_global(ctypes.byref(self.d), *self.fargs, st), "race_fwd_global")
        if which in ("both", "bwd"):
            self.check(self.lib.race_bwd_global(ctypes.byref(self.d), *self.bargs, st), "race_bwd_global")
        self.d.phases = 0


class ProbsStep:
    """One race_probs + race_probs_bwd of x = Q (inv_temp 1/sqrt(d))."""

    def __init__(self, q, planes, L, K):
        import torch
        from race_attention_amd import _lib
        from race_attention_amd.functional import _probs_desc, _strides4
        self.lib, self.check = _lib.load(), _lib.check
        M, B, T, H, D = q.shape
        self.planes = planes.float().contiguous()
        self.d = _probs_desc(q, self.planes, L, K, 1.0 / math.sqrt(D))
        self.P = torch.empty((M, B, H, T, L << K), dtype=torch.float32, device=q.device)
        self.dP = torch.randn(self.P.shape, generator=torch.Generator(device=q.device).manual_seed(7),
                              device=q.device)
        self.dx = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        self.d.g_stride = _strides4(self.dx)
        self.ws = torch.empty(max(self.lib.race_probs_bwd_workspace_bytes(ctypes.byref(self.d)), 16),
                              dtype=torch.uint8, device=q.device)
        self.git = torch.empty((), dtype=torch.float32, device=q.device)
        P_ = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        self.fargs = (P_(q), P_(self.planes), P_(self.P))
        self.bargs = (P_(q), P_(self.planes), P_(self.dP), P_(self.dx), P_(self.git), P_(self.ws),
                      ctypes.c_size_t(self.ws.numel()))

    def run(self, phases=0, which="both"):
        import torch
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        if which in ("both", "fwd"):
            self.check(self.lib.race_probs(ctypes.byref(self.d), *self.fargs, st), "race_probs")
        if which in ("both", "bwd"):
            self.check(self.lib.race_probs_bwd(ctypes.byref(self.d), *self.bargs, st), "race_probs_bwd")


def probs_main(args, q, planes, L, K, wl, T, B, H, D, M):
    """--mode probs: the two probability kernels, each timed with HIP events."""
    import torch
    step = ProbsStep(q, planes, L, K)
    for _ in range(args.warmup):
        step.run()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for s in range(args.steps):
        ev[s][0].record()
        step.run(which="fwd")
        ev[s][1].record()
        step.run(which="bwd")
        ev[s][2].record()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    fwd = statistics.mean(ev[s][0].elapsed_time(ev[s][1]) for s in range(args.steps))
    bwd = statistics.mean(ev[s][1].elapsed_time(ev[s][2]) for s in range(args.steps))
    th = M * B * T * H
    S = L << K
    fb, bb = th * (D * 2 + S * 4), th * (D * 2 + S * 4 + D * 2)
    res = {"metric": "bucket probabilities fwd+bwd tokens/s (HBM-bound)", "value": round(B * T / (ms / 1e3), 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16 in, fp32 P",
           "data": "synthetic (unit-L2 N(0,1) Q, N(0,1) dP and hyperplanes)",
           "config": {"workload": f"{wl}, bucket probabilities of Q: B={B} H={H} N={T} d={D} K={K} L={L} M={M}"},
           "kernels": {"probs": {"ms": round(fwd, 4), "algorithmic_GBs": round(fb / (fwd * 1e-3) / 1e9, 1)},
                       "probs_bwd": {"ms": round(bwd, 4), "algorithmic_GBs": round(bb / (bwd * 1e-3) / 1e9, 1)}},
           "roofline": {"bound": "hbm", "kernel": "probs_bwd", "achieved": round(bb / (bwd * 1e-3) / 1e9, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(bb / (bwd * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "traffic": None}}
    print(json.dumps(res), flush=True)


def model_step_main(args):
    """--workload c3-step / c5-step: one training step of the full model."""
    import torch
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    if args.workload == "c3-step":
        from race_attention_amd.vit import VisionTransformer
        cfg = dict(img_size=28, patch_size=1, num_channels=1, embed_dim=384, num_heads=6, transformer_units=6,
                   drop_rate=0.1, qkv_bias=False, K=2, L=5, M=1, num_classes=10)
        model = VisionTransformer(cfg).to(dev)
        B, T = 64, 28 * 28 + 1
        x = torch.randn(B, 1, 28, 28, device=dev)
        y = torch.randint(0, 10, (B,), device=dev)
        loss_fn = lambda out: torch.nn.functional.cross_entropy(out.float(), y)  # noqa: E731
        wl = "C3 ViT training step (6 RACE blocks, d=384, 6 heads, K=2 L=5 M=1, non-causal), AdamW"
    else:
        from race_attention_amd.lm import LMModel
        cfg = dict(vocab_size=50257, context_length=8192, emb_dim=768, n_heads=12, n_layers=12, drop_rate=0.1,
                   qkv_bias=False, K=8, L=4, M=2)
        model = LMModel(cfg).to(dev)
        B, T = 8, 8192
        x = torch.randint(0, 50257, (B, T), device=dev)
        y = torch.randint(0, 50257, (B, T), device=dev)
        loss_fn = lambda out: torch.nn.functional.cross_entropy(out.flatten(0, 1), y.flatten())  # noqa: E731
        wl = "C5 GPT training step (12 causal RACE blocks, d=768, 12 heads, K=8 L=4 M=2, vocab 50257), AdamW"
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    print(f"bench: {wl}: {sum(p.numel() for p in model.parameters())} parameters", file=sys.stderr, flush=True)

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            out = model(x)
        loss_fn(out).backward()
        opt.step()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print("bench: warm-up done", file=sys.stderr, flush=True)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    res = {"metric": "training step tokens/s (full model, RACE attention)", "value": round(B * T / (ms / 1e3), 1),
           "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
           "gpu_ms_per_step": round(e0.elapsed_time(e1) / args.steps, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16 autocast, fp32 weights",
           "data": "synthetic (N(0,1) images / uniform token ids, random-init weights)",
           "config": {"workload": wl, "global_batch": B, "seq_len": T}}
    print(json.dumps(res), flush=True)


def cpu_baseline_global(sample_T, H, D=64, L=8, K=4, reps=3):
    """The fp64 C restatement (oracle/race_oracle.c) of the globally normalised
    mode, fwd+bwd, on one batch row of H heads x sample_T tokens (OpenMP over
    the H streams); median of reps runs, as tokens/s."""
    import numpy as np
    from oracle import race_oracle as ro
    rng = np.random.default_rng(0)
    x = [rng.standard_normal((1, 1, sample_T, H, D)) for _ in range(4)]
    x[:3] = [a / np.linalg.norm(a, axis=-1, keepdims=True) for a in x[:3]]
    pl = rng.standard_normal((1, L, K, D))
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        ro.race_global_forward(x[0], x[1], x[2], pl, beta=1.0)
        ro.race_global_backward(x[0], x[1], x[2], x[3], pl, beta=1.0)
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    return {"value": round(sample_T / t, 1), "unit": "tokens/s", "cores": min(H, os.cpu_count() or 1), "kind": "port",
            "sample": f"1 batch row x {H} heads x {sample_T} tokens of the same workload, fwd+bwd in the fp64 C "
                      f"restatement (oracle/race_oracle.c, OpenMP over the {H} head streams), median of {reps} runs; "
                      f"{t:.2f} s per run"}


def algorithmic_bytes(name, tok_heads, D, esize, mode="f1"):
    """Compulsory HBM bytes of each kernel: token tensors it must read/write
    (global mode: the backward's first phase also reads O for dL/d den)."""
    unit = tok_heads * D * esize
    units = {"fwd_reduce": 2, "fwd_out": 4, "bwd_reduce": 5 if mode == "f1" else 6, "bwd_out": 6}
    return units.get(name, 0) * unit


def _a16(x):
    return (x + 15) // 16 * 16


def scan_bytes(state_bytes, bwd_ws_bytes, N, T, L, K, D=64):
    """HBM bytes of the two bf16 F1 scans, from the library's buffer sizes.

    k_fwd_scan reads the fp64 per-segment sums [N][fnseg][Spad][D+1] and
    writes the exclusive prefixes [N][fnseg+1][Spad][D+1] (the state);
    k_bwd_scan reads the fp32 (U, alpha) sums [N][nseg][Spad][D+1] and writes
    their suffixes, the same size.  The segment counts follow from the sizes:
    state = N (fnseg+1) Spad (D+1) 8 bytes; backward workspace = 2 N nseg
    Spad (D+1) 4 + align16(16 N nseg nslice), plus, for bucket slices, the dV
    partials [nslice][N][T][D] bf16 and the two dQ / dK d(projection) partial
    buffers [nslice][N][T][8] (fp32 for 8-bit hashes).  Covers the
    single-slice plans (K <= 4, L 2^K <= 128) and 8-bit hashes; None otherwise.
    Returns (fwd_scan bytes, bwd_scan bytes, fnseg, nseg)."""
    S = L << K
    if K <= 4 and S <= 128:
        spad = (S + 31) // 32 * 32
        spad, nslice, parts = (128 if spad == 96 else spad), 1, 0
    elif K == 8:
        nslice = -(-S // 128)
        spad = nslice * 128
        parts = _a16(nslice * N * T * D * 2) + 2 * _a16(nslice * N * T * 8 * 4)
    else:
        return None
    blk = spad * (D + 1)
    fnseg = state_bytes // (N * blk * 8) - 1
    nseg = (bwd_ws_bytes - parts) // (8 * N * blk + 16 * N * nslice)
    if state_bytes != N * (fnseg + 1) * blk * 8 or \
            bwd_ws_bytes != 8 * N * nseg * blk + _a16(16 * N * nseg * nslice) + parts:
        return None
    return (2 * fnseg + 1) * N * blk * 8, 2 * N * nseg * blk * 4, fnseg, nseg


def mfma_figures(ms, tok_heads, D, L, K, workload, T):
    """Matrix-core figures of the aggregation kernel (k_fwd_reduce: the
    segment sums S = P_K^T [V, 1] with the K projection that feeds them).
    algorithmic: 2 S (d+1) + 2 d L K flops per token-head over the kernel's
    HIP-event time, against the dense bf16 peak.  counter: the share of
    SIMD cycles the matrix cores were busy (SQ_VALU_MFMA_BUSY_CYCLES over the
    launch's SIMD cycles), read from the committed rocprofv3 summary of the
    same kernel and workload when there is one (every issued MFMA counts,
    including transposes and hi/lo splits)."""
    S = L << K
    per_th = 2 * S * (D + 1) + 2 * D * L * K
    tf = tok_heads * per_th / (ms * 1e-3) / 1e12
    out = {"kernel": "fwd_reduce", "what": "bucket aggregation P_K^T [V, 1] per segment (+ K projection)",
           "algorithmic_flops_per_token_head": per_th, "algorithmic_achieved": round(tf, 2),
           "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "algorithmic_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 5),
           "counter_busy_frac": None}
    cfile = os.path.join(ROOT, "profiles", f"mfma_fwd_reduce_{workload}.txt")
    if os.path.exists(cfile) and (workload != "c4" or T == 1 << 20):
        for ln in open(cfile):
            if ln.startswith("mfma_busy_frac"):
                out["counter_busy_frac"] = float(ln.split("=")[1])
                out["counter_source"] = os.path.relpath(cfile, ROOT)
    return out


def cpu_baseline(sample_T, H_full, D=64, L=8, K=4, reps=16):
    """Reference CPU path (aten + race_pref.cpp from source) on one head of
    sample_T tokens of the same workload, run reps times (default 16 x 65536
    tokens = 2^20 token-heads, about 12 s on 16 host threads; the reference's
    flat layout copies V once per bucket, about 128 KB of host memory per
    token, which bounds one run's length); the median run is reported as
    tokens/s of the full H-head layer.  Falls back to the fp64 C restatement
    if oracle/_ref is absent."""
    import torch
    from oracle import race_oracle
    threads = torch.get_num_threads()
    ext = race_oracle.ref_race_pref()
    times = []
    if ext is not None:
        from oracle import ref_cpu_path

        def run(T, seed):
            q, k, v, do, planes = make_inputs(1, T, 1, D, L, K, "cpu", seed=seed)
            planes_T = planes[0].reshape(L * K, D).T.contiguous().float()
            Kf, Vf, Qf = [x.float().requires_grad_(True) for x in (k, v, q)]
            dof = do.float()
            t0 = time.perf_counter()
            out = ref_cpu_path.causal_forward(Kf, Vf, Qf, planes_T, K, L, ext=ext)
            out.backward(dof)
            return time.perf_counter() - t0

        run(min(8192, sample_T), 6)  # warm-up: thread pool, allocator
        times = [run(sample_T, 7 + r) for r in range(reps)]
        kind = "reference"
        what = "misc/race.py CPU path: aten projection/softmax/readout + kernels/cpu/race_pref.cpp (built from source)"
    else:
        from oracle import race_oracle as ro
        q, k, v, do, planes = make_inputs(1, sample_T, 1, D, L, K, "cpu", seed=7)
        arrs = [x.double().numpy() for x in (q, k, v, do)]
        pl = planes.double().numpy()
        for _ in range(reps):
            t0 = time.perf_counter()
            ro.race_forward(arrs[0], arrs[1], arrs[2], pl, causal=True, inv_temp=1 / math.sqrt(D))
            ro.race_backward(*arrs, pl, causal=True, inv_temp=1 / math.sqrt(D))
            times.append(time.perf_counter() - t0)
        kind = "port"
        what = "fp64 C restatement (oracle/race_oracle.c), one thread per stream"
        threads = 1
    t = statistics.median(times)
    return {"value": sample_T / t / H_full, "unit": "tokens/s", "cores": threads, "kind": kind,
            "sample": f"1 of {H_full} streams x {sample_T} tokens of the same causal K={K} L={L} d={D} workload, "
                      f"fwd+bwd, median of {reps} runs after a warm-up ({what}); {t:.2f} s per run; "
                      f"value scaled to tokens of the {H_full}-stream layer",
            "host_cpus": os.cpu_count(), "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def max_seq_bisect(H, D, L, K, dev, step=1 << 16):
    """Longest T (multiple of step) for which one layer's fwd+bwd fits in HBM:
    separate Q, K, V, dO inputs, O, dQ, dK, dV outputs, the forward state and
    the workspace, all allocated and the step run once.  The candidate comes
    from the free HBM and the library's own size queries; it is then confirmed
    by running at T (stepping down while that runs out of memory) and by T +
    step running out of memory (stepping up while it does not).  Only an
    allocation failure counts as "does not fit"; any other error fails the run."""
    import torch
    from race_attention_amd import _lib
    from race_attention_amd.functional import make_desc
    lib = _lib.load()

    def need(T):
        x = torch.empty((1, 1, T, H, D), dtype=torch.bfloat16, device="meta")  # shapes and strides only
        d = make_desc(x, x, x, torch.empty(1, L, K, D), L=L, K=K, causal=True, eps=1e-6, inv_temp=0.125)
        ref = ctypes.byref(d)
        return (8 * T * H * D * 2 + lib.race_state_bytes(ref) +
                max(lib.race_fwd_workspace_bytes(ref), lib.race_bwd_workspace_bytes(ref)))

    def fits(T):
        bufs = None
        try:
            bufs = [torch.empty(1, 1, T, H, D, dtype=torch.bfloat16, device=dev) for _ in range(4)]
            for b in bufs:
                b.normal_()
            st = Step(*bufs, torch.randn(1, L, K, D, device=dev), L, K)
            st.run()
            torch.cuda.synchronize()
            del st
            return True
        except torch.cuda.OutOfMemoryError:
            return False  # only an allocation failure means "does not fit"; anything else fails the run
        finally:
            del bufs
            torch.cuda.empty_cache()

    torch.cuda.empty_cache()
    free = torch.cuda.mem_get_info(dev)[0]
    T = step
    while need(T + step) <= free:
        T += step if need(2 * T) > free else T
    T = T // step * step
    tries = 0
    while not fits(T):  # fragmentation or allocator overhead: step down
        T -= step
        tries += 1
        if T <= 0 or tries > 64:
            raise RuntimeError("max-N search: no fitting length found")
    while fits(T + step):  # the estimate was conservative: step up
        T += step
        tries += 1
        if tries > 64:
            break
    return T


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (requested --gpus {args.gpus}, WORLD_SIZE={world}); "
              "the RACE operator shards by head/batch streams with no communication, and multi-GPU runs are "
              "not part of this build", file=sys.stderr)
        sys.exit(2)
    import torch
    if args.workload in ("c3-step", "c5-step"):
        return model_step_main(args)
    dev = torch.device("cuda:0")
    if args.workload == "c5":
        M, B, T, H, D, L, K = 2, 8, 8192, 12, 64, 4, 8
        wl = "C5 decoder attention core fwd+bwd"
    else:
        M, B, T, H, D, L, K = 1, 1, args.seq, args.heads, 64, 8, 4
        wl = "C4 causal RACE layer core fwd+bwd"
    if args.mode == "global":
        wl += ", global normalisation (F2, beta=1)"
    print(f"bench: generating inputs M={M} B={B} T={T} H={H} D={D} L={L} K={K}", file=sys.stderr, flush=True)
    q, k, v, do, planes = make_inputs(B, T, H, D, L, K, dev, M=M)
    if args.mode == "probs":
        return probs_main(args, q, planes, L, K, wl, T, B, H, D, M)
    step = (GlobalStep if args.mode == "global" else Step)(q, k, v, do, planes, L, K)
    for _ in range(args.warmup):
        step.run()
    torch.cuda.synchronize()
    print("bench: warm-up done", file=sys.stderr, flush=True)

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(PHASES) + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        ev[s][0].record()
        for j, (_, which, ph) in enumerate(PHASES):
            step.run(phases=ph, which=which)
            ev[s][j + 1].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    per = {name: statistics.mean(ev[s][j].elapsed_time(ev[s][j + 1]) for s in range(args.steps))
           for j, (name, _, _) in enumerate(PHASES)}
    tokens = B * T
    value = tokens / (ms / 1e3)

    tok_heads = M * B * T * H  # token-streams: each (m, b, h) stream reads its own Q, K, V rows
    kernels = {}
    sc = scan_bytes(*step.sizes, M * B * H, T, L, K, D) if args.mode == "f1" else None
    for name, t_ms in per.items():
        ab = algorithmic_bytes(name, tok_heads, D, 2, args.mode)
        kernels[name] = {"ms": round(t_ms, 4),
                         "algorithmic_GBs": round(ab / (t_ms * 1e-3) / 1e9, 1) if ab else None}
        if sc and name in ("fwd_scan", "bwd_scan"):
            # the scans move segment sums, not token rows: read the sums, write the prefixes
            nb = sc[0] if name == "fwd_scan" else sc[1]
            kernels[name].update(segments=sc[2] if name == "fwd_scan" else sc[3], bytes=nb,
                                 GBs=round(nb / (t_ms * 1e-3) / 1e9, 1),
                                 frac=round(nb / (t_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
    dom = max(per, key=per.get)
    ab = algorithmic_bytes(dom, tok_heads, D, 2, args.mode)
    achieved = ab / (per[dom] * 1e-3) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", f"traffic_{dom}_{args.workload}.txt")
    if os.path.exists(tfile) and args.mode == "f1" and (args.workload != "c4" or T == 1 << 20):
        for ln in open(tfile):
            if ln.startswith("hbm_bytes_per_launch"):
                traffic = float(ln.split("=")[1])
    all_bytes = 11 * tok_heads * D * 2
    res = {
        "metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (unit-L2 N(0,1) Q/K/V, N(0,1) dO and hyperplanes, seeds 0/1234)",
        "config": {"workload": f"{wl}: B={B} H={H} N={T} d={D} K={K} L={L} M={M} bf16",
                   "B": B, "H": H, "seq_len": T, "d": D, "K": K, "L": L, "M": M, "causal": True,
                   "normalisation": "per-bucket (F1)" if args.mode == "f1" else "global (F2)"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "layer_roofline": {"algorithmic_bytes_per_step": all_bytes,
                           "hbm_bound_tokens_per_s": round(tokens / (all_bytes / (HBM_PEAK_GBS * 1e9)), 1),
                           "frac": round(value / (tokens / (all_bytes / (HBM_PEAK_GBS * 1e9))), 4)},
        "kernels": kernels,
    }
    if "fwd_reduce" in per and args.mode == "f1":
        res["mfma"] = mfma_figures(per["fwd_reduce"], tok_heads, D, L, K, args.workload, T)
    if args.copy_calib:
        n = args.copy_calib << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        res["copy_calib_bytes"] = n
        del src, dst
    if args.max_n and args.workload == "c4" and args.mode == "f1":
        del step, q, k, v, do
        torch.cuda.empty_cache()
        print("bench: max-N bisection", file=sys.stderr, flush=True)
        t_mx = time.perf_counter()
        res["max_seq_len_fwd_bwd"] = max_seq_bisect(H, D, L, K, dev)
        res["max_seq_len_note"] = (f"longest N (multiple of 2^16) whose layer fwd+bwd (B=1 H={H} d={D} K={K} L={L} "
                                   "bf16: separate Q, K, V, dO, O, dQ, dK, dV, state, workspace) allocates and runs "
                                   f"in this GPU's HBM; bisection took {time.perf_counter() - t_mx:.1f} s")
    if not args.no_cpu_baseline:
        print("bench: CPU baseline", file=sys.stderr, flush=True)
        if args.mode == "global":
            res["cpu_baseline"] = cpu_baseline_global(min(T, 8192), H * M, D=D, L=L, K=K)
        elif args.workload == "c4":
            res["cpu_baseline"] = cpu_baseline(args.cpu_sample, H * M, D=D, L=L, K=K)
        else:  # 1024 buckets: the reference's flat layout holds 256 KB per token
            res["cpu_baseline"] = cpu_baseline(min(args.cpu_sample, 2048), H * M, D=D, L=L, K=K, reps=8)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
