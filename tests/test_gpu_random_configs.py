"""Randomised parity: seeded random configurations of the operator against
the fp64 oracle, on top of the hand-picked cases of the other test files.

Each case draws K = 1..8, L (L*K <= 32), M (shared or independent planes, or
an expand over M), B, H, T (whole tiles or ragged, up to 700), an explicit or
automatic segmentation, eps, a temperature (1/sqrt(d) or uniform in
[0.1, 2]), a value mean, and (F1) the memory layout of each input: contiguous,
[M,B,H,T,D] storage viewed as [M,B,T,H,D], a D-slice of a fused [.., 3D] row,
or the first T tokens of a longer buffer.  The key-weight / den form and the
global normalisation draw their own extras (masks, den gradients, beta, the
floor).  Bars: the north-star ones on every tensor; the scalar gradient
(d(inv_temp), d(beta)), one sum over every token whose terms can cancel by
three orders of magnitude and more, against the l1 mass of its terms, with
the bar of the tensors for bf16 and 1e-6 for fp32 (its fp32 rounding floor
is about 1e-7 of that mass)."""
import random

import pytest
import torch

from helpers import TOL, make_case, relerr, run_gpu, run_oracle, to64

pytestmark = pytest.mark.gpu

SCALAR_BAR = {torch.float32: 1e-6, torch.bfloat16: 2e-2}


def _draw(rng):
    dtype = torch.float32 if rng.random() < 0.3 else torch.bfloat16
    K = rng.randint(1, 8)
    L = rng.randint(1, min(8, 32 // K))
    M = rng.choice([1, 1, 2])
    share = rng.random() < 0.5
    expand = M == 2 and rng.random() < 0.5
    B, H = rng.choice([1, 2]), rng.choice([1, 2, 3])
    T = 32 * rng.randint(1, 20) if rng.random() < 0.4 else rng.randint(1, 700)
    seg = 0 if rng.random() < 0.5 else rng.randint(1, 12)
    vs = 0.5 if rng.random() < 0.3 else 0.0
    unit = dtype == torch.bfloat16 or rng.random() < 0.5
    if M * B * H * T * (L << K) > 12_000_000:  # the oracle in seconds
        T = max(1, 12_000_000 // (M * B * H * (L << K)))
    return dict(M=M, B=B, T=T, H=H, L=L, K=K, dtype=dtype, unit=unit, share_planes=share, expand_m=expand,
                v_shift=vs), seg


def _relayout(x, kind, rng):
    if kind == "bhtd":
        return x.permute(0, 1, 3, 2, 4).contiguous().permute(0, 1, 3, 2, 4)
    if kind == "fused":
        big = torch.zeros(x.shape[:4] + (3 * x.shape[4],), dtype=x.dtype, device=x.device)
        off = rng.choice([0, 1, 2]) * x.shape[4]
        big[..., off:off + x.shape[4]] = x
        return big[..., off:off + x.shape[4]]
    if kind == "longT":
        big = torch.zeros(x.shape[:2] + (x.shape[2] + 37,) + x.shape[3:], dtype=x.dtype, device=x.device)
        big[:, :, :x.shape[2]] = x
        return big[:, :, :x.shape[2]]
    return x


def _check(name, errs, scalar, dtype):
    print(f"[{name}] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()) + f" scalar/l1={scalar:.2e}", flush=True)
    for nm, e in errs.items():
        assert e <= TOL[dtype], f"{name}: {nm} {e:.3e}"
    assert scalar <= SCALAR_BAR[dtype], f"{name}: scalar gradient {scalar:.3e} of its l1 mass"


def test_random_f1(dev):
    rng = random.Random(20261202)
    for c in range(120):
        cfg, seg = _draw(rng)
        causal = rng.random() < 0.75
        eps = 0.5 if (cfg["T"] <= 2 or rng.random() < 0.15) else 1e-6
        it = 0.125 if rng.random() < 0.6 else rng.uniform(0.1, 2.0)
        kinds = [rng.choice(["contig", "bhtd", "fused", "longT"]) for _ in range(4)]
        q, k, v, do, planes = make_case(seed=70000 + c, **cfg)
        gq, gk, gv, gdo = [_relayout(x.to(dev), kd, rng) if x.stride(0) != 0 or x.shape[0] == 1 else x.to(dev)
                           for x, kd in zip((q, k, v, do), kinds)]
        name = (f"f1 #{c} {cfg['dtype']} {'causal' if causal else 'noncausal'} K={cfg['K']} L={cfg['L']} "
                f"M={cfg['M']} B={cfg['B']} H={cfg['H']} T={cfg['T']} seg={seg} it={it:.3f} {','.join(kinds)}")
        gpu = run_gpu(gq, gk, gv, gdo, planes, L=cfg["L"], K=cfg["K"], causal=causal, inv_temp=it, dev=dev,
                      seg_tiles=seg, eps=eps)
        ref = run_oracle(q, k, v, do, planes, causal=causal, inv_temp=it, eps=eps)
        errs = {nm: relerr(to64(a), b) for nm, a, b in zip(("out", "dq", "dk", "dv"), gpu[:4], ref[:4])}
        _check(name, errs, abs(gpu[4] - ref[4]) / (ref[5] + 1e-30), cfg["dtype"])


def test_random_key_weights_and_den(dev):
    import test_gpu_ex as tx
    from oracle import race_oracle as ro
    rng = random.Random(20261203)
    for c in range(40):
        cfg, seg = _draw(rng)
        it = 0.125 if rng.random() < 0.5 else rng.uniform(0.1, 2.0)
        mk = rng.choice([None, "binary", "frac"])
        q, k, v, do, planes = make_case(seed=71000 + c, **cfg)
        g = torch.Generator().manual_seed(71000 + c)
        M, B, T, H = q.shape[:4]
        kmask = tx._masks(mk, B, T, g)
        dden = torch.randn(M, B, H, T, generator=g) if rng.random() < 0.6 else None
        name = (f"ex #{c} {cfg['dtype']} K={cfg['K']} L={cfg['L']} M={M} B={B} H={H} T={T} seg={seg} it={it:.3f} "
                f"mask={mk} dden={dden is not None}")
        gpu = tx._run(q, k, v, do, planes, L=cfg["L"], K=cfg["K"], it=it, kmask=kmask, dden=dden, dev=dev, seg=seg)
        pl = planes.double().numpy()
        km = kmask.double().numpy() if kmask is not None else None
        o, den = ro.race_forward_ex(to64(q), to64(k), to64(v), pl, kmask=km, causal=False, inv_temp=it)
        dq, dk, dv, git, gabs = ro.race_backward_ex(to64(q), to64(k), to64(v), to64(do), pl, kmask=km,
                                                    dden=to64(dden) if dden is not None else None, causal=False,
                                                    inv_temp=it, with_l1=True)
        errs = {nm: relerr(to64(a), b) for nm, a, b in zip(("out", "den", "dq", "dk", "dv"), gpu[:5],
                                                            (o, den, dq, dk, dv))}
        _check(name, errs, abs(gpu[5] - git) / (gabs + 1e-30), cfg["dtype"])


def test_random_global(dev):
    import test_gpu_global as tg
    rng = random.Random(20261204)
    for c in range(40):
        cfg, seg = _draw(rng)
        beta = 1.0 if rng.random() < 0.5 else rng.uniform(0.2, 3.0)
        floor = 1e-6 if rng.random() < 0.85 else 10.0 ** rng.uniform(-2, 4)
        q, k, v, do, planes = make_case(seed=72000 + c, **cfg)
        g = torch.Generator().manual_seed(72000 + c)
        M, B, T, H = q.shape[:4]
        dden = torch.randn(M, B, H, T, generator=g) if rng.random() < 0.6 else None
        name = (f"gn #{c} {cfg['dtype']} K={cfg['K']} L={cfg['L']} M={M} B={B} H={H} T={T} seg={seg} "
                f"beta={beta:.3f} floor={floor:.2g} dden={dden is not None}")
        gpu = tg._run_gpu(q, k, v, do, dden, planes, L=cfg["L"], K=cfg["K"], beta=beta, dev=dev, seg_tiles=seg,
                          floor=floor)
        ref = tg._run_oracle(q, k, v, do, dden, planes, beta=beta, floor=floor)
        errs = {nm: relerr(to64(a), b) for nm, a, b in zip(("out", "den", "dq", "dk", "dv"), gpu[:5], ref[:5])}
        _check(name, errs, abs(gpu[5] - ref[5]) / (ref[6] + 1e-30), cfg["dtype"])
