"""Shared helpers for the parity tests: seeded inputs, the oracle on the same
values, and the reference's relative-error metric."""
import numpy as np
import torch


def relerr(a, b) -> float:
    """max|a-b| / max|b|, the metric of kernels/cpu/setup.py:169-170."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den + 1e-30))


TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def make_case(M=1, B=1, T=64, H=2, D=64, L=8, K=4, dtype=torch.bfloat16, seed=0, unit=True,
              share_planes=True, expand_m=False, v_shift=0.0):
    """Seeded Q, K, V, dO [M,B,T,H,D] (dtype, CPU), planes fp32 [NP,L,K,D].
    unit=True row-normalises Q, K, V (configs C2/C4); expand_m builds the M
    estimators as an expand of one [B,T,H,D] tensor (stride 0 over M);
    v_shift adds a constant to every component of V before the
    normalisation (values with a mean, whose B sums grow linearly in t)."""
    g = torch.Generator().manual_seed(seed)
    Mi = 1 if expand_m else M
    q, k, v = [torch.randn(Mi, B, T, H, D, generator=g) for _ in range(3)]
    v = v + v_shift
    if unit:
        q, k, v = [torch.nn.functional.normalize(x, dim=-1) for x in (q, k, v)]
    do = torch.randn(M, B, T, H, D, generator=g)
    gp = torch.Generator().manual_seed(seed + 1234)
    planes = torch.randn(1 if share_planes else M, L, K, D, generator=gp)
    q, k, v, do = [x.to(dtype) for x in (q, k, v, do)]
    if expand_m:
        q, k, v = [x.expand(M, -1, -1, -1, -1) for x in (q, k, v)]
    return q, k, v, do, planes


def to64(x: torch.Tensor) -> np.ndarray:
    return x.detach().to(torch.float64).cpu().numpy()


def run_gpu(q, k, v, do, planes, *, L, K, causal, inv_temp, dev, seg_tiles=0, eps=1e-6):
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    qd, kd, vd, dod, pd = [x.to(dev) for x in (q, k, v, do, planes)]
    out, state = race_fwd_raw(qd, kd, vd, pd, L=L, K=K, causal=causal, inv_temp=inv_temp, seg_tiles=seg_tiles,
                              eps=eps)
    dq, dk, dv, git = race_bwd_raw(qd, kd, vd, pd, dod, state, L=L, K=K, causal=causal, inv_temp=inv_temp,
                                   seg_tiles=seg_tiles, eps=eps)
    torch.cuda.synchronize()
    return out.cpu(), dq.cpu(), dk.cpu(), dv.cpu(), float(git.cpu())


def run_oracle(q, k, v, do, planes, *, causal, inv_temp, eps=1e-6):
    from oracle import race_oracle as ro
    o = ro.race_forward(to64(q), to64(k), to64(v), planes.double().numpy(), causal=causal, inv_temp=inv_temp,
                        eps=eps)
    dq, dk, dv, git, gabs = ro.race_backward(to64(q), to64(k), to64(v), to64(do), planes.double().numpy(),
                                             causal=causal, inv_temp=inv_temp, with_l1=True, eps=eps)
    return o, dq, dk, dv, git, gabs


def compare(case_name, gpu, ref, tol):
    """relerr = max|a-b|/max|b| per tensor.  d(inv_temp) is one sum over all
    tokens: fp32 compares |a-b|/|b|; bf16 compares |a-b| against the l1 mass
    sum|du*th| of its terms (ref[5]), the analogue of the max-norm metric for
    a reduction whose terms cancel."""
    names = ("out", "dq", "dk", "dv")
    errs = {nm: relerr(to64(a), b) for nm, a, b in zip(names, gpu[:4], ref[:4])}
    scale = abs(ref[4]) if (tol < 1e-3 or len(ref) < 6) else ref[5]
    errs["dinv_temp"] = abs(gpu[4] - ref[4]) / (scale + 1e-30)
    print(f"[{case_name}] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= tol, f"{case_name}: {nm} relerr {e:.3e} > {tol:.1e}"
