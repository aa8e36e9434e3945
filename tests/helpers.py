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
              share_planes=True, expand_m=False):
    """Seeded Q, K, V, dO [M,B,T,H,D] (dtype, CPU), planes fp32 [NP,L,K,D].
    unit=True row-normalises Q, K, V (configs C2/C4); expand_m builds the M
    estimators as an expand of one [B,T,H,D] tensor (stride 0 over M)."""
    g = torch.Generator().manual_seed(seed)
    Mi = 1 if expand_m else M
    q, k, v = [torch.randn(Mi, B, T, H, D, generator=g) for _ in range(3)]
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
