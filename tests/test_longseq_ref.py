"""The fp64 long-sequence restatement (tests/longseq.py) used by the
full-length GPU checks agrees with the oracle on small causal cases: the
backward suffix constants (dK, dV at early tokens when dO lives only in the
last T0 tokens) and the last-token readout."""
import math

import numpy as np
import torch

import longseq
from helpers import make_case, relerr, to64


def test_suffix_reference_matches_oracle(oracle):
    T, T0, H, D, L, K = 300, 64, 2, 64, 8, 4
    q, k, v, do, planes = make_case(B=1, T=T, H=H, L=L, K=K, dtype=torch.float32, seed=3)
    do[:, :, :T - T0] = 0
    it = 1.0 / math.sqrt(D)
    g = oracle.race_backward(to64(q), to64(k), to64(v), to64(do), planes.double().numpy(), causal=True,
                             inv_temp=it)
    taus = longseq.sample_taus(T, T0)
    assert len(taus) > 10
    pl = planes[0].double()
    for h in range(H):
        dK, dV = longseq.suffix_reference(q, k, v, do, h, pl, it, L, K, T0, 1e-6, taus)
        assert relerr(dK.numpy(), g[1][0, 0, taus, h]) < 1e-10
        assert relerr(dV.numpy(), g[2][0, 0, taus, h]) < 1e-10
        assert np.all(g[0][0, 0, :T - T0, h] == 0)  # dQ is exactly zero before the last T0 tokens


def test_last_token_reference_matches_oracle(oracle):
    T, H, D, L, K = 200, 2, 64, 4, 3
    q, k, v, do, planes = make_case(B=1, T=T, H=H, L=L, K=K, dtype=torch.float32, seed=4)
    it = 0.3
    o = oracle.race_forward(to64(q), to64(k), to64(v), planes.double().numpy(), causal=True, inv_temp=it)
    for h in range(H):
        ref = longseq.last_token_reference(q, k, v, h, planes[0].double(), it, L, K, 1e-6)
        assert relerr(ref.numpy(), o[0, 0, T - 1, h]) < 1e-12
