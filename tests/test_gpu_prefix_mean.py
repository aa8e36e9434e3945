"""GPU prefix mean (race_prefix_mean_fwd/bwd, the operator of the reference
CPU extension kernels/cpu/race_pref.cpp:36-220) against the vectors written by
the compiled reference kernel and against the fp64 oracle.  fp32 in and out,
fp64 accumulation as in the reference: tolerance 1e-5 relative (max|a-b| /
max|b|), tighter than the 1e-4 fp32 bar."""
import os

import numpy as np
import pytest
import torch

from helpers import relerr

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
TOL_PM = 1e-5


def test_prefix_mean_golden(dev):
    from race_attention_amd.functional import prefix_mean_bwd, prefix_mean_fwd
    z = np.load(os.path.join(HERE, "golden", "prefix_mean_ref.npz"))
    w, v, gE = (torch.from_numpy(z[k]).to(dev) for k in ("w", "v", "gE"))
    eps = float(z["eps"])
    E = prefix_mean_fwd(w, v, eps)
    gW, gV = prefix_mean_bwd(w, v, gE, eps)
    torch.cuda.synchronize()
    errs = [relerr(E.cpu(), z["E"]), relerr(gW.cpu(), z["gW"]), relerr(gV.cpu(), z["gV"])]
    print("[prefix_mean golden] E=%.2e gW=%.2e gV=%.2e" % tuple(errs), flush=True)
    assert max(errs) <= TOL_PM


@pytest.mark.parametrize("NS,T,D", [(3, 1, 64), (2, 5, 1), (4, 4097, 64), (1, 300, 100), (2, 130, 512),
                                    (5000, 3, 8)])
def test_prefix_mean_oracle(dev, oracle, NS, T, D):
    from race_attention_amd.functional import prefix_mean_bwd, prefix_mean_fwd
    g = torch.Generator().manual_seed(NS * 7 + T * 3 + D)
    w = torch.rand(NS, T, generator=g)          # probabilities in [0, 1)
    v = torch.randn(NS, T, D, generator=g)
    gE = torch.randn(NS, T, D, generator=g)
    eps = 1e-6
    E = prefix_mean_fwd(w.to(dev), v.to(dev), eps)
    gW, gV = prefix_mean_bwd(w.to(dev), v.to(dev), gE.to(dev), eps)
    torch.cuda.synchronize()
    Er = oracle.prefix_mean_flat(w.numpy(), v.numpy(), eps)
    gWr, gVr = oracle.prefix_mean_flat_bw(w.numpy(), v.numpy(), gE.numpy(), eps)
    errs = [relerr(E.cpu(), Er), relerr(gW.cpu(), gWr), relerr(gV.cpu(), gVr)]
    print(f"[prefix_mean NS={NS} T={T} D={D}] E=%.2e gW=%.2e gV=%.2e" % tuple(errs), flush=True)
    assert max(errs) <= TOL_PM


def test_prefix_mean_autograd_function(dev):
    """RACEPrefixMeanFlatFn (misc/race.py:9-24 drop-in) routes its backward to
    race_prefix_mean_bwd."""
    from race_attention_amd.functional import RACEPrefixMeanFlatFn, prefix_mean_bwd
    g = torch.Generator().manual_seed(11)
    w = torch.rand(3, 70, generator=g).to(dev).requires_grad_(True)
    v = torch.randn(3, 70, 16, generator=g).to(dev).requires_grad_(True)
    gE = torch.randn(3, 70, 16, generator=g).to(dev)
    E = RACEPrefixMeanFlatFn.apply(w, v, 1e-6)
    E.backward(gE)
    gW, gV = prefix_mean_bwd(w.detach(), v.detach(), gE, 1e-6)
    assert torch.equal(w.grad, gW) and torch.equal(v.grad, gV)


def test_prefix_mean_rejects_large_d(dev):
    from race_attention_amd._lib import RaceError
    from race_attention_amd.functional import prefix_mean_fwd
    with pytest.raises(RaceError, match="D=513"):
        prefix_mean_fwd(torch.rand(1, 4, device=dev), torch.randn(1, 4, 513, device=dev))
