"""GPU parity of the bucket probabilities as an output (race_probs /
race_probs_bwd through the C ABI) against the fp64 oracle, and of the
hybrid-consumer helpers (race_attention_amd.buckets; misc/arxiv_64K.py:1580-1644,
misc/vit.py:3193-3262) against an fp64 torch restatement of the reference's
aten path.  Bars: max|a-b|/max|b| <= 1e-4 (fp32), <= 2e-2 (bf16)."""
import itertools
import zlib

import pytest
import torch

from helpers import TOL, make_case, relerr, to64

pytestmark = pytest.mark.gpu

CASES = [
    # name, make_case kwargs (q is the input x), inv_temp
    ("probs_bf16_K4L8", dict(B=2, T=150, H=2, L=8, K=4), 1.0),
    ("probs_bf16_K2L5", dict(B=1, T=77, H=3, L=5, K=2), 0.7),
    ("probs_bf16_K1L3_odd", dict(B=1, T=40, H=2, L=3, K=1), 1.0),
    ("probs_bf16_K8L4_slices", dict(B=1, T=70, H=2, L=4, K=8), 1.0),
    ("probs_bf16_M2_indep", dict(M=2, B=1, T=64, H=2, L=5, K=3, share_planes=False), 1.0),
    ("probs_fp32_K2L5", dict(B=2, T=130, H=2, L=5, K=2, dtype=torch.float32, unit=False), 1.0),
    ("probs_fp32_K4L8_4slices", dict(B=1, T=100, H=2, L=8, K=4, dtype=torch.float32, unit=False), 0.5),
    ("probs_fp32_K6L2", dict(B=1, T=50, H=1, L=2, K=6, dtype=torch.float32, unit=False), 1.0),
]


@pytest.mark.parametrize("name,kw,it", CASES, ids=[c[0] for c in CASES])
def test_probs_parity(dev, name, kw, it):
    from oracle import race_oracle as ro
    from race_attention_amd.functional import race_probs_bwd_raw, race_probs_raw
    x, _, _, _, planes = make_case(seed=zlib.crc32(name.encode()) % 1000, **kw)
    M, B, T, H, _ = x.shape
    L, K = kw["L"], kw["K"]
    g = torch.Generator().manual_seed(zlib.crc32(name.encode()) % 991)
    dP = torch.randn(M, B, H, T, L << K, generator=g)
    xd, pd = x.to(dev), planes.to(dev)
    P = race_probs_raw(xd, pd, L=L, K=K, inv_temp=it)
    dx, git = race_probs_bwd_raw(xd, pd, dP.to(dev), L=L, K=K, inv_temp=it)
    torch.cuda.synchronize()
    pl = planes.double().numpy()
    P_ref = ro.race_probs(to64(x), pl, inv_temp=it)
    dx_ref, git_ref, gabs = ro.race_probs_bwd(to64(x), dP.double().numpy(), pl, inv_temp=it, with_l1=True)
    tol = TOL[x.dtype]
    errs = {"P": relerr(to64(P), P_ref), "dx": relerr(to64(dx), dx_ref),
            "dinv_temp": abs(float(git.cpu()) - git_ref) / ((abs(git_ref) if tol < 1e-3 else gabs) + 1e-30)}
    print(f"[{name}] " + " ".join(f"{a}={b:.2e}" for a, b in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= tol, f"{name}: {nm} {e:.3e} > {tol:.1e}"


def _reference_avg_probs(mod, x):
    """misc/vit.py:3193-3262 in fp64 on the CPU (aten path)."""
    ace = mod.ace
    B, T, _ = x.shape
    H, dk, M = mod.H, mod.d_k, mod.M
    W = {n: p.detach().double() for n, p in mod.named_parameters()}
    xx = x.double().requires_grad_(True)
    lt = W["ace.logit_temp"].clone().requires_grad_(True)
    scale = lt.exp().clamp(1e-2, 20.0)
    Q = torch.nn.functional.linear(xx, W["q_proj.weight"], W.get("q_proj.bias")).view(B, T, H, dk)
    K = torch.nn.functional.linear(xx, W["k_proj.weight"], W.get("k_proj.bias")).view(B, T, H, dk)
    planes = ace.planes().detach().double()                                   # [M,L,K,d] or [L,K,d]
    protos = torch.tensor(list(itertools.product([-1., +1.], repeat=ace.K)), dtype=torch.float64).T
    outs = []
    for Z in (Q, K):
        Zm = Z.unsqueeze(0).expand(M, -1, -1, -1, -1).permute(0, 1, 3, 2, 4)   # [M,B,H,T,dk]
        pl = planes if planes.dim() == 4 else planes.unsqueeze(0).expand(M, -1, -1, -1)
        proj = torch.einsum("mbhtd,mlkd->mbhtlk", Zm, pl)
        probs = torch.softmax((proj.tanh() / scale) @ protos, dim=-1)            # [M,B,H,T,L,R]
        outs.append(probs.reshape(M, B, H, T, -1).mean(dim=0))
    return outs, xx, lt


def test_avg_bucket_probs_from_x(dev):
    """race_avg_bucket_probs_from_x on vit.RACEAttention (fp32, M=2
    independent sketches): both averaged distributions, and the gradients
    of x and logit_temp for a random linear loss."""
    from race_attention_amd import vit
    from race_attention_amd.buckets import race_avg_bucket_probs_from_x
    torch.manual_seed(4)
    m = vit.RACEAttention(128, 128, 0.0, num_heads=2, L=4, K=3, N_M=2)
    x = torch.randn(2, 60, 128)
    (rq, rk), xx, lt = _reference_avg_probs(m, x)
    Gq, Gk = torch.randn(rq.shape, dtype=torch.float64), torch.randn(rk.shape, dtype=torch.float64)
    ((rq * Gq).sum() + (rk * Gk).sum()).backward()
    md = m.to(dev)
    xd = x.to(dev).requires_grad_(True)
    pq, pk = race_avg_bucket_probs_from_x(md, xd)
    ((pq * Gq.float().to(dev)).sum() + (pk * Gk.float().to(dev)).sum()).backward()
    torch.cuda.synchronize()
    errs = {"probsQ": relerr(pq.detach().cpu(), rq.detach()), "probsK": relerr(pk.detach().cpu(), rk.detach()),
            "x.grad": relerr(xd.grad.cpu(), xx.grad),
            "logit_temp": abs(float(md.ace.logit_temp.grad) - float(lt.grad)) / abs(float(lt.grad))}
    print("[race_avg_bucket_probs_from_x] " + " ".join(f"{a}={b:.2e}" for a, b in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= 1e-4, f"{nm}: {e:.3e}"
