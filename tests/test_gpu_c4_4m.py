"""Config C4's second size: causal bf16, B=1, H=8, N=2^22 = 4,194,304, d=64,
K=4, L=8, M=1, unit-norm Q/K/V.  Each Q/K/V/dO/out/dX
tensor holds exactly 2^31 elements, the size at which the reference CUDA host
code's int sizes overflow (kernels/gpu/forward_kernel.cu:72-75); every offset
here is 64-bit or a bounded 32-bit lane offset inside a tile.

Checks (the oracle is too slow for 4M tokens x 8 heads):
  * prefix: dO zero beyond T0 -> every gradient beyond T0 is exactly zero and
    the first T0 tokens equal the oracle run on those T0 tokens alone;
  * last token: the causal output at N-1 against the non-causal run and an
    fp64 evaluation of the sequence totals (two heads);
  * suffix: dO zero before the last T0 tokens -> for every earlier token the
    backward carries are constants of the last T0 tokens; dK and dV at sampled
    early tokens (tile / segment edges and random ones) against the fp64
    closed form of tests/longseq.py, and dQ exactly zero there.
"""
import math

import pytest
import torch

import longseq
from helpers import TOL, relerr, to64

pytestmark = pytest.mark.gpu

B, T, H, D, L, K = 1, 1 << 22, 8, 64, 8, 4
T0 = 8192
EPS = 1e-6
HEADS = (0, 5)


def _inputs(dev):
    g = torch.Generator(device=dev).manual_seed(4242)
    q, k, v = [torch.nn.functional.normalize(torch.randn(1, B, T, H, D, device=dev, generator=g), dim=-1)
               .to(torch.bfloat16) for _ in range(3)]
    planes = torch.randn(1, L, K, D, generator=torch.Generator().manual_seed(77))
    return q, k, v, planes, g


def test_c4_4m(dev, oracle):
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    it = 1.0 / math.sqrt(D)
    q, k, v, planes, g = _inputs(dev)
    assert q.numel() == 2 ** 31
    pd = planes.to(dev)
    print(f"[C4 4M] causal fwd B={B} T={T} H={H} ({q.numel()} elements per tensor)", flush=True)
    out, state = race_fwd_raw(q, k, v, pd, L=L, K=K, causal=True, inv_temp=it)
    out_nc, _ = race_fwd_raw(q, k, v, pd, L=L, K=K, causal=False, inv_temp=it)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(out_nc).all()

    # ---- prefix: dO only in the first T0 tokens
    do = torch.zeros(1, B, T, H, D, device=dev, dtype=torch.bfloat16)
    do[:, :, :T0] = torch.randn(1, B, T0, H, D, device=dev, generator=g).to(torch.bfloat16)
    print("[C4 4M] backward, dO in the first T0 tokens", flush=True)
    dq, dk, dv, _ = race_bwd_raw(q, k, v, pd, do, state, L=L, K=K, causal=True, inv_temp=it)
    torch.cuda.synchronize()
    for name, x in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isfinite(x).all(), name
        assert not x[:, :, T0:].any(), f"{name} nonzero beyond T0"
    sl = lambda x: to64(x[:, :, :T0])  # noqa: E731
    pl = planes.double().numpy()
    o_ref = oracle.race_forward(sl(q), sl(k), sl(v), pl, causal=True, inv_temp=it)
    g_ref = oracle.race_backward(sl(q), sl(k), sl(v), sl(do), pl, causal=True, inv_temp=it)
    errs = {"out": relerr(sl(out), o_ref)}
    errs.update({n: relerr(sl(a), b) for n, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), g_ref[:3])})
    print("[C4 4M prefix T0=%d] " % T0 + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert max(errs.values()) <= TOL[torch.bfloat16]
    del dq, dk, dv, do

    # ---- last token against the non-causal run and fp64 totals
    pl0 = planes[0].double().to(dev)
    e_nc = relerr(to64(out[0, 0, T - 1]), to64(out_nc[0, 0, T - 1]))
    for h in HEADS:
        ref = longseq.last_token_reference(q, k, v, h, pl0, it, L, K, EPS).cpu().numpy()
        e_c, e_n = relerr(to64(out[0, 0, T - 1, h]), ref), relerr(to64(out_nc[0, 0, T - 1, h]), ref)
        print(f"[C4 4M last token h={h}] causal-vs-fp64={e_c:.2e} noncausal-vs-fp64={e_n:.2e}", flush=True)
        assert max(e_c, e_n) <= TOL[torch.bfloat16]
    print(f"[C4 4M last token] causal-vs-noncausal={e_nc:.2e}", flush=True)
    assert e_nc <= TOL[torch.bfloat16]

    # ---- suffix: dO only in the last T0 tokens
    do = torch.zeros(1, B, T, H, D, device=dev, dtype=torch.bfloat16)
    do[:, :, T - T0:] = torch.randn(1, B, T0, H, D, device=dev, generator=g).to(torch.bfloat16)
    print("[C4 4M] backward, dO in the last T0 tokens", flush=True)
    dq, dk, dv, _ = race_bwd_raw(q, k, v, pd, do, state, L=L, K=K, causal=True, inv_temp=it)
    torch.cuda.synchronize()
    assert not dq[:, :, :T - T0].any(), "dq nonzero before the last T0 tokens"
    taus = longseq.sample_taus(T, T0)
    for h in HEADS:
        dK_ref, dV_ref = longseq.suffix_reference(q, k, v, do, h, pl0, it, L, K, T0, EPS, taus)
        e_k = relerr(to64(dk[0, 0, taus, h]), dK_ref.cpu().numpy())
        e_v = relerr(to64(dv[0, 0, taus, h]), dV_ref.cpu().numpy())
        print(f"[C4 4M suffix h={h}, {len(taus)} early tokens] dk={e_k:.2e} dv={e_v:.2e}", flush=True)
        assert max(e_k, e_v) <= TOL[torch.bfloat16]
