"""Long causal walks with a value mean: the backward's forward-state walks.

k_bwd_out re-derives the forward state B(t) by subtracting tile sums from a
state row, and k_fwd_reduce / k_bwd_reduce carry B in fp32 MFMA accumulators.
Those roundings are relative to the state at the forward boundary the walk
starts from.  With zero-mean values |B| grows like sqrt(t); with a mean it
grows like t, so early in a sequence B(t) is far below the state a long walk
starts from -- the hazard of the reference CUDA backward, which rebuilds A(t)
and B(t) by subtracting from the finals (kernels/gpu/backward_kernels.cu:127-135).
Here every segment, forward and backward, is at most 256 tiles, so the fp32
walks are bounded whatever T is: long sequences add segments.

Inputs: Q, K unit-norm N(0,1); V = normalize(N(0,1) + 0.5) (a mean of about
0.45 of each row's norm along the all-ones direction); seeded planes.

  * prefix: dO non-zero only in the first T0 tokens -- the end of the reverse
    walk of the first backward segment, where B(t) is smallest against the
    states the walk passes -- so every gradient beyond T0 is exactly zero and
    the first T0 tokens equal the fp64 oracle on those T0 tokens alone
    (bf16 bar, 2e-2).  At T = 2^20 with the default plan (backward segments of
    2 forward ones, 256 tiles) and with explicit 256-tile segments, the longest
    the library accepts; at T = 2^24 the default plan, 2048 segments of 256
    tiles per stream.
  * suffix (T = 2^24): dO non-zero only in the last T0 tokens -- the reverse
    carries (U, alpha) of every earlier token, over the 2047 earlier backward
    segments per stream, are constants of those tokens: dK and dV at sampled
    early tokens against the fp64 closed form of tests/longseq.py.
"""
import ctypes
import math

import pytest
import torch

import longseq
from helpers import TOL, relerr, to64

pytestmark = pytest.mark.gpu

B, H, D, L, K = 1, 8, 64, 8, 4
T0 = 8192
EPS = 1e-6
SHIFT = 0.5
MAX_SEG_TILES = 256  # segment bound of the library (race_capi.hip kMaxSegTiles)


def _inputs(T, dev, seed):
    """Q, K unit-norm; V = normalize(randn + SHIFT); generated per 2^20-token
    chunk so the fp32 temporaries stay small at 2^24 tokens."""
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for shift in (0.0, 0.0, SHIFT):
        x = torch.empty(1, B, T, H, D, device=dev, dtype=torch.bfloat16)
        for a in range(0, T, 1 << 20):
            b = min(T, a + (1 << 20))
            r = torch.randn(1, B, b - a, H, D, device=dev, generator=g) + shift
            x[:, :, a:b] = torch.nn.functional.normalize(r, dim=-1).to(torch.bfloat16)
        out.append(x)
    planes = torch.randn(1, L, K, D, generator=torch.Generator().manual_seed(seed + 1))
    return (*out, planes, g)


def _fwd_segments(q, planes, seg_tiles):
    """Forward segments per stream of the library's plan (from the state size:
    N x (nseg + 1) rows of 128 buckets x 65 fp64)."""
    from race_attention_amd import _lib
    from race_attention_amd.functional import make_desc
    d = make_desc(q, q, q, planes, L=L, K=K, causal=True, eps=EPS, inv_temp=0.125, seg_tiles=seg_tiles)
    sb = _lib.load().race_state_bytes(ctypes.byref(d))
    assert sb > 0, _lib.last_error()
    return sb // (H * 128 * 65 * 8) - 1


def _check_prefix(name, q, k, v, pd, planes, do, state, oracle, seg_tiles):
    from race_attention_amd.functional import race_bwd_raw
    it = 1.0 / math.sqrt(D)
    dq, dk, dv, _ = race_bwd_raw(q, k, v, pd, do, state, L=L, K=K, causal=True, inv_temp=it, seg_tiles=seg_tiles)
    torch.cuda.synchronize()
    for nm, x in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isfinite(x).all(), nm
        assert not x[:, :, T0:].any(), f"{nm} nonzero beyond T0"
    sl = lambda x: to64(x[:, :, :T0])  # noqa: E731
    pl = planes.double().numpy()
    g_ref = oracle.race_backward(sl(q), sl(k), sl(v), sl(do), pl, causal=True, inv_temp=it)
    errs = {n: relerr(sl(a), b) for n, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), g_ref[:3])}
    print(f"[{name} prefix T0={T0}] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert max(errs.values()) <= TOL[torch.bfloat16], errs
    return errs


@pytest.mark.parametrize("T,seg_tiles", [(1 << 20, 0), (1 << 20, MAX_SEG_TILES)])
def test_long_walk_prefix(dev, oracle, T, seg_tiles):
    from race_attention_amd.functional import race_fwd_raw
    it = 1.0 / math.sqrt(D)
    q, k, v, planes, g = _inputs(T, dev, 2024)
    # the default plan's 2048 forward workgroups: 128-tile segments; explicit: 256
    assert _fwd_segments(q, planes, seg_tiles) == T // 32 // (seg_tiles or 128)
    pd = planes.to(dev)
    name = f"long walk T={T} seg_tiles={seg_tiles}"
    print(f"[{name}] causal fwd+bwd, V mean shift {SHIFT}", flush=True)
    out, state = race_fwd_raw(q, k, v, pd, L=L, K=K, causal=True, inv_temp=it, seg_tiles=seg_tiles)
    torch.cuda.synchronize()
    sl = lambda x: to64(x[:, :, :T0])  # noqa: E731
    o_ref = oracle.race_forward(sl(q), sl(k), sl(v), planes.double().numpy(), causal=True, inv_temp=it)
    e_out = relerr(sl(out), o_ref)
    print(f"[{name} prefix T0={T0}] out={e_out:.2e}", flush=True)
    assert e_out <= TOL[torch.bfloat16]
    do = torch.zeros_like(q)
    do[:, :, :T0] = torch.randn(1, B, T0, H, D, device=dev, generator=g).to(torch.bfloat16)
    _check_prefix(name, q, k, v, pd, planes, do, state, oracle, seg_tiles)


def test_long_walk_16m(dev, oracle):
    """T = 2^24: 2048 segments of 256 tiles per stream, forward and backward;
    prefix and suffix checks on one set of inputs."""
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    T = 1 << 24
    it = 1.0 / math.sqrt(D)
    q, k, v, planes, g = _inputs(T, dev, 777)
    assert _fwd_segments(q, planes, 0) == T // (32 * MAX_SEG_TILES)
    pd = planes.to(dev)
    name = "long walk T=2^24"
    print(f"[{name}] causal fwd, V mean shift {SHIFT}", flush=True)
    _, state = race_fwd_raw(q, k, v, pd, L=L, K=K, causal=True, inv_temp=it)
    torch.cuda.synchronize()

    do = torch.zeros_like(q)
    do[:, :, :T0] = torch.randn(1, B, T0, H, D, device=dev, generator=g).to(torch.bfloat16)
    print(f"[{name}] backward, dO in the first T0 tokens", flush=True)
    _check_prefix(name, q, k, v, pd, planes, do, state, oracle, 0)

    do.zero_()
    do[:, :, T - T0:] = torch.randn(1, B, T0, H, D, device=dev, generator=g).to(torch.bfloat16)
    print(f"[{name}] backward, dO in the last T0 tokens", flush=True)
    dq, dk, dv, _ = race_bwd_raw(q, k, v, pd, do, state, L=L, K=K, causal=True, inv_temp=it)
    torch.cuda.synchronize()
    assert torch.isfinite(dk).all() and torch.isfinite(dv).all()
    assert not dq[:, :, :T - T0].any(), "dq nonzero before the last T0 tokens"
    del dq
    taus = longseq.sample_taus(T, T0)
    pl0 = planes[0].double().to(dev)
    for h in (0, 6):
        dK_ref, dV_ref = longseq.suffix_reference(q, k, v, do, h, pl0, it, L, K, T0, EPS, taus)
        e_k = relerr(to64(dk[0, 0, taus, h]), dK_ref.cpu().numpy())
        e_v = relerr(to64(dv[0, 0, taus, h]), dV_ref.cpu().numpy())
        print(f"[{name} suffix h={h}, {len(taus)} early tokens] dk={e_k:.2e} dv={e_v:.2e}", flush=True)
        assert max(e_k, e_v) <= TOL[torch.bfloat16]
