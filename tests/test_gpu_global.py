"""GPU parity of the globally normalised causal operator ("F2",
race_fwd_global / race_bwd_global through the C ABI) against the fp64 oracle
on the same seeded inputs and hyperplanes, and of the drop-in
CausalRACEAttention module against a CPU fp64 restatement of the reference
module (misc/elsaa_causal_complete.py:438-586).

Tolerances are the north-star bars, max|a-b|/max|b| <= 1e-4 (fp32) and
<= 2e-2 (bf16 with fp32 accumulation), for out, den, dq, dk, dv; d(beta) is one
sum over all tokens and is compared like F1's temperature gradient (fp32:
|a-b|/|b|; bf16: |a-b| against the l1 mass of its terms)."""
import zlib

import numpy as np
import pytest
import torch

from helpers import TOL, make_case, relerr, to64

pytestmark = pytest.mark.gpu


def _run_gpu(q, k, v, do, dden, planes, *, L, K, beta, dev, seg_tiles=0, floor=1e-6):
    from race_attention_amd.functional import race_global_bwd_raw, race_global_fwd_raw
    qd, kd, vd, dod, pd = [x.to(dev) for x in (q, k, v, do, planes)]
    dd = dden.to(dev) if dden is not None else None
    out, den, state = race_global_fwd_raw(qd, kd, vd, pd, L=L, K=K, beta=beta, floor=floor, seg_tiles=seg_tiles)
    dq, dk, dv, gb = race_global_bwd_raw(qd, kd, vd, pd, out, den, dod, dd, state, L=L, K=K, beta=beta,
                                         floor=floor, seg_tiles=seg_tiles)
    torch.cuda.synchronize()
    return out.cpu(), den.cpu(), dq.cpu(), dk.cpu(), dv.cpu(), float(gb.cpu())


def _run_oracle(q, k, v, do, dden, planes, *, beta, floor=1e-6):
    from oracle import race_oracle as ro
    pl = planes.double().numpy()
    o, den = ro.race_global_forward(to64(q), to64(k), to64(v), pl, beta=beta, floor=floor)
    dq, dk, dv, gb, gabs = ro.race_global_backward(to64(q), to64(k), to64(v), to64(do), pl,
                                                   dden=None if dden is None else to64(dden),
                                                   beta=beta, floor=floor, with_l1=True)
    return o, den, dq, dk, dv, gb, gabs


def _compare(name, gpu, ref, tol):
    names = ("out", "den", "dq", "dk", "dv")
    errs = {nm: relerr(to64(a), b) for nm, a, b in zip(names, gpu[:5], ref[:5])}
    scale = abs(ref[5]) if tol < 1e-3 else ref[6]
    errs["dbeta"] = abs(gpu[5] - ref[5]) / (scale + 1e-30)
    print(f"[{name}] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= tol, f"{name}: {nm} relerr {e:.3e} > {tol:.1e}"


CASES = [
    # name, make_case kwargs, beta, seg_tiles, floor, upstream den gradient
    ("gn_bf16_K4L8", dict(B=2, T=200, H=3, L=8, K=4), 1.0, 0, 1e-6, True),
    ("gn_bf16_K4L8_nodden", dict(T=160, H=2, L=8, K=4), 1.0, 0, 1e-6, False),
    ("gn_bf16_K2L5", dict(T=77, H=2, L=5, K=2), 1.0, 0, 1e-6, True),
    ("gn_bf16_K3L8", dict(T=150, H=2, L=8, K=3), 2.5, 0, 1e-6, True),
    ("gn_bf16_K4L4_beta", dict(T=96, H=1, L=4, K=4, unit=False), 0.3, 0, 1e-6, True),
    ("gn_bf16_manyseg", dict(T=500, H=2, L=8, K=4), 1.0, 1, 1e-6, True),
    ("gn_bf16_M2_indep", dict(M=2, T=90, H=2, L=4, K=4, share_planes=False), 1.0, 0, 1e-6, True),
    ("gn_bf16_T1", dict(T=1, H=2, L=8, K=4), 1.0, 0, 1e-6, True),
    ("gn_bf16_T33", dict(T=33, H=1, L=8, K=4), 1.0, 0, 1e-6, True),
    ("gn_bf16_floor", dict(T=70, H=1, L=4, K=4), 1.0, 0, 1e4, True),
    ("gn_fp32_K2L5", dict(T=130, H=2, L=5, K=2, dtype=torch.float32, unit=False), 1.0, 0, 1e-6, True),
    ("gn_fp32_manyseg", dict(T=300, H=1, L=4, K=3, dtype=torch.float32, unit=False), 0.7, 2, 1e-6, True),
    ("gn_fp32_T31", dict(T=31, H=1, L=5, K=2, dtype=torch.float32, unit=False), 1.0, 0, 1e-6, True),
    ("gn_fp32_floor", dict(T=50, H=1, L=3, K=2, dtype=torch.float32, unit=False), 1.0, 0, 1e4, True),
    # bucket slices: per-slice numerator and den partials, summed then divided
    ("gn_bf16_K5L6_2slices", dict(T=150, H=2, L=6, K=5), 1.0, 0, 1e-6, True),
    ("gn_bf16_K8L4_seg", dict(T=300, H=1, L=4, K=8), 1.0, 2, 1e-6, True),
    ("gn_fp32_K4L8_4slices", dict(T=140, H=2, L=8, K=4, dtype=torch.float32, unit=False), 1.0, 0, 1e-6, True),
    ("gn_fp32_K8L2_16slices", dict(T=70, H=1, L=2, K=8, dtype=torch.float32, unit=False), 0.5, 0, 1e-6, True),
    # whole tiles (T a multiple of 32, every bucket real): the unguarded whole-tile kernels, with the default
    # segmentation and over explicit segments with a short last one
    ("gn_bf16_K4L8_whole", dict(B=2, T=512, H=2, L=8, K=4), 1.0, 0, 1e-6, True),
    ("gn_bf16_K4L8_whole_seg3", dict(T=1024, H=2, L=8, K=4), 0.7, 3, 1e-6, True),
    ("gn_bf16_K8L4_whole_seg4", dict(T=1056, H=2, L=4, K=8), 1.0, 4, 1e-6, True),
    ("gn_bf16_K8L4_whole_nodden", dict(T=256, H=1, L=4, K=8), 1.0, 0, 1e-6, False),
    # values with a mean (B grows linearly in t)
    ("gn_bf16_K4L8_vmean", dict(T=2048, H=2, L=8, K=4, v_shift=0.5), 1.0, 0, 1e-6, True),
]


@pytest.mark.parametrize("name,kw,beta,seg,floor,with_dden", CASES, ids=[c[0] for c in CASES])
def test_global_parity(dev, name, kw, beta, seg, floor, with_dden):
    q, k, v, do, planes = make_case(seed=zlib.crc32(name.encode()) % 1000, **kw)
    M, B, T, H, _ = q.shape
    g = torch.Generator().manual_seed(zlib.crc32(name.encode()) % 777)
    dden = torch.randn(M, B, H, T, generator=g) if with_dden else None
    gpu = _run_gpu(q, k, v, do, dden, planes, L=kw["L"], K=kw["K"], beta=beta, dev=dev, seg_tiles=seg, floor=floor)
    ref = _run_oracle(q, k, v, do, dden, planes, beta=beta, floor=floor)
    _compare(name, gpu, ref, TOL[q.dtype])


# Token 0 sees only its own key, so out_0 = v_0 whatever P_Q is, and with no
# den gradient the exact dq_0 is zero.  Where den_0 is small (sharp beta, q_0
# and k_0 in different buckets) any rounding that keeps dP_Q[0][s] from
# cancelling shows up at full size in dq_0: the kernels form dL/d den from
# their own G, sum_s P_Q G (bucket slices: summed over the slices by a
# pre-pass), for which the cancellation holds to fp32 rounding.  Cases:
# T not a multiple of 32 over several segments (and one whole-tile case),
# independent planes.
FIRST_TOKEN_CASES = [
    ("K4L6_beta2", dict(L=6, K=4), 2.0),
    ("K4L5_beta3", dict(L=5, K=4), 3.0),
    ("K4L8_beta4_whole", dict(L=8, K=4, T=1024), 4.0),
    ("K3L8_beta3_pairs", dict(L=8, K=3), 3.0),
    ("K2L5_beta4_pairs", dict(L=5, K=2), 4.0),
    ("K1L7_beta3_pairs", dict(L=7, K=1), 3.0),
    ("K5L4_beta3_sliced", dict(L=4, K=5), 3.0),
    ("K6L3_beta2_2slices", dict(L=3, K=6), 2.0),
    ("K8L1_beta1_2slices", dict(L=1, K=8), 1.0),
    ("K8L4_beta2_8slices_whole", dict(L=4, K=8, T=1024), 2.0),
]


@pytest.mark.parametrize("name,kw,beta", FIRST_TOKEN_CASES, ids=[c[0] for c in FIRST_TOKEN_CASES])
def test_global_first_token_gradient(dev, name, kw, beta):
    args = dict(M=2, B=1, T=318, H=3, seed=58004, share_planes=False)
    args.update(kw)
    q, k, v, do, planes = make_case(**args)
    gpu = _run_gpu(q, k, v, do, None, planes, L=kw["L"], K=kw["K"], beta=beta, dev=dev, seg_tiles=3)
    ref = _run_oracle(q, k, v, do, None, planes, beta=beta)
    scale = np.abs(ref[2]).max()
    first = np.abs(to64(gpu[2])[:, :, 0]).max() / scale
    print(f"[{name}] |dq_0| / max|dq| = {first:.2e}", flush=True)
    assert np.abs(ref[2][:, :, 0]).max() <= 1e-12 * scale  # the oracle's zero
    assert first <= 1e-5, f"{name}: dq at t = 0 is {first:.2e} of max|dq|"
    _compare("first_token_" + name, gpu, ref, TOL[q.dtype])


@pytest.mark.parametrize("kw", [dict(T=200, H=2, L=8, K=4), dict(T=150, H=2, L=3, K=6),
                                dict(T=96, H=1, L=4, K=3, dtype=torch.float32, unit=False)],
                         ids=["K4_one_workgroup", "K6_slices", "fp32_slices"])
def test_global_backward_does_not_read_out(dev, kw):
    """dL/d den comes from the kernels' own sums, so the backward's result is
    the same, bit for bit, when the out argument holds NaN instead of the
    forward's output."""
    from race_attention_amd.functional import race_global_bwd_raw, race_global_fwd_raw
    q, k, v, do, planes = [x.to(dev) for x in make_case(seed=9, **kw)]
    M, B, T, H, _ = q.shape
    dden = torch.randn(M, B, H, T, generator=torch.Generator().manual_seed(2)).to(dev)
    L, K = kw["L"], kw["K"]
    out, den, state = race_global_fwd_raw(q, k, v, planes, L=L, K=K, beta=2.0)
    a = race_global_bwd_raw(q, k, v, planes, out, den, do, dden, state, L=L, K=K, beta=2.0)
    b = race_global_bwd_raw(q, k, v, planes, torch.full_like(out, float("nan")), den, do, dden, state, L=L, K=K,
                            beta=2.0)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_global_deterministic(dev):
    q, k, v, do, planes = make_case(B=1, T=333, H=2, L=8, K=4, seed=3)
    dden = torch.randn(1, 1, 2, 333, generator=torch.Generator().manual_seed(1))
    a = _run_gpu(q, k, v, do, dden, planes, L=8, K=4, beta=1.0, dev=dev)
    b = _run_gpu(q, k, v, do, dden, planes, L=8, K=4, beta=1.0, dev=dev)
    for x, y in zip(a[:5], b[:5]):
        assert torch.equal(x, y)
    assert a[5] == b[5]


def test_global_constant_values(dev):
    """v = c gives out = c exactly in the mathematics (num = c den)."""
    q, k, _, do, planes = make_case(B=1, T=257, H=2, L=8, K=4, seed=5, dtype=torch.float32, unit=False)
    v = torch.full_like(q, 0.375)
    out, den, *_ = _run_gpu(q, k, v, do, None, planes, L=8, K=4, beta=1.0, dev=dev)
    assert torch.allclose(out, v, rtol=0, atol=2e-6)
    assert (den > 0).all()


def test_config_c2_global(dev):
    """C2's shape (causal bf16, B=2 H=8 N=16384 d=64 K=4 L=8, unit-L2 rows)
    in the globally normalised mode, beta = 1 (the module's beta_init)."""
    q, k, v, do, planes = make_case(B=2, T=16384, H=8, L=8, K=4, seed=12)
    dden = torch.randn(1, 2, 8, 16384, generator=torch.Generator().manual_seed(2))
    gpu = _run_gpu(q, k, v, do, dden, planes, L=8, K=4, beta=1.0, dev=dev)
    ref = _run_oracle(q, k, v, do, dden, planes, beta=1.0)
    _compare("C2_global", gpu, ref, 2e-2)


@pytest.mark.parametrize("with_mask", [False, True])
def test_causal_race_attention_module(dev, with_mask):
    """CausalRACEAttention on the GPU in fp32 against the fp64 restatement of
    the reference module: out, d_token and the gradients of x, the Linear
    weights and log_beta for loss = sum(out G) + sum(d_token h)."""
    from f2_torch_ref import module_forward
    from race_attention_amd.causal import CausalRACEAttention
    torch.manual_seed(0)
    B, T, d, h = 2, 150, 128, 2
    m = CausalRACEAttention(d, h, drop=0.0, num_bits=4, num_tables=4, beta_init=1.3)
    x = torch.randn(B, T, d)
    mask = (torch.arange(T)[None, :] < torch.tensor([[T], [T - 37]])).float() if with_mask else None
    G = torch.randn(B, T, d)
    hd = torch.randn(B, T, 1)
    ref_out, ref_dt, leaves = module_forward(m, x, mask)
    ((ref_out * G.double()).sum() + (ref_dt * hd.double()).sum()).backward()

    md = m.to(dev)
    xd = x.to(dev).requires_grad_(True)
    out, dt = md(xd, mask=mask.to(dev) if mask is not None else None, return_den=True)
    ((out * G.to(dev)).sum() + (dt * hd.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    errs = {"out": relerr(out.detach().cpu(), ref_out.detach()), "d_token": relerr(dt.detach().cpu(), ref_dt.detach()),
            "x.grad": relerr(xd.grad.cpu(), leaves["x"].grad)}
    for n, p in md.named_parameters():
        if n != "log_beta":
            errs[n] = relerr(p.grad.cpu(), leaves[n].grad)
    # d log_beta = beta * (sum over every token and hash column of du * th):
    # one sum whose terms cancel, compared against its l1 mass (the oracle's
    # sum |du * th| for the core's own inputs and upstream gradients) times beta
    from oracle import race_oracle as ro
    Qc, Kc, Vc, oc, denc, beta = leaves["_core"]
    lay = lambda z: z.detach().permute(0, 2, 1, 3).unsqueeze(0).numpy()  # noqa: E731  [B,H,T,dk] -> [1,B,T,H,dk]
    *_, gb, gabs = ro.race_global_backward(lay(Qc), lay(Kc), lay(Vc), lay(oc.grad),
                                           md.planes.detach().double().cpu().unsqueeze(0).numpy(),
                                           dden=denc.grad.unsqueeze(0).numpy(), beta=beta, with_l1=True)
    assert abs(gb * beta - float(leaves["log_beta"].grad)) <= 1e-9 * gabs * beta
    errs["log_beta"] = abs(float(md.log_beta.grad) - float(leaves["log_beta"].grad)) / (gabs * beta)
    print("[CausalRACEAttention] " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert torch.equal(md.last_den, dt.detach())
    for nm, e in errs.items():
        assert e <= 1e-4, f"{nm}: {e:.3e}"
