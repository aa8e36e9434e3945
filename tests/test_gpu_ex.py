"""GPU parity of the padded-batch / denominator-proxy forms of the
non-causal operator (race_fwd_ex / race_bwd_ex through the C ABI: key
weights on P_K, the den output and its gradient) against the fp64 oracle,
and of the module mirrors (classification.RACEAttention /
RACEAttentionWithDenom, vit.RACEAttentionWithDenom) against an fp64 torch
restatement of the reference modules (misc/classification.py:520-683,
misc/vit.py:1441-1543).  Bars: max|a-b|/max|b| <= 1e-4 (fp32), <= 2e-2 (bf16)."""
import zlib

import pytest
import torch

from helpers import TOL, make_case, relerr, to64

pytestmark = pytest.mark.gpu


def _masks(kind, B, T, g):
    if kind is None:
        return None
    m = torch.ones(B, T)
    if kind == "binary":
        m[0, T - T // 3:] = 0                                   # trailing padding
        if B > 1:
            m[1, torch.randperm(T, generator=g)[: T // 4]] = 0  # scattered
    else:
        m = torch.rand(B, T, generator=g) * 1.5 + 0.1           # fractional key weights
    return m


def _run(q, k, v, do, planes, *, L, K, it, kmask, dden, dev, seg=0):
    from race_attention_amd.functional import race_bwd_ex_raw, race_fwd_ex_raw
    qd, kd, vd, dod, pd = [x.to(dev) for x in (q, k, v, do, planes)]
    km = kmask.to(dev) if kmask is not None else None
    out, den, st = race_fwd_ex_raw(qd, kd, vd, pd, L=L, K=K, inv_temp=it, kmask=km, want_den=True, seg_tiles=seg)
    dq, dk, dv, git = race_bwd_ex_raw(qd, kd, vd, pd, dod, dden.to(dev) if dden is not None else None, st, L=L,
                                      K=K, inv_temp=it, kmask=km, seg_tiles=seg)
    torch.cuda.synchronize()
    return out.cpu(), den.cpu(), dq.cpu(), dk.cpu(), dv.cpu(), float(git.cpu())


CASES = [
    # name, make_case kwargs, inv_temp, mask kind, upstream den gradient, seg_tiles
    ("ex_bf16_K4L8_binary", dict(B=2, T=150, H=2, L=8, K=4), 1.0, "binary", True, 0),
    ("ex_bf16_K2L5_frac", dict(B=2, T=97, H=2, L=5, K=2), 0.7, "frac", True, 0),
    ("ex_bf16_K3L4_nomask", dict(B=1, T=120, H=3, L=4, K=3), 1.0, None, True, 0),
    ("ex_bf16_K4L8_seg", dict(B=2, T=300, H=1, L=8, K=4), 1.0, "binary", True, 2),
    ("ex_bf16_K8L2_slices", dict(B=2, T=90, H=1, L=2, K=8), 1.0, "binary", True, 0),
    ("ex_bf16_M2_indep", dict(M=2, B=2, T=64, H=2, L=5, K=2, share_planes=False), 1.0, "binary", False, 0),
    ("ex_fp32_K2L5_binary", dict(B=2, T=130, H=2, L=5, K=2, dtype=torch.float32, unit=False), 1.0, "binary", True, 0),
    ("ex_fp32_K4L8_4slices", dict(B=2, T=140, H=2, L=8, K=4, dtype=torch.float32, unit=False), 0.5, "frac", True, 0),
    ("ex_fp32_seg", dict(B=2, T=257, H=1, L=5, K=2, dtype=torch.float32, unit=False), 1.0, "binary", True, 3),
]


@pytest.mark.parametrize("name,kw,it,mk,with_dden,seg", CASES, ids=[c[0] for c in CASES])
def test_ex_parity(dev, name, kw, it, mk, with_dden, seg):
    from oracle import race_oracle as ro
    q, k, v, do, planes = make_case(seed=zlib.crc32(name.encode()) % 1000, **kw)
    M, B, T, H, _ = q.shape
    g = torch.Generator().manual_seed(zlib.crc32(name.encode()) % 997)
    kmask = _masks(mk, B, T, g)
    dden = torch.randn(M, B, H, T, generator=g) if with_dden else None
    gpu = _run(q, k, v, do, planes, L=kw["L"], K=kw["K"], it=it, kmask=kmask, dden=dden, dev=dev, seg=seg)
    pl = planes.double().numpy()
    km = kmask.double().numpy() if kmask is not None else None
    o, den = ro.race_forward_ex(to64(q), to64(k), to64(v), pl, kmask=km, causal=False, inv_temp=it)
    dq, dk, dv, git, gabs = ro.race_backward_ex(to64(q), to64(k), to64(v), to64(do), pl, kmask=km,
                                                dden=to64(dden) if dden is not None else None, causal=False,
                                                inv_temp=it, with_l1=True)
    errs = {nm: relerr(to64(a), b) for nm, a, b in zip(("out", "den", "dq", "dk", "dv"), gpu[:5],
                                                        (o, den, dq, dk, dv))}
    tol = TOL[q.dtype]
    errs["dinv_temp"] = abs(gpu[5] - git) / ((abs(git) if tol < 1e-3 else gabs) + 1e-30)
    print(f"[{name}] " + " ".join(f"{a}={b:.2e}" for a, b in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= tol, f"{name}: {nm} {e:.3e} > {tol:.1e}"


def test_ex_without_extras_equals_race_fwd(dev):
    """No key weights and no den: bit-identical to race_fwd / race_bwd."""
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw, race_bwd_ex_raw, race_fwd_ex_raw
    q, k, v, do, planes = [x.to(dev) for x in make_case(B=1, T=200, H=2, L=8, K=4, seed=4)]
    o1, s1 = race_fwd_raw(q, k, v, planes, L=8, K=4, causal=False, inv_temp=1.0)
    g1 = race_bwd_raw(q, k, v, planes, do, s1, L=8, K=4, causal=False, inv_temp=1.0)
    o2, den, s2 = race_fwd_ex_raw(q, k, v, planes, L=8, K=4, inv_temp=1.0)
    g2 = race_bwd_ex_raw(q, k, v, planes, do, None, s2, L=8, K=4, inv_temp=1.0)
    assert den is None and torch.equal(o1, o2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def _module_errs(mod_gpu, out, dt, ref_out, ref_dt, leaves, xd):
    """relerr of out, d_token and every gradient; d logit_temp (one sum of
    cancelling terms) against the l1 mass of its terms."""
    from f1_torch_ref import temp_grad_l1
    errs = {"out": relerr(out.detach().cpu(), ref_out.detach()), "d_token": relerr(dt.detach().cpu(), ref_dt.detach()),
            "x.grad": relerr(xd.grad.cpu(), leaves["x"].grad)}
    for n, p in mod_gpu.named_parameters():
        if n.endswith("logit_temp"):
            assert abs(float(leaves[n].grad)) <= temp_grad_l1(leaves) * (1 + 1e-12)
            errs[n] = abs(float(p.grad) - float(leaves[n].grad)) / temp_grad_l1(leaves)
        else:
            errs[n] = relerr(p.grad.cpu(), leaves[n].grad)
    return errs


@pytest.mark.parametrize("with_mask", [False, True])
def test_classification_with_denom_module(dev, with_mask):
    """classification.RACEAttentionWithDenom (fp32) against the fp64
    restatement: out, d_race_token and every gradient."""
    from f1_torch_ref import classification_with_denom
    from race_attention_amd.classification import RACEAttentionWithDenom
    torch.manual_seed(1)
    B, T, d, h = 2, 120, 128, 2
    m = RACEAttentionWithDenom(d, h, 0.0, M=2, K=3, L=2)
    x = torch.randn(B, T, d)
    mask = (torch.arange(T)[None, :] < torch.tensor([[T], [T - 29]])).float() if with_mask else None
    G, hd = torch.randn(B, T, d), torch.randn(B, T, 1)
    ref_out, ref_dt, leaves = classification_with_denom(m, x, mask)
    ((ref_out * G.double()).sum() + (ref_dt * hd.double()).sum()).backward()
    md = m.to(dev)
    xd = x.to(dev).requires_grad_(True)
    out, dt = md(xd, mask.to(dev) if mask is not None else None)
    ((out * G.to(dev)).sum() + (dt * hd.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    errs = _module_errs(md, out, dt, ref_out, ref_dt, leaves, xd)
    print(f"[classification.RACEAttentionWithDenom mask={with_mask}] " +
          " ".join(f"{a}={b:.2e}" for a, b in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= 1e-4, f"{nm}: {e:.3e}"


def test_classification_attention_module(dev):
    """classification.RACEAttention(x, mask) (fp32): the padded-batch module
    without the den output, against the same restatement's output."""
    from f1_torch_ref import classification_with_denom
    from race_attention_amd.classification import RACEAttention
    torch.manual_seed(3)
    B, T, d, h = 2, 90, 128, 2
    m = RACEAttention(d, h, 0.0, M=2, K=2, L=5, qkv_bias=True)
    x = torch.randn(B, T, d)
    mask = torch.ones(B, T)
    mask[0, 70:] = 0
    mask[1, ::7] = 0
    G = torch.randn(B, T, d)
    ref_out, _, leaves = classification_with_denom(m, x, mask)
    (ref_out * G.double()).sum().backward()
    md = m.to(dev)
    xd = x.to(dev).requires_grad_(True)
    out = md(xd, mask.to(dev))
    (out * G.to(dev)).sum().backward()
    torch.cuda.synchronize()
    errs = {"out": relerr(out.detach().cpu(), ref_out.detach()), "x.grad": relerr(xd.grad.cpu(), leaves["x"].grad)}
    for n, p in md.named_parameters():
        if not n.endswith("logit_temp"):
            errs[n] = relerr(p.grad.cpu(), leaves[n].grad)
    print("[classification.RACEAttention] " + " ".join(f"{a}={b:.2e}" for a, b in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= 1e-4, f"{nm}: {e:.3e}"


def test_vit_with_denom_module(dev):
    """vit.RACEAttentionWithDenom (fp32, the reference head merge) against the
    fp64 restatement of misc/vit.py:1441-1543."""
    from f1_torch_ref import vit_with_denom
    from race_attention_amd.vit import RACEAttentionWithDenom
    torch.manual_seed(2)
    B, T, d, h = 2, 100, 128, 2
    m = RACEAttentionWithDenom(d, d, 0.0, h, 3, 2, 2)
    x = torch.randn(B, T, d)
    G, hd = torch.randn(B, T, d), torch.randn(B, T, 1)
    ref_out, ref_dt, leaves = vit_with_denom(m, x)
    ((ref_out * G.double()).sum() + (ref_dt * hd.double()).sum()).backward()
    md = m.to(dev)
    xd = x.to(dev).requires_grad_(True)
    out, dt = md(xd)
    ((out * G.to(dev)).sum() + (dt * hd.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    errs = _module_errs(md, out, dt, ref_out, ref_dt, leaves, xd)
    print("[vit.RACEAttentionWithDenom] " + " ".join(f"{a}={b:.2e}" for a, b in errs.items()), flush=True)
    for nm, e in errs.items():
        assert e <= 1e-4, f"{nm}: {e:.3e}"
