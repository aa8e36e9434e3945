"""The backward's own segmentation.  With seg_tiles = 0 the backward plan
joins fmul forward segments into one (fewer, longer workgroups; its
boundaries are forward boundaries, so it reads the forward state rows
s * fmul and min((s + 1) * fmul, fnseg)).  At B=1, H=4, N=8192 the forward
runs 256 one-tile segments per stream (bf16; fp32, with four bucket slices,
128 two-tile ones) and the backward 128 two-tile (bf16) or 32 eight-tile
(fp32) segments.

Checked: the auto plan against the same backward on the forward's
segmentation (explicit seg_tiles), and against the fp64 oracle for F1
(bars 1e-4 fp32, 2e-2 bf16); F2 and the padded-batch forms against the
explicit segmentation.  The workspace query shows the coarser plan."""
import ctypes
import math

import pytest
import torch

from helpers import TOL, make_case, relerr, to64

pytestmark = pytest.mark.gpu

B, T, H, L, K = 1, 8192, 4, 8, 4


def _desc(dtype_id, causal, seg):
    from race_attention_amd import _lib
    d = _lib.RaceDesc()
    d.M, d.B, d.T, d.H, d.D = 1, B, T, H, 64
    d.L, d.K, d.causal, d.dtype = L, K, causal, dtype_id
    d.eps, d.inv_temp = 1e-6, 0.125
    for j in range(4):
        d.q_stride[j] = d.k_stride[j] = d.v_stride[j] = d.o_stride[j] = d.do_stride[j] = d.g_stride[j] = 0
    for arr in (d.q_stride, d.k_stride, d.v_stride, d.o_stride, d.do_stride, d.g_stride):
        arr[2] = H * 64
        arr[3] = 64
    d.seg_tiles = seg
    return d


def _bwd_ws(dtype_id, causal, seg):
    from race_attention_amd import _lib
    return _lib.load().race_bwd_workspace_bytes(ctypes.byref(_desc(dtype_id, causal, seg)))


def _fwd_tps(dtype_id, causal):
    """Tiles per segment of the automatic forward plan, from its state size
    ([N][nseg+1][Spad][D+1] fp64)."""
    from race_attention_amd import _lib
    sb = _lib.load().race_state_bytes(ctypes.byref(_desc(dtype_id, causal, 0)))
    spad = 128
    nseg = sb // (H * spad * 65 * 8) - 1
    ntiles = T // 32
    return -(-ntiles // nseg)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "noncausal"])
def test_coarser_backward_segments(dev, dtype, causal):
    from oracle import race_oracle as ro
    from race_attention_amd import _lib
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    did = _lib.RACE_DTYPE_BF16 if dtype == torch.bfloat16 else _lib.RACE_DTYPE_F32
    tps = _fwd_tps(did, int(causal))  # explicit, the backward keeps the forward's segments
    # the auto backward plan has fewer segments than the forward's
    assert _bwd_ws(did, int(causal), 0) < _bwd_ws(did, int(causal), tps)
    q, k, v, do, planes = make_case(B=B, T=T, H=H, L=L, K=K, dtype=dtype, seed=11, unit=dtype == torch.bfloat16)
    it = 1.0 / math.sqrt(64) if causal else 0.8
    qd, kd, vd, dod, pd = [x.to(dev) for x in (q, k, v, do, planes)]
    out, st = race_fwd_raw(qd, kd, vd, pd, L=L, K=K, causal=causal, inv_temp=it)
    auto = race_bwd_raw(qd, kd, vd, pd, dod, st, L=L, K=K, causal=causal, inv_temp=it)
    fine = race_bwd_raw(qd, kd, vd, pd, dod, st, L=L, K=K, causal=causal, inv_temp=it, seg_tiles=tps)
    torch.cuda.synchronize()
    pl = planes.double().numpy()
    ref = ro.race_backward(to64(q), to64(k), to64(v), to64(do), pl, causal=causal, inv_temp=it, with_l1=True)
    tol = TOL[dtype]
    for nm, a, f, r in zip(("dq", "dk", "dv"), auto[:3], fine[:3], ref[:3]):
        ea, ef, eaf = relerr(to64(a), r), relerr(to64(f), r), relerr(to64(a), to64(f))
        print(f"[{dtype} causal={causal}] {nm}: auto {ea:.2e} fine {ef:.2e} auto-vs-fine {eaf:.2e}", flush=True)
        assert ea <= tol and eaf <= tol, nm
    ga, gf = float(auto[3].cpu()), float(fine[3].cpu())
    scale = abs(ref[3]) if dtype == torch.float32 else ref[4]
    assert abs(ga - ref[3]) <= tol * scale and abs(ga - gf) <= tol * scale


def test_coarser_backward_segments_global(dev):
    """F2 (causal, bf16): auto backward plan against the forward's segmentation."""
    from race_attention_amd.functional import race_global_bwd_raw, race_global_fwd_raw
    q, k, v, do, planes = make_case(B=B, T=T, H=H, L=L, K=K, seed=12)
    qd, kd, vd, dod, pd = [x.to(dev) for x in (q, k, v, do, planes)]
    dden = torch.randn(1, B, H, T, generator=torch.Generator().manual_seed(5)).to(dev)
    out, den, st = race_global_fwd_raw(qd, kd, vd, pd, L=L, K=K, beta=1.0)
    auto = race_global_bwd_raw(qd, kd, vd, pd, out, den, dod, dden, st, L=L, K=K, beta=1.0)
    fine = race_global_bwd_raw(qd, kd, vd, pd, out, den, dod, dden, st, L=L, K=K, beta=1.0, seg_tiles=1)
    torch.cuda.synchronize()
    for nm, a, f in zip(("dq", "dk", "dv"), auto[:3], fine[:3]):
        e = relerr(to64(a), to64(f))
        print(f"[global] {nm}: auto-vs-fine {e:.2e}", flush=True)
        assert e <= TOL[torch.bfloat16], nm


def test_coarser_backward_segments_ex(dev):
    """Padded batch (non-causal, bf16, key weights and a den gradient): auto
    backward plan against the forward's segmentation."""
    from race_attention_amd.functional import race_bwd_ex_raw, race_fwd_ex_raw
    q, k, v, do, planes = make_case(B=B, T=T, H=H, L=L, K=K, seed=13)
    g = torch.Generator().manual_seed(6)
    km = (torch.rand(B, T, generator=g) > 0.2).float()
    dden = torch.randn(1, B, H, T, generator=g)
    qd, kd, vd, dod, pd, kmd, ddd = [x.to(dev) for x in (q, k, v, do, planes, km, dden)]
    out, den, st = race_fwd_ex_raw(qd, kd, vd, pd, L=L, K=K, inv_temp=0.8, kmask=kmd, want_den=True)
    auto = race_bwd_ex_raw(qd, kd, vd, pd, dod, ddd, st, L=L, K=K, inv_temp=0.8, kmask=kmd)
    fine = race_bwd_ex_raw(qd, kd, vd, pd, dod, ddd, st, L=L, K=K, inv_temp=0.8, kmask=kmd, seg_tiles=1)
    torch.cuda.synchronize()
    for nm, a, f in zip(("dq", "dk", "dv"), auto[:3], fine[:3]):
        e = relerr(to64(a), to64(f))
        print(f"[ex] {nm}: auto-vs-fine {e:.2e}", flush=True)
        assert e <= TOL[torch.bfloat16], nm
