"""GPU parity: the HIP operator (through the C ABI) against the fp64 oracle on
the same seeded inputs and hyperplanes.  Tolerances are the north-star bars,
max|a-b|/max|b| <= 1e-4 (fp32) and <= 2e-2 (bf16 with fp32 accumulation)."""
import ctypes
import math
import os
import zlib

import numpy as np
import pytest
import torch

from helpers import TOL, compare, make_case, relerr, run_gpu, run_oracle, to64

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _probe_lib():
    lib = ctypes.CDLL(os.path.join(HERE, "hip", "libmfma_probe.so"))
    lib.probe_mfma.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 5
    lib.probe_rows.argtypes = [ctypes.c_void_p] * 2
    lib.probe_chain.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 5
    lib.probe_chain16.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 5
    lib.probe_xor.argtypes = [ctypes.c_void_p] * 2
    return lib


def test_permlane_xor_sums(dev):
    """xor16_sum / xor32_sum (v_permlane16/32_swap) equal x + x[lane^16|32]."""
    lib = _probe_lib()
    x = torch.randn(64, generator=torch.Generator().manual_seed(9)).to(dev)
    out = torch.zeros(128, device=dev)
    assert lib.probe_xor(x.data_ptr(), out.data_ptr()) == 0
    xc = x.cpu()
    idx = torch.arange(64)
    assert torch.allclose(out[:64].cpu(), xc + xc[idx ^ 16], atol=1e-6)
    assert torch.allclose(out[64:].cpu(), xc + xc[idx ^ 32], atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mfma_chain16(dev, dtype):
    """One accumulator tile reused as a 16-deep operand (16x16x16 MFMA)."""
    lib = _probe_lib()
    g = torch.Generator().manual_seed(4)
    A = torch.randn(16, 64, generator=g).to(dtype)
    Bm = torch.randn(16, 64, generator=g).to(dtype)
    E = torch.randn(16, 16, generator=g).to(dtype)
    D, Dt = torch.zeros(16, 16, device=dev), torch.zeros(16, 16, device=dev)
    assert lib.probe_chain16(int(dtype == torch.bfloat16), A.to(dev).data_ptr(), Bm.to(dev).data_ptr(),
                             E.to(dev).data_ptr(), D.data_ptr(), Dt.data_ptr()) == 0
    X = A.double() @ Bm.double().T
    if dtype == torch.bfloat16:
        X = X.to(torch.bfloat16).double()
    ref = E.double() @ X
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert relerr(D.cpu(), ref) < tol
    assert relerr(Dt.cpu(), ref.T) < tol


def test_dpp_row_scans(dev):
    """16-lane row prefix/suffix/total/broadcast helpers (in-bounds, one wave)."""
    lib = _probe_lib()
    x = torch.randn(64, generator=torch.Generator().manual_seed(2)).to(dev)
    out = torch.zeros(256, device=dev)
    assert lib.probe_rows(x.data_ptr(), out.data_ptr()) == 0
    rows = x.cpu().double().view(4, 16)
    pre = torch.cumsum(rows, 1).reshape(-1)
    suf = torch.flip(torch.cumsum(torch.flip(rows, [1]), 1), [1]).reshape(-1)
    tot = rows.sum(1, keepdim=True).expand(4, 16).reshape(-1)
    o = out.cpu().double()
    assert torch.allclose(o[:64], pre, atol=1e-5)
    assert torch.allclose(o[64:128], suf, atol=1e-5)
    assert torch.allclose(o[128:192], tot, atol=1e-5)
    assert torch.equal(o[192:], rows[:, :1].expand(4, 16).reshape(-1))  # row_newbcast:0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mfma_chain_pi_order(dev, dtype):
    """Accumulator tiles reused as the next MFMA's operand (pi-ordered k)."""
    lib = _probe_lib()
    g = torch.Generator().manual_seed(3)
    A = torch.randn(32, 64, generator=g).to(dtype)
    Bm = torch.randn(16, 64, generator=g).to(dtype)
    E = torch.randn(16, 32, generator=g).to(dtype)
    D, Dt = torch.zeros(16, 16, device=dev), torch.zeros(16, 16, device=dev)
    assert lib.probe_chain(int(dtype == torch.bfloat16), A.to(dev).data_ptr(), Bm.to(dev).data_ptr(),
                           E.to(dev).data_ptr(), D.data_ptr(), Dt.data_ptr()) == 0
    X = A.double() @ Bm.double().T
    if dtype == torch.bfloat16:
        X = X.to(torch.bfloat16).double()      # the chained operand is rounded to bf16
    ref = E.double() @ X
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert relerr(D.cpu(), ref) < tol
    assert relerr(Dt.cpu(), ref.T) < tol


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mfma_fragment_layout(dev, dtype):
    """Row/column mapping of the 16x16 MFMA helpers (in-bounds, one wave)."""
    lib = _probe_lib()
    g = torch.Generator().manual_seed(1)
    A = torch.randn(16, 64, generator=g).to(dtype)
    B = torch.randn(16, 64, generator=g).to(dtype)
    Ad, Bd = A.to(dev).contiguous(), B.to(dev).contiguous()
    C, Cbt, Ct = [torch.zeros(16, 16, device=dev) for _ in range(3)]
    assert lib.probe_mfma(int(dtype == torch.bfloat16), Ad.data_ptr(), Bd.data_ptr(), C.data_ptr(),
                          Cbt.data_ptr(), Ct.data_ptr()) == 0
    ref = A.double() @ B.double().T
    tol = 1e-5 if dtype == torch.float32 else 1e-4
    assert relerr(C.cpu(), ref) < tol
    assert relerr(Cbt.cpu(), ref) < tol
    assert relerr(Ct.cpu(), ref.T) < tol


CASES = [
    # name, dict(make_case kwargs), causal, inv_temp (None -> 1/sqrt(D)), seg_tiles
    ("causal_bf16_K4L8", dict(B=2, T=200, H=3, L=8, K=4), True, None, 0),
    ("causal_bf16_K2L5", dict(T=77, H=2, L=5, K=2), True, None, 0),
    ("causal_bf16_K3L8", dict(T=150, H=2, L=8, K=3), True, None, 0),
    ("causal_bf16_K4L8_tau1", dict(T=96, H=1, L=8, K=4, unit=False), True, 1.0, 0),
    ("causal_bf16_manyseg", dict(T=500, H=2, L=8, K=4), True, None, 1),
    ("causal_bf16_seg3", dict(T=700, H=1, L=5, K=2), True, None, 3),
    ("causal_fp32_K2L5", dict(T=130, H=2, L=5, K=2, dtype=torch.float32, unit=False), True, 1.0, 0),
    ("causal_fp32_manyseg", dict(T=300, H=1, L=4, K=3, dtype=torch.float32, unit=False), True, 0.5, 2),
    ("noncausal_fp32_K2L5", dict(T=300, H=2, L=5, K=2, dtype=torch.float32, unit=False), False, 1.0, 0),
    ("noncausal_fp32_seg", dict(T=257, H=1, L=5, K=2, dtype=torch.float32, unit=False), False, 0.7, 2),
    ("noncausal_bf16_K4L8", dict(T=100, H=2, L=8, K=4), False, 1.0, 0),
    ("causal_bf16_M2_expand", dict(M=2, T=90, H=2, L=8, K=4, expand_m=True), True, None, 0),
    ("noncausal_fp32_M2_indep", dict(M=2, T=64, H=1, L=5, K=2, dtype=torch.float32, unit=False,
                                     share_planes=False), False, 1.0, 0),
    # T=1 with eps=1e-6 is ill-conditioned for dQ/dK: every one of their terms
    # carries a factor eps/(P+eps) (e.g. alpha + v.U = W (g.v) eps/(P_K+eps)),
    # so O(1) rounding swamps an O(1e-5) answer in any precision.  The T=1
    # path is checked with eps=0.5, where those gradients are O(1); the
    # reference eps is exercised from T=2 on.
    ("causal_fp32_T1_eps", dict(T=1, H=1, L=5, K=2, dtype=torch.float32, unit=False, eps=0.5), True, 1.0, 0),
    ("causal_bf16_T1_eps", dict(T=1, H=2, L=8, K=4, eps=0.5), True, None, 0),
    ("causal_bf16_T2", dict(T=2, H=1, L=8, K=4), True, None, 0),
    ("noncausal_fp32_T2", dict(T=2, H=1, L=5, K=2, dtype=torch.float32, unit=False), False, 1.0, 0),
    ("causal_bf16_T32", dict(T=32, H=1, L=8, K=4), True, None, 0),
    ("causal_bf16_T33", dict(T=33, H=1, L=8, K=4), True, None, 0),
    ("causal_fp32_T31", dict(T=31, H=1, L=5, K=2, dtype=torch.float32, unit=False), True, 1.0, 0),
    # Bucket slices (grid z): bf16 with 2^K > 16 runs slices of 128 buckets,
    # fp32 slices of 32; partial outputs are summed per slice.  A table can
    # span several waves (K=5, 6), fill a slice (K=7) or span several slices
    # (K=8), and the last slice can be partly padding.
    ("causal_bf16_K5L6_2slices", dict(T=150, H=2, L=6, K=5), True, None, 0),
    ("noncausal_bf16_K6L3_pad", dict(T=120, H=1, L=3, K=6), False, 1.0, 0),
    ("causal_bf16_K7L1_1slice", dict(T=64, H=1, L=1, K=7), True, None, 0),
    ("causal_bf16_K8L4_M2", dict(M=2, T=100, H=2, L=4, K=8, share_planes=False), True, None, 0),
    ("causal_bf16_K8L4_seg", dict(T=300, H=1, L=4, K=8), True, None, 2),
    ("noncausal_bf16_K8L2", dict(T=90, H=2, L=2, K=8), False, None, 0),
    ("causal_fp32_K4L8_4slices", dict(T=140, H=2, L=8, K=4, dtype=torch.float32, unit=False), True, 1.0, 0),
    ("causal_fp32_K3L5_pad", dict(T=90, H=1, L=5, K=3, dtype=torch.float32, unit=False), True, 0.5, 0),
    ("noncausal_fp32_K5L3", dict(T=100, H=1, L=3, K=5, dtype=torch.float32, unit=False), False, 1.0, 2),
    ("causal_fp32_K8L2_16slices", dict(T=70, H=1, L=2, K=8, dtype=torch.float32, unit=False), True, 0.5, 0),
    # Whole tiles (T a multiple of 32, every bucket real) run the unguarded
    # whole-tile kernels; with an explicit seg_tiles the backward keeps the
    # forward's segments, so these walk several backward segments with carries
    # and prefetches across segment edges and a short last segment: K=8
    # (33 tiles in 9 segments, the last of one tile) and K=4 (32 tiles in
    # 11 segments, the last of two).
    ("causal_bf16_K8L4_whole_seg4", dict(T=1056, H=2, L=4, K=8), True, None, 4),
    ("causal_bf16_K4L8_whole_seg3", dict(T=1024, H=2, L=8, K=4), True, None, 3),
    # values with a mean (V = normalize(N(0,1) + 0.5)): B grows linearly in t, the case that exposes walks of
    # the forward state that are too long, and the one where the bf16 B operand weighs most (error budget)
    ("causal_bf16_K4L8_vmean", dict(T=2048, H=2, L=8, K=4, v_shift=0.5), True, None, 0),
    ("causal_bf16_K4L8_vmean_seg256", dict(T=8192, H=1, L=8, K=4, v_shift=0.5), True, None, 256),
    ("causal_bf16_K8L4_vmean", dict(T=1024, H=2, L=4, K=8, v_shift=0.5), True, None, 0),
    ("causal_fp32_K4L8_vmean_seg", dict(T=1500, H=1, L=8, K=4, dtype=torch.float32, v_shift=0.5), True, None, 40),
    ("noncausal_bf16_K4L8_vmean", dict(T=600, H=2, L=8, K=4, v_shift=0.5), False, 1.0, 0),
    # 8-bit hashes with one table (2 slices: k_dx_finish8 with one live table) and three (6 slices: the
    # generic slice sum), whole tiles and ragged
    ("causal_bf16_K8L1_whole", dict(T=640, H=2, L=1, K=8), True, None, 0),
    ("causal_bf16_K8L3_ragged", dict(T=333, H=2, L=3, K=8), True, None, 3),
]


@pytest.mark.parametrize("name,kw,causal,it,seg", CASES, ids=[c[0] for c in CASES])
def test_parity_small(dev, name, kw, causal, it, seg):
    kw = dict(kw)
    eps = kw.pop("eps", 1e-6)
    q, k, v, do, planes = make_case(seed=zlib.crc32(name.encode()) % 1000, **kw)
    L, K = kw["L"], kw["K"]
    inv_temp = it if it is not None else 1.0 / math.sqrt(q.shape[-1])
    gpu = run_gpu(q, k, v, do, planes, L=L, K=K, causal=causal, inv_temp=inv_temp, dev=dev, seg_tiles=seg, eps=eps)
    ref = run_oracle(q, k, v, do, planes, causal=causal, inv_temp=inv_temp, eps=eps)
    compare(name, gpu, ref, TOL[q.dtype])


# Seeded configurations a randomised sweep found above the bf16 bar before the
# small-table operand pairs and the fp64 walk of B (race_kernels.hip hl_ops,
# walk_f64); the error they had then is in the comment.  Nearly flat bucket
# probabilities (1-2 hash bits at the 1/sqrt(d) temperature) and, for the last
# one, a sharp softmax over a 6-tile reverse walk.
FLAT_CASES = [
    # name, make_case kwargs (with seed), causal, inv_temp, seg_tiles
    ("flat_K2L3_vmean", dict(T=64, H=1, L=3, K=2, v_shift=0.5, seed=9035), True, 0.125, 0),  # dk 5.8e-2
    ("flat_K1L7_M2_expand", dict(M=2, T=493, H=2, L=7, K=1, share_planes=False, expand_m=True, seed=8925),
     True, 0.125, 10),  # dk 4.1e-2
    ("flat_K1L2_M2_indep", dict(M=2, T=608, H=2, L=2, K=1, share_planes=False, seed=8976), True, 0.125, 2),  # dk 3.6e-2
    ("flat_K4L2_seg3", dict(B=2, T=224, H=3, L=2, K=4, seed=9186), True, 0.125, 3),  # dk 2.3e-2
    ("sharp_K6L3_walk6", dict(B=2, T=176, H=2, L=3, K=6, share_planes=False, v_shift=0.5, seed=9090),
     True, 1.9777229262274862, 6),  # dk 2.6e-2
    ("flat_noncausal_K2L5_vmean", dict(B=2, T=318, H=2, L=5, K=2, v_shift=0.5, seed=1014), False, 0.125, 7),
]


@pytest.mark.parametrize("name,kw,causal,it,seg", FLAT_CASES, ids=[c[0] for c in FLAT_CASES])
def test_parity_flat_tables(dev, name, kw, causal, it, seg):
    q, k, v, do, planes = make_case(**kw)
    gpu = run_gpu(q, k, v, do, planes, L=kw["L"], K=kw["K"], causal=causal, inv_temp=it, dev=dev, seg_tiles=seg)
    ref = run_oracle(q, k, v, do, planes, causal=causal, inv_temp=it)
    compare(name, gpu, ref, TOL[q.dtype])


# Whole tiles at sharp temperatures over long segments, from a randomised sweep of long walks (old dK in the
# comment): the whole-tile instantiations walk B in fp32 unless K |inv_temp| > 2 or the temperature is a
# device scalar (race_capi.hip exact_walk), and then in fp64.
SHARP_CASES = [
    # name, make_case kwargs (with seed), inv_temp, seg_tiles
    ("sharp_K8L1_whole_seg128", dict(T=9376, H=1, L=1, K=8, v_shift=0.5, seed=1036), 2.0, 128),  # dk 2.5e-1
    ("sharp_K4L8_whole_seg64", dict(T=3648, H=1, L=8, K=4, v_shift=1.0, seed=1025), 2.0, 64),  # dk 3.4e-1
    ("sharp_K4L8_whole_seg256", dict(T=14528, H=1, L=8, K=4, seed=1057), 2.0, 256),  # dk 4.1e-2
    ("sharp_K4L8_whole_tau1", dict(T=13280, H=1, L=8, K=4, v_shift=1.0, seed=1035), 1.0, 256),  # dk 2.3e-2
]


@pytest.mark.parametrize("name,kw,it,seg", SHARP_CASES, ids=[c[0] for c in SHARP_CASES])
def test_parity_sharp_whole_tiles(dev, name, kw, it, seg):
    q, k, v, do, planes = make_case(**kw)
    gpu = run_gpu(q, k, v, do, planes, L=kw["L"], K=kw["K"], causal=True, inv_temp=it, dev=dev, seg_tiles=seg)
    ref = run_oracle(q, k, v, do, planes, causal=True, inv_temp=it)
    compare(name, gpu, ref, TOL[q.dtype])


def test_device_temperature_takes_the_exact_walk(dev):
    """A device temperature (race_desc.inv_temp_ptr) runs the fp64 walk whatever its value: at the default
    temperature its result is within the bar of the oracle and close to the host temperature's fp32 walk."""
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    q, k, v, do, planes = make_case(T=2048, H=2, L=8, K=4, v_shift=0.5, seed=77)
    it = 0.125
    ref = run_oracle(q, k, v, do, planes, causal=True, inv_temp=it)
    host = run_gpu(q, k, v, do, planes, L=8, K=4, causal=True, inv_temp=it, dev=dev, seg_tiles=64)
    t = torch.tensor(it, device=dev)
    qd, kd, vd, dod, pd = [x.to(dev) for x in (q, k, v, do, planes)]
    out, st = race_fwd_raw(qd, kd, vd, pd, L=8, K=4, causal=True, inv_temp=t, seg_tiles=64)
    dq, dk, dv, git = race_bwd_raw(qd, kd, vd, pd, dod, st, L=8, K=4, causal=True, inv_temp=t, seg_tiles=64)
    torch.cuda.synchronize()
    devt = (out.cpu(), dq.cpu(), dk.cpu(), dv.cpu(), float(git.cpu()))
    compare("device temperature, fp64 walk", devt, ref, TOL[q.dtype])
    for nm, a, b in zip(("out", "dq", "dk", "dv"), devt[:4], host[:4]):
        e = relerr(to64(a), to64(b))
        print(f"[device vs host temperature] {nm} {e:.2e}", flush=True)
        assert e < 1e-2, (nm, e)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_t1_reference_eps_out_dv(dev, dtype):
    """T=1 at the reference eps (1e-6): out and dV are well conditioned there
    (out = sum_l v . P_Q P_K / (P_K + eps), dV its transpose), so they are
    checked to the usual bars; dQ and dK carry the factor eps/(P + eps) and are
    covered at eps=0.5 by the *_T1_eps cases."""
    fp32 = dtype == torch.float32
    L, K = (5, 2) if fp32 else (8, 4)
    q, k, v, do, planes = make_case(T=1, H=2, L=L, K=K, dtype=dtype, unit=not fp32, seed=21)
    it = 1.0 if fp32 else 1.0 / math.sqrt(q.shape[-1])
    gpu = run_gpu(q, k, v, do, planes, L=L, K=K, causal=True, inv_temp=it, dev=dev)
    ref = run_oracle(q, k, v, do, planes, causal=True, inv_temp=it)
    tol = TOL[dtype]
    for nm, a, b in (("out", gpu[0], ref[0]), ("dv", gpu[3], ref[3])):
        e = relerr(to64(a), b)
        print(f"[T1 {dtype}] {nm}={e:.2e}", flush=True)
        assert e <= tol, f"T=1 {nm} relerr {e:.3e} > {tol:.1e}"


def test_strided_fused_qkv_layout(dev):
    """Q, K, V as views into one [B, T, 3*H, D] projection (token stride 3*H*D)."""
    B, T, H, D, L, K = 2, 120, 2, 64, 8, 4
    g = torch.Generator().manual_seed(5)
    qkv = torch.nn.functional.normalize(torch.randn(B, T, 3 * H, D, generator=g), dim=-1).to(torch.bfloat16)
    do = torch.randn(1, B, T, H, D, generator=g).to(torch.bfloat16)
    planes = torch.randn(1, L, K, D, generator=g)
    qd = qkv.to(dev)
    views = [qd[:, :, j * H:(j + 1) * H].unsqueeze(0) for j in range(3)]
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    it = 1 / 8
    out, st = race_fwd_raw(*views, planes.to(dev), L=L, K=K, causal=True, inv_temp=it)
    dq, dk, dv, git = race_bwd_raw(*views, planes.to(dev), do.to(dev), st, L=L, K=K, causal=True, inv_temp=it)
    cpu = [qkv[:, :, j * H:(j + 1) * H].unsqueeze(0) for j in range(3)]
    ref = run_oracle(*cpu, do, planes, causal=True, inv_temp=it)
    compare("fused_qkv", (out.cpu(), dq.cpu(), dk.cpu(), dv.cpu(), float(git.cpu())), ref, 2e-2)


def test_golden_fixture(dev):
    """Committed oracle vectors (tests/golden/make_race_golden.py)."""
    z = np.load(os.path.join(HERE, "golden", "race_golden.npz"))
    names = sorted({k.split("__")[0] for k in z.files})
    for nm in names:
        f = lambda s: z[f"{nm}__{s}"]  # noqa: E731
        dtype = torch.bfloat16 if int(f("bf16")) else torch.float32
        q, k, v, do = [torch.from_numpy(f(s)).to(dtype) for s in ("q", "k", "v", "do")]
        planes = torch.from_numpy(f("planes")).float()
        L, K, causal, it = int(f("L")), int(f("K")), bool(f("causal")), float(f("inv_temp"))
        gpu = run_gpu(q, k, v, do, planes, L=L, K=K, causal=causal, inv_temp=it, dev=dev)
        ref = (f("out"), f("dq"), f("dk"), f("dv"), float(f("dinv_temp")), float(f("dinv_temp_l1")))
        compare("golden_" + nm, gpu, ref, TOL[dtype])


def test_deterministic(dev):
    q, k, v, do, planes = make_case(B=1, T=333, H=2, L=8, K=4, seed=3)
    a = run_gpu(q, k, v, do, planes, L=8, K=4, causal=True, inv_temp=0.125, dev=dev)
    b = run_gpu(q, k, v, do, planes, L=8, K=4, causal=True, inv_temp=0.125, dev=dev)
    for x, y in zip(a[:4], b[:4]):
        assert torch.equal(x, y)
    assert a[4] == b[4]


def test_config_c1(dev):
    """C1: non-causal fp32, B=1 H=4 N=4096 d=64 K=2 L=5 M=1, tau = exp(0) = 1, N(0,1) inputs."""
    q, k, v, do, planes = make_case(B=1, T=4096, H=4, L=5, K=2, dtype=torch.float32, unit=False, seed=11)
    gpu = run_gpu(q, k, v, do, planes, L=5, K=2, causal=False, inv_temp=1.0, dev=dev)
    ref = run_oracle(q, k, v, do, planes, causal=False, inv_temp=1.0)
    compare("C1", gpu, ref, 1e-4)


def test_config_c2(dev):
    """C2: causal bf16, B=2 H=8 N=16384 d=64 K=4 L=8 M=1, unit-L2 rows."""
    q, k, v, do, planes = make_case(B=2, T=16384, H=8, L=8, K=4, seed=12)
    it = 1.0 / 8.0
    gpu = run_gpu(q, k, v, do, planes, L=8, K=4, causal=True, inv_temp=it, dev=dev)
    ref = run_oracle(q, k, v, do, planes, causal=True, inv_temp=it)
    compare("C2", gpu, ref, 2e-2)


def test_config_c5_attention(dev):
    """C5's attention layer at full shape: causal bf16, K=8 (256 buckets),
    L=4, M=2 independent sketches, B=8, 12 heads, N=8192, d=64 -- 8 bucket
    slices per stream.  Streams are independent, so two heads of the first
    batch row of each estimator are checked against the oracle."""
    M, B, T, H, L, K = 2, 8, 8192, 12, 4, 8
    q, k, v, do, planes = make_case(M=M, B=B, T=T, H=H, L=L, K=K, seed=21, share_planes=False)
    it = 1.0 / 8.0
    out, dq, dk, dv, _ = run_gpu(q, k, v, do, planes, L=L, K=K, causal=True, inv_temp=it, dev=dev)
    sub = lambda x: x[:, :1, :, :2]  # noqa: E731
    ref = run_oracle(sub(q), sub(k), sub(v), sub(do), planes, causal=True, inv_temp=it)
    errs = {nm: relerr(to64(sub(a)), b) for nm, a, b in zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv), ref[:4])}
    print("[C5 attention] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for x in (out, dq, dk, dv):
        assert torch.isfinite(x).all()
    assert max(errs.values()) <= TOL[torch.bfloat16]
