"""race_fwd_noalloc, the forward whose scratch is the library's file-scope
device array (no caller workspace or state), against race_fwd through the C
ABI: two calls in a row on one GPU (the second with a smaller input, so it
runs on whatever the first left in the array), bit-identical to race_fwd with
the same segmentation and within the bf16 bar of the oracle; the automatic
segmentation coarsened to fit the array; fp32 and bf16 K=8 with per-slice
partial outputs in the array; replays of a captured HIP graph; and the size
rejection (CPU)."""
import ctypes
import math

import pytest
import torch

from helpers import TOL, make_case, relerr, run_oracle, to64

CAP = 64 << 20


def _desc(q, planes, L, K, causal, inv_temp, seg_tiles):
    from race_attention_amd.functional import _strides4, make_desc
    d = make_desc(q, q, q, planes, L=L, K=K, causal=causal, eps=1e-6, inv_temp=inv_temp, seg_tiles=seg_tiles)
    d.o_stride = _strides4(q)
    return d


def _both(q, k, v, planes, L, K, causal, inv_temp, seg_tiles, ref_seg_tiles=None):
    """(noalloc out, race_fwd out) for the same inputs; race_fwd runs with
    ref_seg_tiles (default: the same seg_tiles)."""
    from race_attention_amd import _lib
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out_na = torch.full(q.shape, float("nan"), dtype=q.dtype, device=q.device)
    d = _desc(q, planes, L, K, causal, inv_temp, seg_tiles)
    _lib.check(lib.race_fwd_noalloc(ctypes.byref(d), P(q), P(k), P(v), P(planes), P(out_na), st), "race_fwd_noalloc")
    d = _desc(q, planes, L, K, causal, inv_temp, seg_tiles if ref_seg_tiles is None else ref_seg_tiles)
    out = torch.empty_like(out_na)
    sb, wb = lib.race_state_bytes(ctypes.byref(d)), lib.race_fwd_workspace_bytes(ctypes.byref(d))
    state = torch.empty(sb, dtype=torch.uint8, device=q.device)
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=q.device)
    _lib.check(lib.race_fwd(ctypes.byref(d), P(q), P(k), P(v), P(planes), P(out), P(state), P(ws),
                            ctypes.c_size_t(ws.numel()), st), "race_fwd")
    torch.cuda.synchronize()
    return out_na, out


@pytest.mark.gpu
def test_noalloc_two_calls_match_race_fwd(dev):
    for T, H, seg, seed in ((3000, 4, 8, 1), (500, 2, 4, 2)):  # the second call is smaller
        L, K = 8, 4
        q, k, v, do, planes = make_case(B=1, T=T, H=H, L=L, K=K, seed=seed)
        it = 1.0 / math.sqrt(64)
        qd, kd, vd = [x.to(dev) for x in (q, k, v)]
        pd = planes.to(dev).float().contiguous()
        out_na, out = _both(qd, kd, vd, pd, L, K, True, it, seg)
        print(f"[noalloc T={T} H={H} seg_tiles={seg}] bit-identical={torch.equal(out_na, out)}", flush=True)
        assert torch.equal(out_na, out)
        ref = run_oracle(q, k, v, do, planes, causal=True, inv_temp=it)[0]
        e = relerr(to64(out_na.cpu()), ref)
        print(f"[noalloc T={T} H={H}] out vs oracle {e:.2e}", flush=True)
        assert e <= TOL[torch.bfloat16]


@pytest.mark.gpu
def test_noalloc_two_calls_bf16_slices(dev):
    """bf16 with 8-bit hashes (K=8, L=4: 1024 buckets in 8 slices) writes its
    bf16 partial outputs into the array too: two calls in a row, the second
    smaller, bit-identical to race_fwd with the same segmentation (explicit:
    the default one's state and sums for 1024 buckets would exceed the array,
    which the no-allocation forward answers with longer segments) and within
    the bf16 bar of the oracle."""
    for T, H, seg, seed in ((1500, 2, 8, 3), (600, 1, 4, 4)):
        L, K = 4, 8
        q, k, v, do, planes = make_case(B=1, T=T, H=H, L=L, K=K, seed=seed)
        it = 1.0 / math.sqrt(64)
        qd, kd, vd = [x.to(dev) for x in (q, k, v)]
        pd = planes.to(dev).float().contiguous()
        out_na, out = _both(qd, kd, vd, pd, L, K, True, it, seg)
        print(f"[noalloc K=8 T={T} H={H} seg_tiles={seg}] bit-identical={torch.equal(out_na, out)}", flush=True)
        assert torch.equal(out_na, out)
        ref = run_oracle(q, k, v, do, planes, causal=True, inv_temp=it)[0]
        e = relerr(to64(out_na.cpu()), ref)
        print(f"[noalloc K=8 T={T} H={H}] out vs oracle {e:.2e}", flush=True)
        assert e <= TOL[torch.bfloat16]


@pytest.mark.gpu
def test_noalloc_graph_capture_replays(dev):
    """race_fwd_noalloc captured into a HIP graph (torch.cuda.CUDAGraph) after
    one warm-up call, which looks the array's address up outside the capture:
    three replays, each on new input values copied into the captured tensors
    with eager work and a synchronisation before and after, are bit-identical
    to race_fwd on the same inputs."""
    from race_attention_amd import _lib
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    L, K, T, H, it = 8, 4, 2000, 2, 0.125
    q, k, v, _, planes = make_case(B=1, T=T, H=H, L=L, K=K, seed=41)
    qd, kd, vd = [x.to(dev).contiguous() for x in (q, k, v)]
    pd = planes.to(dev).float().contiguous()
    out = torch.empty_like(qd)
    d = _desc(qd, pd, L, K, True, it, 0)

    def call():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.race_fwd_noalloc(ctypes.byref(d), P(qd), P(kd), P(vd), P(pd), P(out), st),
                   "race_fwd_noalloc")

    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    torch.cuda.synchronize()
    for rep in range(3):
        gen = torch.Generator(device=dev).manual_seed(100 + rep)
        for x in (qd, kd, vd):
            x.copy_(torch.nn.functional.normalize(torch.randn(x.shape, device=dev, generator=gen), dim=-1))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        _, ref = _both(qd, kd, vd, pd, L, K, True, it, 0)
        print(f"[noalloc graph replay {rep}] bit-identical={torch.equal(got, ref)}", flush=True)
        assert torch.equal(got, ref)


@pytest.mark.gpu
def test_noalloc_automatic_segmentation_fits(dev):
    """T = 2^19, 8 heads: the default plan's state and sums (about 137 MB)
    exceed the array, so the forward runs longer segments: bit-identical to
    race_fwd with that segmentation, and within the bf16 bar of race_fwd's
    default one."""
    L, K, H, T = 8, 4, 8, 1 << 19
    g = torch.Generator(device=dev).manual_seed(9)
    q, k, v = [torch.nn.functional.normalize(torch.randn(1, 1, T, H, 64, device=dev, generator=g), dim=-1)
               .to(torch.bfloat16) for _ in range(3)]
    pd = torch.randn(1, L, K, 64, device=dev, generator=g)
    row = 8 * 128 * 65 * 8
    nseg = (CAP - (row + 512)) // (2 * row)
    tps = -(-(T // 32) // nseg)
    out_na, out = _both(q, k, v, pd, L, K, True, 0.125, 0, ref_seg_tiles=tps)
    print(f"[noalloc auto T={T}] coarsened to {tps} tiles per segment, bit-identical={torch.equal(out_na, out)}",
          flush=True)
    assert torch.equal(out_na, out)
    _, out_def = _both(q, k, v, pd, L, K, True, 0.125, 0, ref_seg_tiles=0)
    e = relerr(to64(out_na), to64(out_def))
    print(f"[noalloc auto] vs race_fwd default segmentation {e:.2e}", flush=True)
    assert e <= TOL[torch.bfloat16]


@pytest.mark.gpu
def test_noalloc_fp32_partials_in_scratch(dev):
    """fp32 runs bucket slices whose fp32 partial outputs also live in the array."""
    L, K, T, H = 5, 3, 1000, 2
    q, k, v, do, planes = make_case(B=2, T=T, H=H, L=L, K=K, dtype=torch.float32, unit=False, seed=5)
    qd, kd, vd = [x.to(dev) for x in (q, k, v)]
    pd = planes.to(dev).float().contiguous()
    out_na, out = _both(qd, kd, vd, pd, L, K, False, 0.7, 0)
    assert torch.equal(out_na, out)
    ref = run_oracle(q, k, v, do, planes, causal=False, inv_temp=0.7)[0]
    e = relerr(to64(out_na.cpu()), ref)
    print(f"[noalloc fp32 non-causal] out vs oracle {e:.2e}", flush=True)
    assert e <= TOL[torch.float32]


def test_noalloc_rejects_oversized_scratch():
    """fp32, 4 bucket slices, 8 heads x 2^20 tokens: 8.6 GB of partial
    outputs cannot live in the 64 MiB array -- a clear error before any GPU
    call (runs on the CPU)."""
    from race_attention_amd import _lib
    lib = _lib.load()
    d = _lib.RaceDesc()
    d.M, d.B, d.T, d.H, d.D = 1, 1, 1 << 20, 8, 64
    d.L, d.K, d.causal, d.dtype = 8, 4, 1, _lib.RACE_DTYPE_F32
    d.eps, d.inv_temp = 1e-6, 0.125
    for f in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(d, f)[2], getattr(d, f)[3] = 512, 64
    p = ctypes.c_void_p(256)
    rc = lib.race_fwd_noalloc(ctypes.byref(d), p, p, p, p, p, None)
    assert rc == -2
    msg = _lib.last_error()
    assert "race_fwd_noalloc" in msg and "use race_fwd" in msg and str(CAP) in msg
