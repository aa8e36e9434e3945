"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and rejects invalid requests before launching anything.
No compute call is made here (no GPU in this environment)."""
import ctypes
import os
import re

import pytest

from race_attention_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "race_attention.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(race_[a-z_]+)\s*\(", src))


def test_header_matches_binding_list():
    assert _declared() == set(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.race_abi_version() == 3


def test_desc_layout_matches_header():
    # int64 x5, int32 x4, float x2, int64, 6 x int64[4], int32 x2
    assert ctypes.sizeof(_lib.RaceDesc) == 5 * 8 + 4 * 4 + 2 * 4 + 8 + 6 * 32 + 2 * 4 + 8  # ..., inv_temp_ptr
    assert _lib.RaceDesc.planes_m_stride.offset == 64
    assert _lib.RaceDesc.inv_temp_ptr.offset == 272


def _desc(**kw):
    d = _lib.RaceDesc()
    d.M, d.B, d.T, d.H, d.D = 1, 1, 1 << 20, 8, 64
    d.L, d.K, d.causal, d.dtype = 8, 4, 1, _lib.RACE_DTYPE_BF16
    d.eps, d.inv_temp = 1e-6, 0.125
    for j in range(4):
        d.q_stride[j] = d.k_stride[j] = d.v_stride[j] = d.o_stride[j] = d.do_stride[j] = d.g_stride[j] = 0
    d.q_stride[2] = d.k_stride[2] = d.v_stride[2] = d.o_stride[2] = d.do_stride[2] = d.g_stride[2] = 512
    d.q_stride[3] = d.k_stride[3] = d.v_stride[3] = d.o_stride[3] = d.do_stride[3] = d.g_stride[3] = 64
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def _state(N, rows, spad=128):
    """State bytes: N x rows x spad buckets of 65 fp64 (B, A)."""
    return N * rows * spad * 65 * 8


def test_plan_sizes_c4():
    lib = _lib.load()
    d = _desc()
    sb = lib.race_state_bytes(ctypes.byref(d))
    # N=8 streams, 256 segments (+1 total), 128 buckets
    assert sb == _state(8, 257)
    assert lib.race_fwd_workspace_bytes(ctypes.byref(d)) == 8 * 256 * 128 * 65 * 8
    # the backward runs 128 segments of 2 forward ones (1024 workgroups; the
    # 256-tile segment bound stops the joining there): (U, alpha) sums and
    # suffixes fp32, and the [2][N][nseg][nslice] temperature partials fp64
    assert lib.race_bwd_workspace_bytes(ctypes.byref(d)) == 2 * 8 * 128 * 128 * 65 * 4 + 2 * 8 * 128 * 8
    # an explicit seg_tiles keeps the forward's segmentation in the backward
    d.seg_tiles = 128
    assert lib.race_bwd_workspace_bytes(ctypes.byref(d)) == 2 * 8 * 256 * 128 * 65 * 4 + 2 * 8 * 256 * 8


def test_segments_bounded_at_long_sequences():
    """Segments, forward and backward, are at most 256 tiles at any T (this
    bounds the backward's fp32 walks of the forward state): at T = 2^22 the
    default plan runs 512 segments per stream instead of 256 of 512 tiles, and
    the backward keeps them; at 37.5 M tokens (one layer's max-N in 288 GB)
    4584 segments per stream."""
    lib = _lib.load()
    d = _desc(T=1 << 22)
    assert lib.race_state_bytes(ctypes.byref(d)) == _state(8, 513)
    assert lib.race_bwd_workspace_bytes(ctypes.byref(d)) == 2 * 8 * 512 * 128 * 65 * 4 + 2 * 8 * 512 * 8
    d = _desc(T=37552128)
    assert lib.race_state_bytes(ctypes.byref(d)) == _state(8, 37552128 // 8192 + 1)
    assert lib.race_bwd_workspace_bytes(ctypes.byref(d)) == (2 * 8 * 4584 * 128 * 65 * 4 +
                                                              -(-2 * 8 * 4584 * 8 // 16) * 16)


def test_explicit_segments_above_the_walk_bound_rejected():
    """An explicit seg_tiles above 256 would lengthen the backward's walks:
    the backward calls reject it.  A forward alone walks its segments only
    upwards from an fp64 state row and accepts it, and so do the probability
    outputs, which walk no state."""
    lib = _lib.load()
    d = _desc(seg_tiles=256)
    assert lib.race_bwd_workspace_bytes(ctypes.byref(d)) > 0
    d = _desc(seg_tiles=257)
    assert lib.race_state_bytes(ctypes.byref(d)) > 0
    assert lib.race_fwd_workspace_bytes(ctypes.byref(d)) > 0
    assert lib.race_probs_bwd_workspace_bytes(ctypes.byref(d)) > 0
    assert lib.race_bwd_workspace_bytes(ctypes.byref(d)) == 0 and "seg_tiles=257" in _lib.last_error()
    assert lib.race_bwd_global_workspace_bytes(ctypes.byref(d)) == 0
    p = ctypes.c_void_p(256)
    rc = lib.race_bwd(ctypes.byref(d), p, p, p, p, p, p, p, p, p, None, p, 1 << 30, None)
    assert rc == -2 and "seg_tiles" in _lib.last_error()
    rc = lib.race_bwd_ex(ctypes.byref(d), p, p, p, p, None, p, None, p, p, p, p, None, p, 1 << 30, None)
    assert rc == -2 and "seg_tiles" in _lib.last_error()


def test_launch_grid_bound_in_work_items():
    """A launch counts its work-items in 32 bits (the dispatch packet's grid
    size): a plan whose tile grid would exceed 2^32 - 1 work-items is rejected
    before any launch -- here 16.8 M sliced workgroups of 512 threads from an
    explicit one-tile segmentation."""
    lib = _lib.load()
    d = _desc(K=8, L=4, M=1, B=1, H=64, T=1 << 20, seg_tiles=1)
    assert lib.race_state_bytes(ctypes.byref(d)) == 0 and "2^32 work-items" in _lib.last_error()
    rc = lib.race_fwd(ctypes.byref(d), None, None, None, None, None, None, None, 0, None)
    assert rc == -2 and "2^32 work-items" in _lib.last_error()
    d = _desc(K=8, L=4, M=1, B=1, H=64, T=1 << 20, seg_tiles=16)   # 1/16 of the workgroups
    assert lib.race_state_bytes(ctypes.byref(d)) > 0


def test_noalloc_null_descriptor_rejected():
    lib = _lib.load()
    rc = lib.race_fwd_noalloc(None, None, None, None, None, None, None)
    assert rc == -1 and "descriptor is NULL" in _lib.last_error()


def test_device_temperature_skips_host_value_check():
    """With inv_temp_ptr set the float field is not read (a device scalar is
    validated by its producer); a misaligned pointer is rejected."""
    lib = _lib.load()
    d = _desc(T=64, inv_temp=float("nan"))
    assert lib.race_state_bytes(ctypes.byref(d)) == 0 and "inv_temp" in _lib.last_error()
    d.inv_temp_ptr = 256
    assert lib.race_state_bytes(ctypes.byref(d)) > 0
    d.inv_temp_ptr = 258
    assert lib.race_state_bytes(ctypes.byref(d)) == 0 and "inv_temp_ptr" in _lib.last_error()


@pytest.mark.parametrize("field,value,code,msg", [
    ("D", 32, -2, "head dim"),
    ("K", 9, -2, "hash bits"),
    ("L", 9, -2, "projection columns"),
    ("L", 0, -1, "L and K"),
    ("T", 0, -1, "must be >= 1"),
    ("T", (1 << 35) + 1, -2, "T <= 2^35"),
    ("dtype", 7, -1, "dtype"),
])
def test_invalid_descriptors_rejected(field, value, code, msg):
    lib = _lib.load()
    d = _desc(**{field: value})
    assert lib.race_state_bytes(ctypes.byref(d)) == 0
    assert msg in _lib.last_error()
    rc = lib.race_fwd(ctypes.byref(d), None, None, None, None, None, None, None, 0, None)
    assert rc == code
    assert msg in _lib.last_error()


def _plan(**kw):
    lib = _lib.load()
    d = _desc(**kw)
    return (lib.race_state_bytes(ctypes.byref(d)), lib.race_fwd_workspace_bytes(ctypes.byref(d)),
            lib.race_bwd_workspace_bytes(ctypes.byref(d)))


@pytest.mark.parametrize("dtype,K,L,M,B,H,T,spad", [
    # fp32: slices of 32 buckets, L*2^K = 128 -> 4 slices
    (_lib.RACE_DTYPE_F32, 4, 8, 1, 1, 8, 4096, 128),
    # bf16, 2^K > 16: slices of 128 buckets; the decoder config's K=8, L=4
    # (1024 buckets, 8 slices), M=2 estimators, 8 x 12 heads
    (_lib.RACE_DTYPE_BF16, 8, 4, 2, 8, 12, 8192, 1024),
    (_lib.RACE_DTYPE_BF16, 5, 6, 1, 1, 2, 1000, 256),
])
def test_sliced_plans(dtype, K, L, M, B, H, T, spad):
    """Bucket counts beyond one workgroup run as slices: the state holds every
    (padded) bucket, and the workspaces add per-slice partial outputs in the
    element type (O forward; dQ, dK, dV backward)."""
    sb, fw, bw = _plan(dtype=dtype, K=K, L=L, M=M, B=B, H=H, T=T)
    N = M * B * H
    row = spad * 65
    assert sb > 0 and sb % _state(N, 1, spad) == 0
    nseg = sb // _state(N, 1, spad) - 1
    SP = 32 if dtype == _lib.RACE_DTYPE_F32 else 128
    es = 4 if dtype == _lib.RACE_DTYPE_F32 else 2
    part = -(-((spad // SP) * N * T * 64 * es) // 16) * 16
    assert fw >= N * nseg * row * 8 + part
    # the backward runs between 1 and nseg segments (whole forward segments);
    # dQ and dK go through each slice's dproj columns: SP / 2^K tables of K
    # columns (K columns of a wider table), rounded up to 8, 16 or 32; bf16
    # tables wider than a slice (K=8: two slices per table) keep them in fp32
    nslice = spad // SP
    cols = (SP >> K) * K if (1 << K) <= SP else K
    xc = next(c for c in (8, 16, 32) if c >= min(cols, 32))
    xes = 4 if (1 << K) > SP else es
    xpart = -(-(nslice * N * T * xc * xes) // 16) * 16
    lo, hi = 2 * N * row * 4, 2 * N * nseg * row * 4 + 2 * N * nseg * nslice * 8 + 16
    assert lo + part + 2 * xpart <= bw <= hi + part + 2 * xpart


def test_null_and_misaligned_pointers_rejected():
    lib = _lib.load()
    d = _desc(T=64)
    rc = lib.race_fwd(ctypes.byref(d), None, None, None, None, None, None, None, 0, None)
    assert rc == -1 and "q is NULL" in _lib.last_error()
    rc = lib.race_fwd(ctypes.byref(d), ctypes.c_void_p(8), None, None, None, None, None, None, 0, None)
    assert rc == -1 and "aligned" in _lib.last_error()
    d.q_stride[2] = 100   # 200 bytes: not a multiple of 16
    rc = lib.race_fwd(ctypes.byref(d), ctypes.c_void_p(16), None, None, None, None, None, None, 0, None)
    assert rc == -1 and "stride" in _lib.last_error()


def test_workspace_too_small_rejected():
    lib = _lib.load()
    d = _desc(T=64)
    p = ctypes.c_void_p(256)
    rc = lib.race_fwd(ctypes.byref(d), p, p, p, p, p, p, p, 16, None)
    assert rc == -3 and "workspace" in _lib.last_error()


def _max_stride(esize):
    # ((32 - 1) * stride + 64) * esize <= 2^31 - 1, rounded down to a 16-byte multiple
    m = ((2 ** 31 - 1) // esize - 64) // 31
    return m - m % (16 // esize)


@pytest.mark.parametrize("dtype,esize", [(_lib.RACE_DTYPE_BF16, 2), (_lib.RACE_DTYPE_F32, 4)])
def test_token_stride_byte_bound(dtype, esize):
    """Lane byte offsets inside a 32-token tile are 32-bit: the largest token
    stride whose tile spans at most 2^31 - 1 bytes is accepted (the call then
    stops at the too-small workspace), the next 16-byte multiple is rejected."""
    lib = _lib.load()
    # the accepted stride also keeps a tile's byte stride (32 rows) below
    # 2^32, the bound of the kernels' 32 x 32-bit tile base offsets
    assert 32 * _max_stride(esize) * esize < 2 ** 32
    p = ctypes.c_void_p(256)
    for which in ("q_stride", "o_stride"):
        d = _desc(T=64, H=1, dtype=dtype)
        getattr(d, which)[2] = _max_stride(esize)
        rc = lib.race_fwd(ctypes.byref(d), p, p, p, p, p, p, p, 16, None)
        assert rc == -3 and "workspace" in _lib.last_error()
        getattr(d, which)[2] = _max_stride(esize) + 16 // esize
        rc = lib.race_fwd(ctypes.byref(d), p, p, p, p, p, p, p, 16, None)
        assert rc == -2 and "32-bit tile offsets" in _lib.last_error()


@pytest.mark.parametrize("field,j,value,msg", [
    ("o_stride", 3, 0, "stride 0 over H"),
    ("o_stride", 3, 32, "head stride"),
    ("g_stride", 0, 0, "stride 0 over M"),
    ("g_stride", 1, 0, "stride 0 over B"),
])
def test_written_tensors_must_not_alias(field, j, value, msg):
    """Outputs with a zero stride over a dimension of size > 1, or heads
    closer than D elements, would have workgroups of different streams write
    the same rows: rejected (inputs may alias, e.g. the stride-0 M expand)."""
    lib = _lib.load()
    d = _desc(T=64, M=2, B=2)
    for f in ("q_stride", "k_stride", "v_stride", "o_stride", "do_stride", "g_stride"):
        getattr(d, f)[0], getattr(d, f)[1] = 2 * 64 * 512, 64 * 512
    getattr(d, field)[j] = value
    p = ctypes.c_void_p(256)
    if field == "o_stride":
        rc = lib.race_fwd(ctypes.byref(d), p, p, p, p, p, p, p, 16, None)
    else:
        rc = lib.race_bwd(ctypes.byref(d), p, p, p, p, p, p, p, p, p, None, p, 16, None)
    assert rc == -1 and msg in _lib.last_error()
    # inputs may share rows: a stride-0 M expand of q is accepted
    d = _desc(T=64, M=2, B=2)
    for f in ("k_stride", "v_stride", "o_stride", "do_stride", "g_stride"):
        getattr(d, f)[0], getattr(d, f)[1] = 2 * 64 * 512, 64 * 512
    d.q_stride[0], d.q_stride[1] = 0, 64 * 512
    rc = lib.race_fwd(ctypes.byref(d), p, p, p, p, p, p, p, 16, None)
    assert rc == -3


def test_prefix_mean_argument_checks():
    lib = _lib.load()
    assert lib.race_prefix_mean_workspace_bytes(4, 100, 64) > 0
    assert lib.race_prefix_mean_workspace_bytes(0, 100, 64) == 0
    rc = lib.race_prefix_mean_fwd(None, None, None, 4, 100, 64, 1e-6, None, 0, None)
    assert rc == -1
    p = ctypes.c_void_p(256)
    rc = lib.race_prefix_mean_fwd(p, p, p, 4, 100, 1024, 1e-6, p, 1 << 30, None)
    assert rc == -2 and "D=1024" in _lib.last_error()


# ------------------------------------------------- global normalisation (F2)
def test_global_workspace_sizes():
    """F2 adds per-token fp32 buffers: den partials per slice (sliced
    instantiations, forward), rden/gden (backward) and, sliced, each slice's
    share of sum_s P_Q dO.B_s (backward)."""
    lib = _lib.load()
    d = _desc()
    N, T = 8, 1 << 20
    tok = N * T * 4
    assert lib.race_fwd_global_workspace_bytes(ctypes.byref(d)) == lib.race_fwd_workspace_bytes(ctypes.byref(d))
    assert lib.race_bwd_global_workspace_bytes(ctypes.byref(d)) == lib.race_bwd_workspace_bytes(ctypes.byref(d)) + 2 * tok
    d = _desc(dtype=_lib.RACE_DTYPE_F32, T=4096)      # 4 slices of 32 buckets
    f1 = lib.race_fwd_workspace_bytes(ctypes.byref(d))
    assert lib.race_fwd_global_workspace_bytes(ctypes.byref(d)) == f1 + 4 * N * 4096 * 4
    b1 = lib.race_bwd_workspace_bytes(ctypes.byref(d))
    assert lib.race_bwd_global_workspace_bytes(ctypes.byref(d)) == b1 + (2 + 4) * N * 4096 * 4


@pytest.mark.parametrize("field,value,code,msg", [
    ("causal", 0, -2, "causal operator only"),
    ("eps", 0.0, -1, "must be > 0"),
    ("K", 9, -2, "hash bits"),
])
def test_global_invalid_descriptors_rejected(field, value, code, msg):
    lib = _lib.load()
    d = _desc(**{field: value})
    rc = lib.race_fwd_global(ctypes.byref(d), None, None, None, None, None, None, None, None, 0, None)
    assert rc == code and msg in _lib.last_error()
    rc = lib.race_bwd_global(ctypes.byref(d), *([None] * 14), 0, None)
    assert rc == code and msg in _lib.last_error()


def test_global_null_den_and_workspace_rejected():
    lib = _lib.load()
    d = _desc(T=64)
    p = ctypes.c_void_p(256)
    rc = lib.race_fwd_global(ctypes.byref(d), p, p, p, p, p, None, p, p, 1 << 30, None)
    assert rc == -1 and "den is NULL" in _lib.last_error()
    rc = lib.race_fwd_global(ctypes.byref(d), p, p, p, p, p, ctypes.c_void_p(258), p, p, 1 << 30, None)
    assert rc == -1 and "den is not 4-byte aligned" in _lib.last_error()
    rc = lib.race_fwd_global(ctypes.byref(d), p, p, p, p, p, p, p, p, 16, None)
    assert rc == -3 and "workspace" in _lib.last_error()
    # dden is optional, but when given it is checked like den
    rc = lib.race_bwd_global(ctypes.byref(d), p, p, p, p, p, p, p, ctypes.c_void_p(6), p, p, p, p, None, p,
                             1 << 30, None)
    assert rc == -1 and "dden is not 4-byte aligned" in _lib.last_error()
    need = lib.race_bwd_global_workspace_bytes(ctypes.byref(d))
    rc = lib.race_bwd_global(ctypes.byref(d), p, p, p, p, p, p, p, None, p, p, p, p, None, p, need - 1, None)
    assert rc == -3 and "workspace" in _lib.last_error()


# ------------------------------------------------- key weights and den (F1 extras)
def test_ex_rejects_causal_extras_and_checks_pointers():
    lib = _lib.load()
    d = _desc(T=64)        # causal
    p = ctypes.c_void_p(256)
    rc = lib.race_fwd_ex(ctypes.byref(d), p, p, p, p, p, p, None, p, p, 1 << 30, None)
    assert rc == -2 and "non-causal" in _lib.last_error()
    rc = lib.race_bwd_ex(ctypes.byref(d), p, p, p, p, None, p, p, p, p, p, p, None, p, 1 << 30, None)
    assert rc == -2 and "non-causal" in _lib.last_error()
    d = _desc(T=64, causal=0)
    rc = lib.race_fwd_ex(ctypes.byref(d), p, p, p, p, ctypes.c_void_p(258), p, None, p, p, 1 << 30, None)
    assert rc == -1 and "kmask is not 4-byte aligned" in _lib.last_error()
    assert lib.race_fwd_ex_workspace_bytes(ctypes.byref(d)) == lib.race_fwd_workspace_bytes(ctypes.byref(d))
    rc = lib.race_fwd_ex(ctypes.byref(d), p, p, p, p, None, p, p, p, p, 16, None)
    assert rc == -3 and "workspace" in _lib.last_error()


def test_probs_argument_checks():
    lib = _lib.load()
    d = _desc(T=64)
    p = ctypes.c_void_p(256)
    assert lib.race_probs(ctypes.byref(d), None, p, p, None) == -1 and "x is NULL" in _lib.last_error()
    assert lib.race_probs(ctypes.byref(d), p, p, None, None) == -1 and "P is NULL" in _lib.last_error()
    need = lib.race_probs_bwd_workspace_bytes(ctypes.byref(d))
    assert need == 8 * 2 * 8      # fp64 temperature partials: 8 streams x 2 segments (2 tiles), no slices
    rc = lib.race_probs_bwd(ctypes.byref(d), p, p, p, p, None, p, need - 1, None)
    assert rc == -3 and "workspace" in _lib.last_error()


@pytest.mark.parametrize("K,L,M,B,H,T,fnseg,nseg", [
    (4, 8, 1, 1, 8, 1 << 20, 256, 128),   # C4: 256 forward segments of 128 tiles, 128 backward ones of 256
    (4, 8, 1, 1, 8, 1 << 22, 512, 512),   # every segment at the 256-tile bound
    (8, 4, 2, 8, 12, 8192, 2, 1),          # C5: 8 slices; 2 forward segments, 1 backward
    (2, 5, 1, 4, 3, 1000, None, None),     # 20 buckets, one 32-bucket slice
])
def test_bench_scan_bytes(K, L, M, B, H, T, fnseg, nseg):
    """bench.py's scan byte model recovers the plan's segment counts from the
    library's buffer sizes (the sizes must match its formulas exactly) and
    counts each scan's reads and writes of segment rows."""
    import bench
    sb, _, bw = _plan(dtype=_lib.RACE_DTYPE_BF16, K=K, L=L, M=M, B=B, H=H, T=T)
    N = M * B * H
    got = bench.scan_bytes(sb, bw, N, T, L, K)
    assert got is not None
    fb, bb, fn, bn = got
    if fnseg is not None:
        assert (fn, bn) == (fnseg, nseg)
    spad = -(-(L << K) // 128) * 128 if K > 4 else (L << K) + (-(L << K)) % 32
    assert fb == (2 * fn + 1) * N * spad * 65 * 8
    assert bb == 2 * N * bn * spad * 65 * 4


def test_backward_segments_cover_short_sequences_whole():
    """The decoder core's shape (shared sketch: 96 streams of 8192 tokens, K=8,
    L=4, 8 slices): the forward runs 3 segments of 86 tiles; the backward
    covers each stream's 256 tiles in one segment -- within the 256-tile
    bound -- rather than in 172 + 84 tiles."""
    import bench
    sb, _, bw = _plan(dtype=_lib.RACE_DTYPE_BF16, K=8, L=4, M=1, B=8, H=12, T=8192)
    _, _, fnseg, nseg = bench.scan_bytes(sb, bw, 96, 8192, 4, 8)
    assert (fnseg, nseg) == (3, 1)
    # beyond the bound the backward segments stay within it: 2^16 tokens = 2048 tiles
    sb, _, bw = _plan(dtype=_lib.RACE_DTYPE_BF16, K=8, L=4, M=1, B=8, H=12, T=1 << 16)
    _, _, fnseg, nseg = bench.scan_bytes(sb, bw, 96, 1 << 16, 4, 8)
    assert -(-2048 // nseg) <= 256, (fnseg, nseg)
