"""CPU checker for the RACE attention operator (F1 and F2 semantics).

TEST INFRASTRUCTURE ONLY.  tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may use this module, and only as the checker; the product
(race_attention_amd) never imports it and has no CPU fallback.

Two layers:
  * ``race_forward`` / ``race_backward``: ctypes front-end of the fp64 C
    restatement in race_oracle.c (misc/race.py:63-142, misc/vit.py:918-978,
    kernels/cpu/race_pref.cpp:36-220).  Inputs are [M,B,T,H,D] arrays like the
    reference's BatchedACE; planes are [NP,L,K,D] (NP = 1 when shared,
    misc/race.py:39-51).
  * ``race_forward_ex`` / ``race_backward_ex``: F1 with per-token key
    weights (the padding mask, misc/classification.py:576-592) and the den
    output of misc/classification.py:641-659 and misc/vit.py:1452-1510.
  * ``race_probs`` / ``race_probs_bwd``: the bucket probabilities of one
    input and their backward (misc/arxiv_64K.py:1580-1644, misc/vit.py:3193-3262).
  * ``race_global_forward`` / ``race_global_backward``: the same C file's
    restatement of the globally normalised causal mode ("F2",
    misc/elsaa_causal_complete.py:438-586, misc/race_kernel.py:8-124).
  * ``prefix_mean_flat`` / ``prefix_mean_flat_bw``: restatement of the
    reference CPU kernel's flat prefix mean (race_pref.cpp:36-101, :104-220).
  * ``ref_race_pref()``: the reference's own race_pref.cpp compiled from its
    source into oracle/_ref/ (None when not built), used to pin the
    restatement.

Parity status of each function (what pins it) is listed in
tests/test_oracle.py; every exported function has at least one pin.
"""
from __future__ import annotations

import ctypes
import glob
import importlib.util
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build() -> None:
    """Compile liborace.so (and oracle/_ref when the reference tree exists)."""
    subprocess.check_call(["make", "-s", "-C", HERE, "all"])


def _lib():
    global _LIB
    if _LIB is None:
        # RACE_ORACLE_LIB selects another build of the same source (the
        # sanitizer builds of `make -C oracle sanitize`)
        path = os.environ.get("RACE_ORACLE_LIB") or os.path.join(HERE, "liborace.so")
        if not os.path.exists(path):
            subprocess.check_call(["make", "-s", "-C", HERE, "liborace.so"])
        lib = ctypes.CDLL(path)
        dp = ctypes.POINTER(ctypes.c_double)
        fp = ctypes.POINTER(ctypes.c_float)
        ip = ctypes.POINTER(ctypes.c_int64)
        i64, ci, cd = ctypes.c_int64, ctypes.c_int, ctypes.c_double
        lib.oracle_race_forward.argtypes = [dp, dp, dp, dp, ip, i64, i64, i64, ci, ci, ci, cd, cd, dp]
        lib.oracle_race_forward.restype = ci
        lib.oracle_race_backward.argtypes = [dp, dp, dp, dp, dp, ip, i64, i64, i64, ci, ci, ci, cd, cd,
                                             dp, dp, dp, dp, dp]
        lib.oracle_race_backward.restype = ci
        lib.oracle_race_global_forward.argtypes = [dp, dp, dp, dp, ip, i64, i64, i64, ci, ci, cd, cd, dp, dp]
        lib.oracle_race_global_forward.restype = ci
        lib.oracle_race_global_backward.argtypes = [dp, dp, dp, dp, dp, dp, ip, i64, i64, i64, ci, ci, cd, cd,
                                                    dp, dp, dp, dp, dp]
        lib.oracle_race_global_backward.restype = ci
        lib.oracle_race_forward_ex.argtypes = [dp, dp, dp, dp, dp, ip, i64, i64, i64, ci, ci, ci, cd, cd, dp, dp]
        lib.oracle_race_forward_ex.restype = ci
        lib.oracle_race_backward_ex.argtypes = [dp, dp, dp, dp, dp, dp, dp, ip, i64, i64, i64, ci, ci, ci, cd, cd,
                                                dp, dp, dp, dp, dp]
        lib.oracle_race_backward_ex.restype = ci
        lib.oracle_race_probs.argtypes = [dp, dp, ip, i64, i64, i64, ci, ci, cd, dp]
        lib.oracle_race_probs.restype = ci
        lib.oracle_race_probs_bwd.argtypes = [dp, dp, dp, ip, i64, i64, i64, ci, ci, cd, dp, dp, dp]
        lib.oracle_race_probs_bwd.restype = ci
        lib.oracle_prefix_mean_flat.argtypes = [fp, fp, i64, i64, i64, cd, fp]
        lib.oracle_prefix_mean_flat.restype = None
        lib.oracle_prefix_mean_flat_bw.argtypes = [fp, fp, fp, i64, i64, i64, cd, fp, fp]
        lib.oracle_prefix_mean_flat_bw.restype = None
        _LIB = lib
    return _LIB


def _dptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _fptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def to_streams(x):
    """[M,B,T,H,D] -> [N=M*B*H, T, D] with stream n = (m*B + b)*H + h
    (misc/race.py:73-76)."""
    M, B, T, H, D = x.shape
    return np.ascontiguousarray(np.transpose(np.asarray(x, dtype=np.float64), (0, 1, 3, 2, 4))
                                .reshape(M * B * H, T, D))


def from_streams(y, M, B, H):
    """[N,T,D] -> [M,B,T,H,D] (misc/race.py:141)."""
    N, T, D = y.shape
    return np.ascontiguousarray(y.reshape(M, B, H, T, D).transpose(0, 1, 3, 2, 4))


def _plane_map(M, B, H, n_planes):
    m_of_n = np.repeat(np.arange(M, dtype=np.int64), B * H)
    if n_planes == 1:
        return np.zeros(M * B * H, dtype=np.int64)
    assert n_planes == M, "planes must be [1,L,K,D] (shared) or [M,L,K,D]"
    return np.ascontiguousarray(m_of_n)


def race_forward(q, k, v, planes, *, causal: bool, eps: float = 1e-6, inv_temp: float):
    """fp64 forward. q,k,v: [M,B,T,H,D]; planes [NP,L,K,D]. Returns [M,B,T,H,D]."""
    M, B, T, H, D = q.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, Dp = planes.shape
    assert Dp == D
    qs, ks, vs = to_streams(q), to_streams(k), to_streams(v)
    pm = _plane_map(M, B, H, NP)
    out = np.zeros_like(qs)
    rc = _lib().oracle_race_forward(_dptr(qs), _dptr(ks), _dptr(vs), _dptr(planes),
                                    pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                    qs.shape[0], T, D, L, K, int(causal), float(eps),
                                    float(inv_temp), _dptr(out))
    if rc != 0:
        raise ValueError("oracle_race_forward rejected its arguments")
    return from_streams(out, M, B, H)


def race_backward(q, k, v, dout, planes, *, causal: bool, eps: float = 1e-6, inv_temp: float,
                  with_l1: bool = False):
    """fp64 backward. Returns (dq, dk, dv, grad_inv_temp); grads are [M,B,T,H,D]
    and grad_inv_temp = dL/d(1/tau) summed over all streams.  with_l1 appends
    sum |du * th|, the l1 mass of the terms of that sum."""
    M, B, T, H, D = q.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, _ = planes.shape
    qs, ks, vs, gs = to_streams(q), to_streams(k), to_streams(v), to_streams(dout)
    pm = _plane_map(M, B, H, NP)
    dq, dk, dv = np.zeros_like(qs), np.zeros_like(qs), np.zeros_like(qs)
    git = np.zeros(2, dtype=np.float64)
    rc = _lib().oracle_race_backward(_dptr(qs), _dptr(ks), _dptr(vs), _dptr(gs), _dptr(planes),
                                     pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                     qs.shape[0], T, D, L, K, int(causal), float(eps),
                                     float(inv_temp), _dptr(dq), _dptr(dk), _dptr(dv), _dptr(git),
                                     _dptr(git[1:]))
    if rc != 0:
        raise ValueError("oracle_race_backward rejected its arguments")
    res = (from_streams(dq, M, B, H), from_streams(dk, M, B, H), from_streams(dv, M, B, H), float(git[0]))
    return res + (float(git[1]),) if with_l1 else res


def mask_to_streams(mask, M, H):
    """[B,T] per-token key weights -> [N,T] (stream n = (m*B + b)*H + h)."""
    m = np.asarray(mask, dtype=np.float64)
    B, T = m.shape
    return np.ascontiguousarray(np.broadcast_to(m[None, :, None, :], (M, B, H, T)).reshape(M * B * H, T))


def race_forward_ex(q, k, v, planes, *, kmask=None, causal: bool, eps: float = 1e-6, inv_temp: float):
    """fp64 F1 forward with key weights kmask [B,T] (None = 1) on P_K.
    Returns (out [M,B,T,H,D], den [M,B,H,T]), den = sum_s P_Q A_s(t) unclamped."""
    M, B, T, H, D = q.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, _ = planes.shape
    qs, ks, vs = to_streams(q), to_streams(k), to_streams(v)
    kw = mask_to_streams(kmask, M, H) if kmask is not None else None
    pm = _plane_map(M, B, H, NP)
    out = np.zeros_like(qs)
    den = np.zeros((qs.shape[0], T), dtype=np.float64)
    rc = _lib().oracle_race_forward_ex(_dptr(qs), _dptr(ks), _dptr(vs), _dptr(kw) if kw is not None else None,
                                       _dptr(planes), pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                       qs.shape[0], T, D, L, K, int(causal), float(eps), float(inv_temp),
                                       _dptr(out), _dptr(den))
    if rc != 0:
        raise ValueError("oracle_race_forward_ex rejected its arguments")
    return from_streams(out, M, B, H), den.reshape(M, B, H, T)


def race_backward_ex(q, k, v, dout, planes, *, kmask=None, dden=None, causal: bool, eps: float = 1e-6,
                     inv_temp: float, with_l1: bool = False):
    """fp64 backward of race_forward_ex for dout [M,B,T,H,D] and dden
    [M,B,H,T] (None = 0).  Returns (dq, dk, dv, grad_inv_temp[, l1])."""
    M, B, T, H, D = q.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, _ = planes.shape
    qs, ks, vs, gs = to_streams(q), to_streams(k), to_streams(v), to_streams(dout)
    kw = mask_to_streams(kmask, M, H) if kmask is not None else None
    hs = den_to_streams(dden, M, B, H) if dden is not None else None
    pm = _plane_map(M, B, H, NP)
    dq, dk, dv = np.zeros_like(qs), np.zeros_like(qs), np.zeros_like(qs)
    git = np.zeros(2, dtype=np.float64)
    rc = _lib().oracle_race_backward_ex(_dptr(qs), _dptr(ks), _dptr(vs), _dptr(kw) if kw is not None else None,
                                        _dptr(gs), _dptr(hs) if hs is not None else None, _dptr(planes),
                                        pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), qs.shape[0], T, D, L, K,
                                        int(causal), float(eps), float(inv_temp), _dptr(dq), _dptr(dk), _dptr(dv),
                                        _dptr(git), _dptr(git[1:]))
    if rc != 0:
        raise ValueError("oracle_race_backward_ex rejected its arguments")
    res = (from_streams(dq, M, B, H), from_streams(dk, M, B, H), from_streams(dv, M, B, H), float(git[0]))
    return res + (float(git[1]),) if with_l1 else res


def race_probs(x, planes, *, inv_temp: float):
    """fp64 bucket probabilities of x [M,B,T,H,D] -> [M,B,H,T,L*2^K]."""
    M, B, T, H, D = x.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, _ = planes.shape
    xs = to_streams(x)
    pm = _plane_map(M, B, H, NP)
    P = np.zeros((xs.shape[0], T, L << K), dtype=np.float64)
    rc = _lib().oracle_race_probs(_dptr(xs), _dptr(planes), pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                  xs.shape[0], T, D, L, K, float(inv_temp), _dptr(P))
    if rc != 0:
        raise ValueError("oracle_race_probs rejected its arguments")
    return P.reshape(M, B, H, T, L << K)


def race_probs_bwd(x, dP, planes, *, inv_temp: float, with_l1: bool = False):
    """fp64 backward of race_probs: dP [M,B,H,T,S] -> (dx [M,B,T,H,D],
    grad_inv_temp[, l1])."""
    M, B, T, H, D = x.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, _ = planes.shape
    xs = to_streams(x)
    dPs = np.ascontiguousarray(np.asarray(dP, dtype=np.float64).reshape(M * B * H, T, L << K))
    pm = _plane_map(M, B, H, NP)
    dx = np.zeros_like(xs)
    git = np.zeros(2, dtype=np.float64)
    rc = _lib().oracle_race_probs_bwd(_dptr(xs), _dptr(dPs), _dptr(planes),
                                      pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), xs.shape[0], T, D, L, K,
                                      float(inv_temp), _dptr(dx), _dptr(git), _dptr(git[1:]))
    if rc != 0:
        raise ValueError("oracle_race_probs_bwd rejected its arguments")
    res = (from_streams(dx, M, B, H), float(git[0]))
    return res + (float(git[1]),) if with_l1 else res


def den_to_streams(h, M, B, H):
    """[M,B,H,T] (or [N,T]) per-token array -> [N,T] float64, stream-major."""
    return np.ascontiguousarray(np.asarray(h, dtype=np.float64).reshape(M * B * H, -1))


def race_global_forward(q, k, v, planes, *, floor: float = 1e-6, beta: float):
    """fp64 F2 forward (causal).  q,k,v [M,B,T,H,D]; planes [NP,L,K,D].
    Returns (out [M,B,T,H,D], den [M,B,H,T]) with out = num / max(den, floor)
    and den the sum over all L*2^K buckets of P_Q A(t) (unclamped)."""
    M, B, T, H, D = q.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, Dp = planes.shape
    assert Dp == D
    qs, ks, vs = to_streams(q), to_streams(k), to_streams(v)
    pm = _plane_map(M, B, H, NP)
    out = np.zeros_like(qs)
    den = np.zeros((qs.shape[0], T), dtype=np.float64)
    rc = _lib().oracle_race_global_forward(_dptr(qs), _dptr(ks), _dptr(vs), _dptr(planes),
                                           pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                           qs.shape[0], T, D, L, K, float(floor), float(beta),
                                           _dptr(out), _dptr(den))
    if rc != 0:
        raise ValueError("oracle_race_global_forward rejected its arguments")
    return from_streams(out, M, B, H), den.reshape(M, B, H, T)


def race_global_backward(q, k, v, dout, planes, *, dden=None, floor: float = 1e-6, beta: float,
                         with_l1: bool = False):
    """fp64 F2 backward for upstream gradients dout [M,B,T,H,D] and dden
    [M,B,H,T] (None = 0).  Returns (dq, dk, dv, grad_beta[, l1 mass of the
    grad_beta summands])."""
    M, B, T, H, D = q.shape
    planes = np.ascontiguousarray(np.asarray(planes, dtype=np.float64))
    NP, L, K, _ = planes.shape
    qs, ks, vs, gs = to_streams(q), to_streams(k), to_streams(v), to_streams(dout)
    hs = den_to_streams(dden, M, B, H) if dden is not None else None
    pm = _plane_map(M, B, H, NP)
    dq, dk, dv = np.zeros_like(qs), np.zeros_like(qs), np.zeros_like(qs)
    gb = np.zeros(2, dtype=np.float64)
    rc = _lib().oracle_race_global_backward(_dptr(qs), _dptr(ks), _dptr(vs), _dptr(gs),
                                            _dptr(hs) if hs is not None else None, _dptr(planes),
                                            pm.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                            qs.shape[0], T, D, L, K, float(floor), float(beta),
                                            _dptr(dq), _dptr(dk), _dptr(dv), _dptr(gb), _dptr(gb[1:]))
    if rc != 0:
        raise ValueError("oracle_race_global_backward rejected its arguments")
    res = (from_streams(dq, M, B, H), from_streams(dk, M, B, H), from_streams(dv, M, B, H), float(gb[0]))
    return res + (float(gb[1]),) if with_l1 else res


def prefix_mean_flat(w, v, eps: float = 1e-6):
    """Restatement of race_prefix_mean_flat: w [NS,T] f32, v [NS,T,D] f32 -> E."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    NS, T, D = v.shape
    E = np.empty_like(v)
    _lib().oracle_prefix_mean_flat(_fptr(w), _fptr(v), NS, T, D, float(eps), _fptr(E))
    return E


def prefix_mean_flat_bw(w, v, gE, eps: float = 1e-6):
    """Restatement of race_prefix_mean_flat_bw -> (gW [NS,T], gV [NS,T,D])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    gE = np.ascontiguousarray(gE, dtype=np.float32)
    NS, T, D = v.shape
    gW = np.empty_like(w)
    gV = np.empty_like(v)
    _lib().oracle_prefix_mean_flat_bw(_fptr(w), _fptr(v), _fptr(gE), NS, T, D, float(eps),
                                      _fptr(gW), _fptr(gV))
    return gW, gV


def ref_race_pref():
    """The reference's race_pref.cpp built from source into oracle/_ref/, or None."""
    hits = glob.glob(os.path.join(HERE, "_ref", "race_pref*.so"))
    if not hits:
        return None
    import torch  # noqa: F401  (the extension links against torch)
    spec = importlib.util.spec_from_file_location("race_pref", hits[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def corner_signs(K: int):
    """[R,K] corner coordinates used by race_oracle.c (bit K-1-k of r)."""
    R = 1 << K
    r = np.arange(R)[:, None]
    k = np.arange(K)[None, :]
    return np.where((r >> (K - 1 - k)) & 1, 1.0, -1.0)
