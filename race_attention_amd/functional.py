"""Torch-facing calls into the HIP library and the autograd Functions.

``race_attention(Qhf, Khf, Vhf, planes, ...)`` is the operator behind the
reference's BatchedACE.forward (misc/race.py:63-142 causal,
misc/vit.py:918-978 non-causal): inputs [M,B,T,H,D] (D = 64, bf16 or fp32,
any strides with a contiguous last dimension, an M stride of 0 for the
reference's M-fold expand), hyperplanes [L,K,D] shared or [M,L,K,D]
per-estimator, output [M,B,T,H,D].  Forward and backward run as HIP kernels on
the current stream; bucket probabilities are recomputed in the backward.

``race_attention_ex(..., kmask=, with_den=)`` is the non-causal operator of
padded batches and of the denominator proxy: per-token key weights on P_K
(misc/classification.py:576-592) and den = sum_s P_Q A_s
(misc/classification.py:641-659, misc/vit.py:1452-1510).

``race_attention_global(Q, K, V, planes, beta, ...)`` is the globally
normalised causal operator ("F2") behind CausalRACEAttention
(misc/elsaa_causal_complete.py:438-586): it returns out = num / max(den, 1e-6)
and den [M,B,H,T] (fp32), both differentiable (the module's d_token is built
from den).

``RACEPrefixMeanFlatFn`` is the autograd Function of misc/race.py:9-24 with the
flat prefix mean computed by the HIP kernels instead of the CPU extension.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.RACE_DTYPE_BF16, torch.float32: _lib.RACE_DTYPE_F32}


def _require_gpu(*tensors):
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError("race_attention_amd runs on ROCm GPUs only; got a tensor on "
                               f"{t.device}")


def _strides4(x: torch.Tensor):
    if x.dim() != 5:
        raise ValueError(f"expected a [M,B,T,H,D] tensor, got shape {tuple(x.shape)}")
    if x.stride(4) != 1:
        raise ValueError("the last (head) dimension must be contiguous")
    return (ctypes.c_int64 * 4)(*[x.stride(j) if x.size(j) > 1 else 0 for j in range(4)])


def _aligned(x: torch.Tensor) -> torch.Tensor:
    """Make x usable by the kernels: contiguous D, 16-byte aligned rows."""
    es = x.element_size()
    ok = (x.stride(4) == 1 and x.data_ptr() % 16 == 0 and
          all((x.stride(j) * es) % 16 == 0 or x.size(j) == 1 for j in range(4)) and
          (x.size(2) == 1 or x.stride(2) >= x.size(4)))
    return x if ok else x.contiguous()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _no_rows(x: torch.Tensor) -> bool:
    """True for an [M,B,T,H,D] tensor with no (m, b, t, h) rows: an empty
    batch or sequence.  The operator then has nothing to compute, and the raw
    calls return empty outputs (and a zero temperature gradient) without a
    launch, as torch's own ops do on empty tensors; the C ABI itself requires
    M, B, T, H >= 1."""
    return x.dim() == 5 and x.shape[:4].numel() == 0


def _zero_grad_scalar(want, dev):
    return torch.zeros((), dtype=torch.float32, device=dev) if want else None


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def make_desc(q, k, v, planes, *, L, K, causal, eps, inv_temp, seg_tiles=0):
    M, B, T, H, D = q.shape
    d = _lib.RaceDesc()
    d.M, d.B, d.T, d.H, d.D = M, B, T, H, D
    d.L, d.K = int(L), int(K)
    d.causal = 1 if causal else 0
    if q.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {q.dtype} (bf16 or fp32)")
    d.dtype = _DTYPES[q.dtype]
    d.eps = float(eps)
    if torch.is_tensor(inv_temp) and inv_temp.is_cuda:
        # a device temperature stays on the GPU: the kernels read it through
        # inv_temp_ptr (no host synchronisation); the descriptor keeps the
        # fp32 scalar alive until the call has been enqueued
        t = inv_temp.detach().to(device=q.device, dtype=torch.float32).reshape(()).contiguous()
        d.inv_temp = 1.0
        d.inv_temp_ptr = t.data_ptr()
        d._temp_keep = t
    else:
        d.inv_temp = float(inv_temp)
    if planes.dim() == 3:
        d.planes_m_stride = 0
    elif planes.dim() == 4 and planes.size(0) == 1:
        d.planes_m_stride = 0
    elif planes.dim() == 4 and planes.size(0) == M:
        d.planes_m_stride = L * K * D
    else:
        raise ValueError(f"planes must be [L,K,D], [1,L,K,D] or [M,L,K,D]; got {tuple(planes.shape)}")
    d.q_stride, d.k_stride, d.v_stride = _strides4(q), _strides4(k), _strides4(v)
    d.seg_tiles = int(seg_tiles)
    return d


def _check_inputs(q, k, v, planes, L, K):
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"Q, K, V shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("Q, K, V dtypes differ")
    if planes.shape[-3:] != (L, K, q.shape[-1]):
        raise ValueError(f"planes trailing shape {tuple(planes.shape[-3:])} != (L, K, D) = ({L}, {K}, {q.shape[-1]})")


def race_fwd_raw(q, k, v, planes, *, L, K, causal, eps=1e-6, inv_temp, seg_tiles=0):
    """Forward only: returns (out [M,B,T,H,D] contiguous, state for race_bwd_raw)."""
    _require_gpu(q, k, v, planes)
    _check_inputs(q, k, v, planes, L, K)
    if _no_rows(q):
        return torch.empty(q.shape, dtype=q.dtype, device=q.device), torch.empty(0, dtype=torch.uint8, device=q.device)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    planes = planes.to(device=q.device, dtype=torch.float32).contiguous()
    lib = _lib.load()
    d = make_desc(q, k, v, planes, L=L, K=K, causal=causal, eps=eps, inv_temp=inv_temp, seg_tiles=seg_tiles)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    d.o_stride = _strides4(out)
    sb = lib.race_state_bytes(ctypes.byref(d))
    if sb == 0:
        _lib.check(-1, "race_state_bytes")
    wb = lib.race_fwd_workspace_bytes(ctypes.byref(d))
    state = torch.empty(sb, dtype=torch.uint8, device=q.device)
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=q.device)
    rc = lib.race_fwd(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(planes), _ptr(out), _ptr(state),
                      _ptr(ws), ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_fwd")
    return out, state


def race_bwd_raw(q, k, v, planes, dout, state, *, L, K, causal, eps=1e-6, inv_temp, seg_tiles=0,
                 want_temp_grad=True):
    """Backward: returns (dq, dk, dv, grad_inv_temp (0-dim fp32 tensor or None))."""
    _require_gpu(q, k, v, planes, dout, state)
    if _no_rows(q):
        e = [torch.empty(q.shape, dtype=q.dtype, device=q.device) for _ in range(3)]
        return e[0], e[1], e[2], _zero_grad_scalar(want_temp_grad, q.device)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    dout = _aligned(dout.to(q.dtype))
    planes = planes.to(device=q.device, dtype=torch.float32).contiguous()
    lib = _lib.load()
    d = make_desc(q, k, v, planes, L=L, K=K, causal=causal, eps=eps, inv_temp=inv_temp, seg_tiles=seg_tiles)
    d.do_stride = _strides4(dout)
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    d.g_stride = _strides4(dq)
    if state.numel() != lib.race_state_bytes(ctypes.byref(d)):
        raise ValueError("state buffer does not match this descriptor")
    wb = lib.race_bwd_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=q.device)
    git = torch.empty((), dtype=torch.float32, device=q.device) if want_temp_grad else None
    rc = lib.race_bwd(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(planes), _ptr(dout), _ptr(state),
                      _ptr(dq), _ptr(dk), _ptr(dv), _ptr(git) if git is not None else None,
                      _ptr(ws), ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_bwd")
    return dq, dk, dv, git


def _temp_value(temp, x):
    """The temperature an autograd Function runs with: a python float as is; a
    tensor as an fp32 0-dim device copy taken now (read in-kernel, so the
    forward never waits for the GPU, and the backward sees the forward's value
    even if the source is updated in place meanwhile)."""
    if torch.is_tensor(temp):
        if temp.is_cuda:
            return temp.detach().to(device=x.device, dtype=torch.float32).reshape(()).clone()
        return float(temp)
    return float(temp)


class RACEFunction(torch.autograd.Function):
    """Autograd Function of the RACE operator (F1 semantics).

    forward(Qhf, Khf, Vhf, planes, inv_temp, L, K, causal, eps) -> [M,B,T,H,D].
    inv_temp is a python float or a 0-dim tensor (then it receives a
    gradient).  planes are buffers (no gradient), as in the reference
    (misc/race.py:42-51)."""

    @staticmethod
    def forward(ctx, Qhf, Khf, Vhf, planes, inv_temp, L, K, causal, eps):
        it = _temp_value(inv_temp, Qhf)
        out, state = race_fwd_raw(Qhf, Khf, Vhf, planes, L=L, K=K, causal=causal, eps=eps, inv_temp=it)
        ctx.save_for_backward(Qhf, Khf, Vhf, planes, state)
        ctx.cfg = (L, K, causal, eps, it)
        ctx.temp_is_tensor = torch.is_tensor(inv_temp)
        return out

    @staticmethod
    def backward(ctx, dout):
        Qhf, Khf, Vhf, planes, state = ctx.saved_tensors
        L, K, causal, eps, it = ctx.cfg
        want = ctx.temp_is_tensor and ctx.needs_input_grad[4]
        dq, dk, dv, git = race_bwd_raw(Qhf, Khf, Vhf, planes, dout, state, L=L, K=K, causal=causal, eps=eps,
                                       inv_temp=it, want_temp_grad=want)
        return (dq if ctx.needs_input_grad[0] else None,
                dk if ctx.needs_input_grad[1] else None,
                dv if ctx.needs_input_grad[2] else None,
                None, git if want else None, None, None, None, None)


def race_attention(Qhf, Khf, Vhf, planes, *, L, K, causal, inv_temp, eps=1e-6):
    """Differentiable RACE operator on [M,B,T,H,D] tensors (see module doc)."""
    return RACEFunction.apply(Qhf, Khf, Vhf, planes, inv_temp, L, K, causal, eps)


# ------------------------------------------------- bucket probabilities as an output
def _probs_desc(x, planes, L, K, inv_temp):
    if x.dim() != 5:
        raise ValueError(f"expected x [M,B,T,H,D], got {tuple(x.shape)}")
    if planes.shape[-3:] != (L, K, x.shape[-1]):
        raise ValueError(f"planes trailing shape {tuple(planes.shape[-3:])} != (L, K, D)")
    return make_desc(x, x, x, planes, L=L, K=K, causal=False, eps=1e-6, inv_temp=inv_temp)


def race_probs_raw(x, planes, *, L, K, inv_temp):
    """Bucket probabilities of x [M,B,T,H,D]: fp32 [M,B,H,T,L*2^K]."""
    _require_gpu(x, planes)
    x = _aligned(x)
    planes = planes.to(device=x.device, dtype=torch.float32).contiguous()
    M, B, T, H, _ = x.shape
    if _no_rows(x):
        _probs_desc(x, planes, L, K, inv_temp)  # argument checks only
        return torch.empty((M, B, H, T, L << K), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    d = _probs_desc(x, planes, L, K, inv_temp)
    P = torch.empty((M, B, H, T, L << K), dtype=torch.float32, device=x.device)
    _lib.check(lib.race_probs(ctypes.byref(d), _ptr(x), _ptr(planes), _ptr(P), _stream()), "race_probs")
    return P


def race_probs_bwd_raw(x, planes, dP, *, L, K, inv_temp, want_temp_grad=True):
    """dP [M,B,H,T,S] -> (dx [M,B,T,H,D], grad_inv_temp or None)."""
    _require_gpu(x, planes, dP)
    x = _aligned(x)
    planes = planes.to(device=x.device, dtype=torch.float32).contiguous()
    M, B, T, H, _ = x.shape
    if dP.shape != (M, B, H, T, L << K):
        raise ValueError(f"dP must be [M,B,H,T,S] = {(M, B, H, T, L << K)}; got {tuple(dP.shape)}")
    if _no_rows(x):
        return torch.empty(x.shape, dtype=x.dtype, device=x.device), _zero_grad_scalar(want_temp_grad, x.device)
    dP = dP.to(torch.float32).contiguous()
    lib = _lib.load()
    d = _probs_desc(x, planes, L, K, inv_temp)
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    d.g_stride = _strides4(dx)
    ws = torch.empty(max(lib.race_probs_bwd_workspace_bytes(ctypes.byref(d)), 16), dtype=torch.uint8, device=x.device)
    git = torch.empty((), dtype=torch.float32, device=x.device) if want_temp_grad else None
    rc = lib.race_probs_bwd(ctypes.byref(d), _ptr(x), _ptr(planes), _ptr(dP), _ptr(dx),
                            _ptr(git) if git is not None else None, _ptr(ws), ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_probs_bwd")
    return dx, git


class RACEProbsFunction(torch.autograd.Function):
    """Bucket probabilities as a differentiable output:
    forward(x, planes, inv_temp, L, K) -> P [M,B,H,T,L*2^K] fp32; x and
    inv_temp (a 0-dim tensor) receive gradients."""

    @staticmethod
    def forward(ctx, x, planes, inv_temp, L, K):
        it = _temp_value(inv_temp, x)
        P = race_probs_raw(x, planes, L=L, K=K, inv_temp=it)
        ctx.save_for_backward(x, planes)
        ctx.cfg = (L, K, it, torch.is_tensor(inv_temp))
        return P

    @staticmethod
    def backward(ctx, dP):
        x, planes = ctx.saved_tensors
        L, K, it, is_t = ctx.cfg
        want = is_t and ctx.needs_input_grad[2]
        dx, git = race_probs_bwd_raw(x, planes, dP, L=L, K=K, inv_temp=it, want_temp_grad=want)
        return (dx if ctx.needs_input_grad[0] else None, None, git if want else None, None, None)


def race_bucket_probs(x, planes, *, L, K, inv_temp):
    """Soft bucket probabilities of x [M,B,T,H,D] -> [M,B,H,T,L,2^K] fp32
    (differentiable in x and a tensor inv_temp)."""
    M, B, T, H, _ = x.shape
    return RACEProbsFunction.apply(x, planes, inv_temp, L, K).view(M, B, H, T, L, 1 << K)


# ------------------------------------------------- key weights and den (F1 extras)
def _kmask_check(kmask, B, T, dev):
    if kmask is None:
        return None
    if kmask.shape != (B, T):
        raise ValueError(f"kmask must be [B,T] = {(B, T)}; got {tuple(kmask.shape)}")
    return kmask.to(device=dev, dtype=torch.float32).contiguous()


def race_fwd_ex_raw(q, k, v, planes, *, L, K, inv_temp, kmask=None, want_den=False, eps=1e-6, seg_tiles=0):
    """Non-causal forward with key weights kmask [B,T] (None = 1) and the den
    output: returns (out [M,B,T,H,D], den [M,B,H,T] fp32 or None, state)."""
    _require_gpu(q, k, v, planes)
    _check_inputs(q, k, v, planes, L, K)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    planes = planes.to(device=q.device, dtype=torch.float32).contiguous()
    M, B, T, H, _ = q.shape
    kmask = _kmask_check(kmask, B, T, q.device)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    den = torch.empty((M, B, H, T), dtype=torch.float32, device=q.device) if want_den else None
    if _no_rows(q):
        return out, den, torch.empty(0, dtype=torch.uint8, device=q.device)
    lib = _lib.load()
    d = make_desc(q, k, v, planes, L=L, K=K, causal=False, eps=eps, inv_temp=inv_temp, seg_tiles=seg_tiles)
    d.o_stride = _strides4(out)
    sb = lib.race_state_bytes(ctypes.byref(d))
    if sb == 0:
        _lib.check(-1, "race_state_bytes")
    wb = lib.race_fwd_ex_workspace_bytes(ctypes.byref(d))
    state = torch.empty(sb, dtype=torch.uint8, device=q.device)
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=q.device)
    rc = lib.race_fwd_ex(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(planes),
                         _ptr(kmask) if kmask is not None else None, _ptr(out),
                         _ptr(den) if den is not None else None, _ptr(state), _ptr(ws),
                         ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_fwd_ex")
    return out, den, state


def race_bwd_ex_raw(q, k, v, planes, dout, dden, state, *, L, K, inv_temp, kmask=None, eps=1e-6, seg_tiles=0,
                    want_temp_grad=True):
    """Backward of race_fwd_ex_raw: returns (dq, dk, dv, grad_inv_temp or None)."""
    _require_gpu(q, k, v, planes, state)
    if _no_rows(q):
        e = [torch.empty(q.shape, dtype=q.dtype, device=q.device) for _ in range(3)]
        return e[0], e[1], e[2], _zero_grad_scalar(want_temp_grad, q.device)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    M, B, T, H, _ = q.shape
    dout = _aligned(dout.to(q.dtype)) if dout is not None else torch.zeros(q.shape, dtype=q.dtype, device=q.device)
    planes = planes.to(device=q.device, dtype=torch.float32).contiguous()
    kmask = _kmask_check(kmask, B, T, q.device)
    if dden is not None:
        dden = _den_check(dden.to(torch.float32), M, B, H, T, "dden")
    lib = _lib.load()
    d = make_desc(q, k, v, planes, L=L, K=K, causal=False, eps=eps, inv_temp=inv_temp, seg_tiles=seg_tiles)
    d.do_stride = _strides4(dout)
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    d.g_stride = _strides4(dq)
    if state.numel() != lib.race_state_bytes(ctypes.byref(d)):
        raise ValueError("state buffer does not match this descriptor")
    wb = lib.race_bwd_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=q.device)
    git = torch.empty((), dtype=torch.float32, device=q.device) if want_temp_grad else None
    rc = lib.race_bwd_ex(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(planes),
                         _ptr(kmask) if kmask is not None else None, _ptr(dout),
                         _ptr(dden) if dden is not None else None, _ptr(state), _ptr(dq), _ptr(dk), _ptr(dv),
                         _ptr(git) if git is not None else None, _ptr(ws), ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_bwd_ex")
    return dq, dk, dv, git


class RACEExFunction(torch.autograd.Function):
    """Autograd Function of the non-causal operator with key weights and the
    den output: forward(Q, K, V, planes, inv_temp, kmask, L, K, eps,
    want_den) -> (out, den); den is an empty tensor unless want_den.  kmask
    (key weights, [B,T]) receives no gradient."""

    @staticmethod
    def forward(ctx, Q, Kx, V, planes, inv_temp, kmask, L, K, eps, want_den):
        it = _temp_value(inv_temp, Q)
        out, den, state = race_fwd_ex_raw(Q, Kx, V, planes, L=L, K=K, inv_temp=it, kmask=kmask,
                                          want_den=want_den, eps=eps)
        ctx.save_for_backward(Q, Kx, V, planes, kmask if kmask is not None else torch.empty(0), state)
        ctx.cfg = (L, K, eps, it, kmask is not None)
        ctx.temp_is_tensor = torch.is_tensor(inv_temp)
        ctx.set_materialize_grads(False)
        if den is None:
            den = torch.empty(0, dtype=torch.float32, device=Q.device)
        return out, den

    @staticmethod
    def backward(ctx, dout, dden):
        Q, Kx, V, planes, kmask, state = ctx.saved_tensors
        L, K, eps, it, has_mask = ctx.cfg
        want = ctx.temp_is_tensor and ctx.needs_input_grad[4]
        if dden is not None and dden.numel() == 0:
            dden = None
        dq, dk, dv, git = race_bwd_ex_raw(Q, Kx, V, planes, dout, dden, state, L=L, K=K, inv_temp=it,
                                          kmask=kmask if has_mask else None, eps=eps, want_temp_grad=want)
        return (dq if ctx.needs_input_grad[0] else None,
                dk if ctx.needs_input_grad[1] else None,
                dv if ctx.needs_input_grad[2] else None,
                None, git if want else None, None, None, None, None, None)


def race_attention_ex(Qhf, Khf, Vhf, planes, *, L, K, inv_temp, kmask=None, with_den=False, eps=1e-6):
    """Non-causal RACE on [M,B,T,H,D] with per-token key weights kmask [B,T]
    on P_K.  Returns out, or (out, den [M,B,H,T] unclamped) with with_den."""
    out, den = RACEExFunction.apply(Qhf, Khf, Vhf, planes, inv_temp, kmask, L, K, eps, bool(with_den))
    return (out, den) if with_den else out


# ------------------------------------------------- global normalisation (F2)
def _den_check(den, M, B, H, T, name):
    if den.shape != (M, B, H, T) or den.dtype != torch.float32:
        raise ValueError(f"{name} must be float32 [M,B,H,T] = {(M, B, H, T)}; got {den.dtype} {tuple(den.shape)}")
    return den.contiguous()


def race_global_fwd_raw(q, k, v, planes, *, L, K, beta, floor=1e-6, seg_tiles=0):
    """F2 forward: returns (out [M,B,T,H,D], den [M,B,H,T] fp32, state)."""
    _require_gpu(q, k, v, planes)
    _check_inputs(q, k, v, planes, L, K)
    M, B, T, H, _ = q.shape
    if _no_rows(q):
        return (torch.empty(q.shape, dtype=q.dtype, device=q.device),
                torch.empty((M, B, H, T), dtype=torch.float32, device=q.device),
                torch.empty(0, dtype=torch.uint8, device=q.device))
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    planes = planes.to(device=q.device, dtype=torch.float32).contiguous()
    lib = _lib.load()
    d = make_desc(q, k, v, planes, L=L, K=K, causal=True, eps=floor, inv_temp=beta, seg_tiles=seg_tiles)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    den = torch.empty((M, B, H, T), dtype=torch.float32, device=q.device)
    d.o_stride = _strides4(out)
    sb = lib.race_state_bytes(ctypes.byref(d))
    if sb == 0:
        _lib.check(-1, "race_state_bytes")
    wb = lib.race_fwd_global_workspace_bytes(ctypes.byref(d))
    state = torch.empty(sb, dtype=torch.uint8, device=q.device)
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=q.device)
    rc = lib.race_fwd_global(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(planes), _ptr(out), _ptr(den),
                             _ptr(state), _ptr(ws), ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_fwd_global")
    return out, den, state


def race_global_bwd_raw(q, k, v, planes, out, den, dout, dden, state, *, L, K, beta, floor=1e-6, seg_tiles=0,
                        want_beta_grad=True):
    """F2 backward: returns (dq, dk, dv, grad_beta (0-dim fp32 tensor or None)).
    dden (gradient of den, [M,B,H,T]) may be None."""
    _require_gpu(q, k, v, planes, out, den, dout, state)
    if _no_rows(q):
        e = [torch.empty(q.shape, dtype=q.dtype, device=q.device) for _ in range(3)]
        return e[0], e[1], e[2], _zero_grad_scalar(want_beta_grad, q.device)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    out = _aligned(out)
    dout = _aligned(dout.to(q.dtype))
    planes = planes.to(device=q.device, dtype=torch.float32).contiguous()
    M, B, T, H, _ = q.shape
    den = _den_check(den, M, B, H, T, "den")
    if dden is not None:
        dden = _den_check(dden.to(torch.float32), M, B, H, T, "dden")
    lib = _lib.load()
    d = make_desc(q, k, v, planes, L=L, K=K, causal=True, eps=floor, inv_temp=beta, seg_tiles=seg_tiles)
    d.o_stride = _strides4(out)
    d.do_stride = _strides4(dout)
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    d.g_stride = _strides4(dq)
    if state.numel() != lib.race_state_bytes(ctypes.byref(d)):
        raise ValueError("state buffer does not match this descriptor")
    wb = lib.race_bwd_global_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=q.device)
    gb = torch.empty((), dtype=torch.float32, device=q.device) if want_beta_grad else None
    rc = lib.race_bwd_global(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(planes), _ptr(out), _ptr(den),
                             _ptr(dout), _ptr(dden) if dden is not None else None, _ptr(state),
                             _ptr(dq), _ptr(dk), _ptr(dv), _ptr(gb) if gb is not None else None,
                             _ptr(ws), ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_bwd_global")
    return dq, dk, dv, gb


class RACEGlobalFunction(torch.autograd.Function):
    """Autograd Function of the globally normalised causal operator (F2).

    forward(Q, K, V, planes, beta, L, K, floor) -> (out [M,B,T,H,D], den
    [M,B,H,T] fp32).  beta is a python float or a 0-dim tensor (then it
    receives a gradient); planes are buffers (no gradient), as in the
    reference (misc/elsaa_causal_complete.py:473-474).  Replaces
    _RaceChunkwiseTritonFn (misc/elsaa_causal_complete.py:384-436) together
    with the probabilities, chunk states and division around it."""

    @staticmethod
    def forward(ctx, Q, Kx, V, planes, beta, L, K, floor):
        b = _temp_value(beta, Q)
        out, den, state = race_global_fwd_raw(Q, Kx, V, planes, L=L, K=K, beta=b, floor=floor)
        ctx.save_for_backward(Q, Kx, V, planes, out, den, state)
        ctx.cfg = (L, K, floor, b)
        ctx.beta_is_tensor = torch.is_tensor(beta)
        ctx.set_materialize_grads(False)  # an unused den arrives as None, not zeros
        return out, den

    @staticmethod
    def backward(ctx, dout, dden):
        Q, Kx, V, planes, out, den, state = ctx.saved_tensors
        L, K, floor, b = ctx.cfg
        want = ctx.beta_is_tensor and ctx.needs_input_grad[4]
        if dout is None:
            dout = torch.zeros_like(out)
        dq, dk, dv, gb = race_global_bwd_raw(Q, Kx, V, planes, out, den, dout, dden, state, L=L, K=K, beta=b,
                                             floor=floor, want_beta_grad=want)
        return (dq if ctx.needs_input_grad[0] else None,
                dk if ctx.needs_input_grad[1] else None,
                dv if ctx.needs_input_grad[2] else None,
                None, gb if want else None, None, None, None)


def race_attention_global(Qhf, Khf, Vhf, planes, *, L, K, beta, floor=1e-6):
    """Differentiable F2 operator on [M,B,T,H,D] tensors -> (out, den [M,B,H,T])."""
    return RACEGlobalFunction.apply(Qhf, Khf, Vhf, planes, beta, L, K, floor)


# ------------------------------------------------------------- prefix mean
def prefix_mean_fwd(w: torch.Tensor, v: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """race_prefix_mean_flat on the GPU: w [NS,T], v [NS,T,D] fp32 -> E [NS,T,D]."""
    _require_gpu(w, v)
    if w.dtype != torch.float32 or v.dtype != torch.float32:
        raise TypeError("probsK_flat and V_flat must be float32")      # race_pref.cpp:9
    if w.dim() != 2 or v.dim() != 3 or w.shape != v.shape[:2]:
        raise ValueError("shapes must be [NS,T] and [NS,T,D] with matching NS and T")
    w, v = w.contiguous(), v.contiguous()
    NS, T, D = v.shape
    E = torch.empty_like(v)
    if v.numel() == 0:  # race_pref.cpp returns its empty output too
        return E
    lib = _lib.load()
    wb = lib.race_prefix_mean_workspace_bytes(NS, T, D)
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=v.device)
    rc = lib.race_prefix_mean_fwd(_ptr(w), _ptr(v), _ptr(E), NS, T, D, float(eps), _ptr(ws),
                                  ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_prefix_mean_fwd")
    return E


def prefix_mean_bwd(w, v, gE, eps: float = 1e-6):
    """race_prefix_mean_flat_bw on the GPU -> (gW [NS,T], gV [NS,T,D])."""
    _require_gpu(w, v, gE)
    w, v, gE = w.contiguous(), v.contiguous(), gE.contiguous().to(torch.float32)
    NS, T, D = v.shape
    gW = torch.empty_like(w)
    gV = torch.empty_like(v)
    if v.numel() == 0:
        return gW.zero_(), gV
    lib = _lib.load()
    wb = lib.race_prefix_mean_workspace_bytes(NS, T, D)
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=v.device)
    rc = lib.race_prefix_mean_bwd(_ptr(w), _ptr(v), _ptr(gE), _ptr(gW), _ptr(gV), NS, T, D, float(eps),
                                  _ptr(ws), ctypes.c_size_t(ws.numel()), _stream())
    _lib.check(rc, "race_prefix_mean_bwd")
    return gW, gV


class RACEPrefixMeanFlatFn(torch.autograd.Function):
    """misc/race.py:9-24 with the HIP prefix-mean kernels."""

    @staticmethod
    def forward(ctx, probsK_flat, V_flat, eps):
        E_flat = prefix_mean_fwd(probsK_flat, V_flat, float(eps))
        ctx.save_for_backward(probsK_flat, V_flat)
        ctx.eps = float(eps)
        return E_flat

    @staticmethod
    def backward(ctx, gradE_flat):
        probsK_flat, V_flat = ctx.saved_tensors
        gW, gV = prefix_mean_bwd(probsK_flat, V_flat, gradE_flat.contiguous(), ctx.eps)
        return gW, gV, None
