"""Pins for the globally normalised causal mode ("F2") of the CPU oracle --
CPU only.

F2 (CausalRACEAttention, misc/elsaa_causal_complete.py:438-586; Triton
readout misc/race_kernel.py:8-124):
    out_t = sum_s P_Q[t,s] B_s(t) / max(sum_s P_Q[t,s] A_s(t), 1e-6)
with A, B the inclusive causal prefixes of P_K and P_K v over all L tables.

What pins oracle.race_global_forward / race_global_backward:
  first token          out_0 = v_0 exactly (one key: num = den * v_0)
  constant values      out_t = c for v = c (num = c * den)
  kernel form          the Triton kernel's own formulation: the masked product
                       tril(phiQ phiK^T) applied to V and summed over tables
                       (race_kernel.py:57-123), probabilities from the closed
                       form prod_k sigmoid(2 beta c_rk tanh(proj_k))
  chunked fallback     a torch fp64 restatement of the module's chunked path
                       (inter-chunk states + intra-chunk masked products,
                       misc/elsaa_causal_complete.py:483-586); its autograd
                       pins the analytic backward (dq, dk, dv, d beta, d den)
  gradients            central finite differences in fp64, with an upstream
                       gradient on den and with the clamp active
"""
import itertools

import numpy as np
import pytest
import torch


def _inputs(rng, M=1, B=1, T=9, H=2, D=8):
    return [rng.standard_normal((M, B, T, H, D)) for _ in range(4)]


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _probs(x, planes, beta):
    """[T,L*R] bucket probabilities of one stream x [T,D] (closed form)."""
    L, K, D = planes.shape
    u = np.tanh(np.einsum("td,lkd->tlk", x, planes)) * beta
    c = np.array(list(itertools.product([-1., +1.], repeat=K)))
    return np.prod(_sig(2.0 * c[None, None] * u[:, :, None, :]), axis=-1).reshape(x.shape[0], -1)


def test_first_token_and_constant_values(oracle):
    rng = np.random.default_rng(1)
    q, k, v, _ = _inputs(rng, M=1, B=2, T=11, H=3)
    pl = rng.standard_normal((1, 3, 2, 8))
    out, den = oracle.race_global_forward(q, k, v, pl, beta=1.4)
    np.testing.assert_allclose(out[:, :, 0], v[:, :, 0], rtol=1e-13, atol=1e-14)
    assert np.all(den > 0)
    c = np.full_like(v, -0.35)
    out_c, den_c = oracle.race_global_forward(q, k, c, pl, beta=1.4)
    np.testing.assert_allclose(out_c, c, rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(den_c, den, rtol=1e-14)       # den does not read v


@pytest.mark.parametrize("K,L", [(1, 2), (2, 3), (4, 2)])
def test_kernel_form_brute_force(oracle, K, L):
    """num = tril(sum_l phiQ_l phiK_l^T) V, den = row sums (race_kernel.py:77-109)."""
    rng = np.random.default_rng(10 + K)
    T, D, beta = 13, 8, 0.9
    q, k, v, _ = _inputs(rng, T=T, H=1, D=D)
    pl = rng.standard_normal((1, L, K, D))
    out, den = oracle.race_global_forward(q, k, v, pl, beta=beta)
    PQ = _probs(q[0, 0, :, 0], pl[0], beta)
    PK = _probs(k[0, 0, :, 0], pl[0], beta)
    Mx = np.tril(PQ @ PK.T)
    num = Mx @ v[0, 0, :, 0]
    dn = Mx.sum(axis=1)
    np.testing.assert_allclose(den[0, 0, 0], dn, rtol=1e-12)
    np.testing.assert_allclose(out[0, 0, :, 0], num / np.maximum(dn, 1e-6)[:, None], rtol=1e-12, atol=1e-14)


def test_clamp_floor(oracle):
    """A floor above every den divides by the floor instead (clamp_min)."""
    rng = np.random.default_rng(3)
    q, k, v, _ = _inputs(rng, T=6, H=1)
    pl = rng.standard_normal((1, 2, 2, 8))
    out, den = oracle.race_global_forward(q, k, v, pl, beta=1.0)
    fl = 10.0 * den.max()
    out_f, den_f = oracle.race_global_forward(q, k, v, pl, beta=1.0, floor=fl)
    np.testing.assert_allclose(den_f, den, rtol=1e-14)
    num = out * den[0, 0, 0][None, None, :, None, None]   # den > 1e-6 here
    np.testing.assert_allclose(out_f, num / fl, rtol=1e-12, atol=1e-15)


from f2_torch_ref import chunked as _chunked  # noqa: E402


@pytest.mark.parametrize("C", [4, 16])
def test_chunked_restatement_and_autograd(oracle, C):
    rng = np.random.default_rng(20 + C)
    B, T, H, D, L, K, beta = 2, 11, 2, 8, 3, 2, 1.3
    q, k, v, g = _inputs(rng, M=1, B=B, T=T, H=H, D=D)
    h = rng.standard_normal((1, B, H, T))
    pl = rng.standard_normal((1, L, K, D))
    out, den = oracle.race_global_forward(q, k, v, pl, beta=beta)
    dq, dk, dv, gb = oracle.race_global_backward(q, k, v, g, pl, dden=h, beta=beta)

    def bhtd(x):
        return torch.tensor(x[0]).permute(0, 2, 1, 3).contiguous().requires_grad_(True)

    Q, Kt, V = bhtd(q), bhtd(k), bhtd(v)
    bt = torch.tensor(beta, dtype=torch.float64, requires_grad=True)
    o_t, d_t = _chunked(Q, Kt, V, torch.tensor(pl[0]), bt, C)
    np.testing.assert_allclose(o_t.detach().permute(0, 2, 1, 3).numpy(), out[0], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(d_t.detach().numpy(), den[0], rtol=1e-12)
    G = torch.tensor(g[0]).permute(0, 2, 1, 3)
    loss = (o_t * G).sum() + (d_t * torch.tensor(h[0])).sum()
    loss.backward()
    for mine, ref in ((dq, Q), (dk, Kt), (dv, V)):
        np.testing.assert_allclose(mine[0], ref.grad.permute(0, 2, 1, 3).numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gb, bt.grad.item(), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("floor_active", [False, True])
def test_gradients_finite_difference(oracle, floor_active):
    rng = np.random.default_rng(31 + floor_active)
    L, K, D, T, beta = 2, 2, 4, 6, 0.8
    q, k, v, g = _inputs(rng, T=T, H=1, D=D)
    hd = rng.standard_normal((1, 1, 1, T))
    pl = rng.standard_normal((1, L, K, D))
    _, den = oracle.race_global_forward(q, k, v, pl, beta=beta)
    fl = 3.0 * den.max() if floor_active else 1e-6
    dq, dk, dv, gb = oracle.race_global_backward(q, k, v, g, pl, dden=hd, beta=beta, floor=fl)

    def loss(qq, kk, vv, bb):
        o, d = oracle.race_global_forward(qq, kk, vv, pl, beta=bb, floor=fl)
        return np.sum(o * g) + np.sum(d * hd)

    eps = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        fd = np.zeros_like(arr)
        it_ = np.nditer(arr, flags=["multi_index"])
        for _ in it_:
            idx = it_.multi_index
            a0 = arr[idx]
            arr[idx] = a0 + eps
            lp = loss(q, k, v, beta)
            arr[idx] = a0 - eps
            lm = loss(q, k, v, beta)
            arr[idx] = a0
            fd[idx] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-8)
    fd_b = (loss(q, k, v, beta + eps) - loss(q, k, v, beta - eps)) / (2 * eps)
    np.testing.assert_allclose(gb, fd_b, rtol=1e-6, atol=1e-8)


def test_shared_and_per_estimator_planes(oracle):
    rng = np.random.default_rng(40)
    q, k, v, _ = _inputs(rng, M=2, B=1, T=7, H=2)
    pl = rng.standard_normal((2, 2, 2, q.shape[-1]))
    both, den = oracle.race_global_forward(q, k, v, pl, beta=1.0)
    for m in range(2):
        one, d1 = oracle.race_global_forward(q[m:m + 1], k[m:m + 1], v[m:m + 1], pl[m:m + 1], beta=1.0)
        np.testing.assert_allclose(both[m:m + 1], one, rtol=1e-13, atol=1e-14)
        np.testing.assert_allclose(den[m:m + 1], d1, rtol=1e-13)
