"""Pins for the F1 extras of the CPU oracle -- per-token key weights (the
padding mask of misc/classification.py:576-592) and the den output of
misc/classification.py:641-659 / misc/vit.py:1452-1510 -- CPU only.

What pins oracle.race_forward_ex / race_backward_ex:
  no extras          equal to race_forward (F1) with all-ones weights
  0/1 weights        the same as deleting the masked keys' tokens: outputs of
                     the kept queries equal F1 on the compressed sequence
                     (the per-sample valid-length loop of
                     misc/classification_glue_extended.py:838-848 is the
                     trailing-padding case), causal and non-causal
  den                brute force sum_s P_Q[t,s] A_s(t) from closed-form probabilities
  gradients          central finite differences in fp64 (fractional weights,
                     an upstream den gradient; causal and non-causal)
"""
import itertools

import numpy as np
import pytest


def _inputs(rng, M=1, B=1, T=9, H=2, D=8):
    return [rng.standard_normal((M, B, T, H, D)) for _ in range(4)]


def _probs(x, planes, it):
    L, K, D = planes.shape
    u = np.tanh(np.einsum("td,lkd->tlk", x, planes)) * it
    c = np.array(list(itertools.product([-1., +1.], repeat=K)))
    return np.prod(1.0 / (1.0 + np.exp(-2.0 * c[None, None] * u[:, :, None, :])), axis=-1).reshape(x.shape[0], -1)


@pytest.mark.parametrize("causal", [True, False])
def test_no_extras_equals_f1(oracle, causal):
    rng = np.random.default_rng(1 + causal)
    q, k, v, _ = _inputs(rng, M=2, B=2, T=10, H=2)
    pl = rng.standard_normal((2, 3, 2, 8))
    ref = oracle.race_forward(q, k, v, pl, causal=causal, inv_temp=0.8)
    out, _ = oracle.race_forward_ex(q, k, v, pl, causal=causal, inv_temp=0.8)
    np.testing.assert_array_equal(out, ref)
    ones = np.ones((2, 10))
    out1, _ = oracle.race_forward_ex(q, k, v, pl, kmask=ones, causal=causal, inv_temp=0.8)
    np.testing.assert_array_equal(out1, ref)


@pytest.mark.parametrize("causal", [True, False])
def test_binary_mask_equals_deleted_tokens(oracle, causal):
    rng = np.random.default_rng(5 + causal)
    B, T, H = 2, 12, 2
    q, k, v, _ = _inputs(rng, B=B, T=T, H=H)
    pl = rng.standard_normal((1, 2, 3, 8))
    mask = np.ones((B, T))
    mask[0, 9:] = 0                       # trailing padding (valid length 9)
    mask[1, [2, 5, 6, 11]] = 0            # scattered
    out, den = oracle.race_forward_ex(q, k, v, pl, kmask=mask, causal=causal, inv_temp=1.1)
    for b in range(B):
        keep = np.nonzero(mask[b])[0]
        sub = [x[:, b:b + 1, keep] for x in (q, k, v)]
        ref = oracle.race_forward(*sub, pl, causal=causal, inv_temp=1.1)
        np.testing.assert_allclose(out[:, b:b + 1, keep], ref, rtol=1e-12, atol=1e-14)
        _, den_ref = oracle.race_forward_ex(*sub, pl, causal=causal, inv_temp=1.1)
        np.testing.assert_allclose(den[:, b:b + 1][..., keep], den_ref, rtol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_den_brute_force(oracle, causal):
    rng = np.random.default_rng(9 + causal)
    T, D, L, K, it = 11, 8, 2, 3, 0.6
    q, k, v, _ = _inputs(rng, T=T, H=1, D=D)
    pl = rng.standard_normal((1, L, K, D))
    w = rng.uniform(0.2, 1.5, size=(1, T))
    _, den = oracle.race_forward_ex(q, k, v, pl, kmask=w, causal=causal, inv_temp=it)
    PQ = _probs(q[0, 0, :, 0], pl[0], it)
    PK = _probs(k[0, 0, :, 0], pl[0], it) * w[0][:, None]
    for t in range(T):
        A = PK[:t + 1].sum(0) if causal else PK.sum(0)
        np.testing.assert_allclose(den[0, 0, 0, t], PQ[t] @ A, rtol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_gradients_finite_difference(oracle, causal):
    rng = np.random.default_rng(21 + causal)
    L, K, D, T, it = 2, 2, 4, 6, 0.8
    q, k, v, g = _inputs(rng, T=T, H=1, D=D)
    h = rng.standard_normal((1, 1, 1, T))
    w = rng.uniform(0.3, 1.2, size=(1, T))
    pl = rng.standard_normal((1, L, K, D))
    dq, dk, dv, git = oracle.race_backward_ex(q, k, v, g, pl, kmask=w, dden=h, causal=causal, inv_temp=it)

    def loss(qq, kk, vv, ii):
        o, d = oracle.race_forward_ex(qq, kk, vv, pl, kmask=w, causal=causal, inv_temp=ii)
        return np.sum(o * g) + np.sum(d * h)

    e = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        fd = np.zeros_like(arr)
        it_ = np.nditer(arr, flags=["multi_index"])
        for _ in it_:
            idx = it_.multi_index
            a0 = arr[idx]
            arr[idx] = a0 + e
            lp = loss(q, k, v, it)
            arr[idx] = a0 - e
            lm = loss(q, k, v, it)
            arr[idx] = a0
            fd[idx] = (lp - lm) / (2 * e)
        np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-8)
    fd_it = (loss(q, k, v, it + e) - loss(q, k, v, it - e)) / (2 * e)
    np.testing.assert_allclose(git, fd_it, rtol=1e-6, atol=1e-8)
