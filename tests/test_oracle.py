"""Pins for the CPU oracle (oracle/race_oracle.c) -- CPU only.

What pins each oracle function (a plausible mistake fails at least one):
  corner ordering        itertools.product, the reference's own construction
                         (misc/race.py:54-58); hard-hash limit (sign of proj)
  soft hash              closed form prod_k sigmoid(2 c_rk u_k); T=1 closed form;
                         odd symmetry; tau -> inf uniform limit
  causal aggregation     reference kernel race_pref.cpp compiled from source
                         (oracle/_ref) through the reference CPU path; golden
                         vectors written by that kernel; brute force O(T^2)
  readout sum over S     constant-v identity (sum_s P_Q = L) and L-duplication
  non-causal             equals causal at t = T-1; uniform limit closed form
  gradients              central finite differences in fp64 (dq, dk, dv, d inv_temp);
                         reference CPU path autograd (causal)
  prefix mean (flat)     reference kernel outputs (live and golden fixture)
"""
import itertools
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _inputs(rng, M=1, B=1, T=9, H=2, D=8):
    return [rng.standard_normal((M, B, T, H, D)) for _ in range(4)]


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def test_corner_order_matches_itertools(oracle):
    for K in (1, 2, 3, 4, 8):
        ref = np.array(list(itertools.product([-1., +1.], repeat=K)))
        assert np.array_equal(oracle.corner_signs(K), ref)


def _probs_closed_form(x, planes, inv_temp):
    """P[t,l,r] = prod_k sigmoid(2 c_rk u_k) for one stream x [T,D], planes [L,K,D]."""
    L, K, D = planes.shape
    u = np.tanh(np.einsum("td,lkd->tlk", x, planes)) * inv_temp
    c = np.array(list(itertools.product([-1., +1.], repeat=K)))       # [R,K]
    return np.prod(_sig(2.0 * c[None, None, :, :] * u[:, :, None, :]), axis=-1)  # [T,L,R]


@pytest.mark.parametrize("K", [1, 2, 4])
def test_single_token_closed_form(oracle, K):
    """T=1: out = sum_s P_Q[s] P_K[s] v / (P_K[s] + eps) with P from the closed form."""
    rng = np.random.default_rng(K)
    L, D, eps, it = 3, 8, 1e-6, 0.7
    q, k, v, _ = _inputs(rng, T=1, H=1, D=D)
    pl = rng.standard_normal((1, L, K, D))
    out = oracle.race_forward(q, k, v, pl, causal=True, eps=eps, inv_temp=it)
    PQ = _probs_closed_form(q[0, 0, :, 0], pl[0], it).reshape(-1)
    PK = _probs_closed_form(k[0, 0, :, 0], pl[0], it).reshape(-1)
    expect = np.sum(PQ * PK / (PK + eps)) * v[0, 0, 0, 0]
    np.testing.assert_allclose(out[0, 0, 0, 0], expect, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("causal", [True, False])
def test_constant_values_sum_over_all_buckets(oracle, causal):
    """v_t = c, eps = 0  =>  out_t = c * sum_s P_Q[t,s] = c * L  (no 1/L)."""
    rng = np.random.default_rng(3)
    L, K, D = 5, 2, 8
    q, k, _, _ = _inputs(rng, T=13, H=2, D=D)
    c = rng.standard_normal(D)
    v = np.broadcast_to(c, q.shape).copy()
    pl = rng.standard_normal((1, L, K, D))
    out = oracle.race_forward(q, k, v, pl, causal=causal, eps=0.0, inv_temp=1.3)
    np.testing.assert_allclose(out, np.broadcast_to(L * c, out.shape), rtol=1e-12, atol=1e-12)


def test_table_duplication_scales_by_L(oracle):
    rng = np.random.default_rng(4)
    K, D = 3, 8
    q, k, v, _ = _inputs(rng, T=11, D=D)
    one = rng.standard_normal((1, 1, K, D))
    o1 = oracle.race_forward(q, k, v, one, causal=True, inv_temp=0.5)
    o4 = oracle.race_forward(q, k, v, np.repeat(one, 4, axis=1), causal=True, inv_temp=0.5)
    np.testing.assert_allclose(o4, 4 * o1, rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("causal", [True, False])
def test_uniform_limit(oracle, causal):
    """inv_temp = 0 -> P = 1/R: causal out_t = L * mean(v_0..t) (eps=0); non-causal L*mean(v)."""
    rng = np.random.default_rng(5)
    L, K = 3, 2
    q, k, v, _ = _inputs(rng, T=10)
    pl = rng.standard_normal((1, L, K, q.shape[-1]))
    out = oracle.race_forward(q, k, v, pl, causal=causal, eps=0.0, inv_temp=0.0)
    T = v.shape[2]
    if causal:
        expect = L * np.cumsum(v, axis=2) / np.arange(1, T + 1)[None, None, :, None, None]
    else:
        expect = np.broadcast_to(L * v.mean(axis=2, keepdims=True), v.shape)
    np.testing.assert_allclose(out, expect, rtol=1e-12, atol=1e-12)


def test_hard_hash_limit(oracle):
    """inv_temp -> large: P becomes one-hot at the corner whose bits follow
    sign(proj) (bit K-1-k of r set iff proj_k > 0); causal output becomes the
    bucket-wise running mean of v, summed over tables."""
    rng = np.random.default_rng(6)
    L, K, D, T = 2, 3, 8, 24
    q, k, v, _ = _inputs(rng, T=T, H=1, D=D)
    pl = rng.standard_normal((1, L, K, D))
    out = oracle.race_forward(q, k, v, pl, causal=True, eps=1e-12, inv_temp=2e3)

    def code(x):
        bits = (np.einsum("td,lkd->tlk", x, pl[0]) > 0).astype(int)     # [T,L,K]
        return (bits * (1 << (K - 1 - np.arange(K)))).sum(-1)          # [T,L]

    cq, ck = code(q[0, 0, :, 0]), code(k[0, 0, :, 0])
    vv = v[0, 0, :, 0]
    expect = np.zeros((T, D))
    for t in range(T):
        for l in range(L):
            sel = [tau for tau in range(t + 1) if ck[tau, l] == cq[t, l]]
            if sel:
                expect[t] += vv[sel].mean(0)
    np.testing.assert_allclose(out[0, 0, :, 0], expect, atol=2e-3)


def test_odd_symmetry(oracle):
    """P(-x)[r] = P(x)[R-1-r], a relabelling shared by Q and K: out(-q,-k,v) = out(q,k,v)."""
    rng = np.random.default_rng(7)
    q, k, v, _ = _inputs(rng, T=12)
    pl = rng.standard_normal((1, 2, 3, q.shape[-1]))
    a = oracle.race_forward(q, k, v, pl, causal=True, inv_temp=0.9)
    b = oracle.race_forward(-q, -k, v, pl, causal=True, inv_temp=0.9)
    np.testing.assert_allclose(a, b, rtol=1e-11, atol=1e-13)


def test_noncausal_equals_causal_last_token(oracle):
    rng = np.random.default_rng(8)
    q, k, v, _ = _inputs(rng, T=15)
    pl = rng.standard_normal((1, 3, 2, q.shape[-1]))
    c = oracle.race_forward(q, k, v, pl, causal=True, inv_temp=1.0)
    # non-causal output at any t with the full state == causal state at T-1 applied to q_t
    qq = np.broadcast_to(q[:, :, -1:], q.shape).copy()
    nc = oracle.race_forward(qq, k, v, pl, causal=False, inv_temp=1.0)
    np.testing.assert_allclose(nc[:, :, 0], c[:, :, -1], rtol=1e-12, atol=1e-13)


def test_causal_brute_force(oracle):
    """O(T^2) definition from the closed-form probabilities."""
    rng = np.random.default_rng(9)
    L, K, D, T, eps, it = 2, 2, 8, 7, 1e-6, 1.7
    q, k, v, _ = _inputs(rng, T=T, H=1, D=D)
    pl = rng.standard_normal((1, L, K, D))
    out = oracle.race_forward(q, k, v, pl, causal=True, eps=eps, inv_temp=it)
    PQ = _probs_closed_form(q[0, 0, :, 0], pl[0], it).reshape(T, -1)
    PK = _probs_closed_form(k[0, 0, :, 0], pl[0], it).reshape(T, -1)
    vv = v[0, 0, :, 0]
    for t in range(T):
        o = np.zeros(D)
        for s in range(PQ.shape[1]):
            A = sum(PK[tau, s] for tau in range(t + 1))
            Bs = sum(PK[tau, s] * vv[tau] for tau in range(t + 1))
            o += PQ[t, s] * Bs / (A + eps)
        np.testing.assert_allclose(out[0, 0, t, 0], o, rtol=1e-12, atol=1e-14)


def test_independent_planes_per_estimator(oracle):
    rng = np.random.default_rng(10)
    q, k, v, _ = _inputs(rng, M=2, B=1, T=8, H=2)
    pl = rng.standard_normal((2, 2, 2, q.shape[-1]))
    both = oracle.race_forward(q, k, v, pl, causal=False, inv_temp=1.0)
    for m in range(2):
        one = oracle.race_forward(q[m:m + 1], k[m:m + 1], v[m:m + 1], pl[m:m + 1],
                                  causal=False, inv_temp=1.0)
        np.testing.assert_allclose(both[m:m + 1], one, rtol=1e-13, atol=1e-14)


@pytest.mark.parametrize("causal", [True, False])
def test_gradients_finite_difference(oracle, causal):
    rng = np.random.default_rng(11 + causal)
    L, K, D, T, it = 2, 2, 4, 6, 0.8
    q, k, v, g = _inputs(rng, T=T, H=1, D=D)
    pl = rng.standard_normal((1, L, K, D))
    dq, dk, dv, git = oracle.race_backward(q, k, v, g, pl, causal=causal, inv_temp=it)

    def loss(qq, kk, vv, ii):
        return np.sum(oracle.race_forward(qq, kk, vv, pl, causal=causal, inv_temp=ii) * g)

    h = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        fd = np.zeros_like(arr)
        it_ = np.nditer(arr, flags=["multi_index"])
        for _ in it_:
            idx = it_.multi_index
            a0 = arr[idx]
            arr[idx] = a0 + h
            lp = loss(q, k, v, it)
            arr[idx] = a0 - h
            lm = loss(q, k, v, it)
            arr[idx] = a0
            fd[idx] = (lp - lm) / (2 * h)
        np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-8)
    fd_it = (loss(q, k, v, it + h) - loss(q, k, v, it - h)) / (2 * h)
    np.testing.assert_allclose(git, fd_it, rtol=1e-6, atol=1e-8)


def _ref_or_skip(oracle):
    ext = oracle.ref_race_pref()
    if ext is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return ext


def test_prefix_mean_restatement_vs_reference_kernel(oracle):
    import torch
    ext = _ref_or_skip(oracle)
    rng = np.random.default_rng(12)
    NS, T, D = 24, 200, 16
    w = rng.random((NS, T)).astype(np.float32)
    v = rng.standard_normal((NS, T, D)).astype(np.float32)
    g = rng.standard_normal((NS, T, D)).astype(np.float32)
    E = oracle.prefix_mean_flat(w, v)
    E_ref = ext.race_prefix_mean_flat(torch.from_numpy(w), torch.from_numpy(v), 1e-6).numpy()
    assert np.array_equal(E, E_ref)
    gW, gV = oracle.prefix_mean_flat_bw(w, v, g)
    gW_ref, gV_ref = ext.race_prefix_mean_flat_bw(torch.from_numpy(w), torch.from_numpy(v),
                                                  torch.from_numpy(g), 1e-6)
    assert np.array_equal(gW, gW_ref.numpy())
    assert np.array_equal(gV, gV_ref.numpy())


def test_prefix_mean_golden_vectors(oracle):
    """Vectors written by the reference kernel (tests/golden/make_prefix_mean_golden.py)."""
    z = np.load(os.path.join(GOLDEN, "prefix_mean_ref.npz"))
    E = oracle.prefix_mean_flat(z["w"], z["v"], float(z["eps"]))
    assert np.array_equal(E, z["E"])
    gW, gV = oracle.prefix_mean_flat_bw(z["w"], z["v"], z["gE"], float(z["eps"]))
    assert np.array_equal(gW, z["gW"])
    assert np.array_equal(gV, z["gV"])


def test_oracle_vs_reference_cpu_path(oracle):
    """Full causal operator: oracle (fp64) vs the reference CPU path (fp32 aten +
    compiled race_pref.cpp), forward and all input gradients."""
    import torch
    from oracle import ref_cpu_path
    ext = _ref_or_skip(oracle)
    rng = np.random.default_rng(13)
    M, B, T, H, D, L, K = 1, 2, 41, 3, 16, 4, 3
    q, k, v, g = _inputs(rng, M=M, B=B, T=T, H=H, D=D)
    pl = rng.standard_normal((1, L, K, D))
    o = oracle.race_forward(q, k, v, pl, causal=True, inv_temp=1 / np.sqrt(D))
    dq, dk, dv, _ = oracle.race_backward(q, k, v, g, pl, causal=True, inv_temp=1 / np.sqrt(D))
    planes_T = torch.tensor(pl[0].reshape(L * K, D).T, dtype=torch.float32)
    Kt, Vt, Qt = [torch.tensor(x, dtype=torch.float32, requires_grad=True) for x in (k, v, q)]
    out = ref_cpu_path.causal_forward(Kt, Vt, Qt, planes_T, K, L, ext=ext)
    out.backward(torch.tensor(g, dtype=torch.float32))

    def rel(a, b):
        return np.abs(a - b).max() / np.abs(a).max()

    assert rel(o, out.detach().numpy()) < 1e-5
    assert rel(dq, Qt.grad.numpy()) < 1e-5
    assert rel(dk, Kt.grad.numpy()) < 1e-5
    assert rel(dv, Vt.grad.numpy()) < 1e-5
