"""The bf16 error-budget restatement (tests/error_budget.py) is the operator
itself when no rounding is applied: it equals the fp64 oracle (which follows
kernels/cpu/race_pref.cpp) to fp64 rounding, including ragged last tiles.  Its
rounding switches are then the only difference from the exact operator."""
import numpy as np

import error_budget as eb


def test_budget_restatement_is_the_operator(oracle):
    for T, shift in ((70, 0.0), (160, 0.5)):
        q, k, v, g, planes = eb.inputs(T=T, H=2, shift=shift)
        it = 1.0 / 8.0
        got = eb.run(q, k, v, g, planes, it)
        o = oracle.race_forward(q, k, v, planes, causal=True, inv_temp=it)
        dq, dk, dv, _ = oracle.race_backward(q, k, v, g, planes, causal=True, inv_temp=it)
        for name, a, b in zip(("out", "dq", "dk", "dv"), got, (o, dq, dk, dv)):
            e = eb.relerr(a, b)
            assert e < 1e-11, (T, name, e)


def test_bf16_rounding_is_exact_to_nearest_even():
    """bf16 keeps 8 significant bits: spacing 2^-7 just above 1."""
    x = np.array([1.0, 1.0 + 2 ** -7, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5])
    r = eb.bf16(x)
    assert r[0] == 1.0 and r[1] == 1.0 + 2 ** -7   # representable
    assert r[2] == 1.0                            # tie: to the even significand
    assert r[3] == 1.0 + 2 ** -6                  # tie: 1 + 2^-7 is odd, 1 + 2^-6 even
    assert r[4] == 1.0 + 2 ** -7                  # above the tie: up
    assert r[5] == -2.5


def test_slice_partials_add_up_to_the_table():
    """The softmax backward of a 256-bucket table as two 128-bucket slices'
    partials, du_z = sum_{r in z} P dP c_r - (sum_{r in z} P dP) tanh(u), adds
    up to the whole table's (sum_r P c_r = tanh(u) over a table): with no
    rounding of the partials, the two forms agree to fp64 rounding."""
    rng = np.random.default_rng(3)
    T, L, K, it = 40, 4, 8, 0.125
    planes = rng.standard_normal((L, K, 64))
    x = rng.standard_normal((T, 64))
    P, th = eb.soft_hash(x, planes, it)
    dP = rng.standard_normal(P.shape) + 0.5
    whole = eb.soft_hash_bwd(P, dP, th, planes, it)
    parts = eb.soft_hash_bwd(P, dP, th, planes, it, xpart=lambda y: y)
    assert np.abs(parts - whole).max() <= 1e-12 * np.abs(whole).max()
    # a bf16 rounding of each partial is relative to the partials
    rounded = eb.soft_hash_bwd(P, dP, th, planes, it, xpart=eb.bf16)
    assert np.abs(rounded - whole).max() > 0


def test_small_table_operand_pairs():
    """Two-bit tables at the 1/sqrt(d) temperature: bucket probabilities are
    nearly flat, and the softmax backward of dQ and dK cancels what a table's
    buckets share.  With single bf16 operands for P_K, W and U the restatement's
    dQ / dK error is at the bf16 bar; with the small-table instantiations' hi +
    lo pairs (hl) it is a third of that.  hl without roundings is the exact
    operator."""
    q, k, v, g, planes = eb.inputs(T=608, H=2, L=5, K=2, seed=0)
    it = 1.0 / 8.0
    exact = eb.run(q, k, v, g, planes, it)
    single = [eb.relerr(a, b) for a, b in zip(eb.run(q, k, v, g, planes, it, on=eb.ROUNDINGS), exact)]
    pairs = [eb.relerr(a, b) for a, b in zip(eb.run(q, k, v, g, planes, it, on=eb.ROUNDINGS, hl=True), exact)]
    assert max(single[1:3]) > 1.2e-2, single
    assert max(pairs[1:3]) < 6e-3, pairs
    none = eb.run(q, k, v, g, planes, it, hl=True)
    assert max(eb.relerr(a, b) for a, b in zip(none, exact)) < 1e-11


def _gn_case(K, L, T, seed, dden):
    rng = np.random.default_rng(seed)
    nrm = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)  # noqa: E731
    q, k, v = (eb.bf16(nrm(rng.standard_normal((2, 1, T, 2, 64)))) for _ in range(3))
    g = eb.bf16(rng.standard_normal((2, 1, T, 2, 64)))
    h = rng.standard_normal((2, 1, 2, T)) if dden else None
    planes = rng.standard_normal((2, L, K, 64)).astype(np.float32).astype(np.float64)
    return q, k, v, g, h, planes


def test_gn_restatement_is_the_operator(oracle):
    """The globally normalised restatement (stream_gn) with no rounding equals
    the fp64 F2 oracle, out, den and every gradient, with either form of
    dL/d den (the kernels' own sums, or dO . out with token 0 as dO . v_0) and
    with the slice partials summed."""
    for K, L, T, beta, dden in ((4, 8, 100, 1.0, True), (2, 5, 70, 3.0, False), (6, 3, 90, 2.0, True)):
        q, k, v, g, h, planes = _gn_case(K, L, T, K, dden)
        o, den = oracle.race_global_forward(q, k, v, planes, beta=beta)
        dq, dk, dv, _ = oracle.race_global_backward(q, k, v, g, planes, dden=h, beta=beta)
        for own_gd in (True, False):
            got = eb.run_gn(q, k, v, g, h, planes, beta, own_gd=own_gd, slice_parts=K > 4)
            for name, a, b in zip(("out", "den", "dq", "dk", "dv"), got, (o, den, dq, dk, dv)):
                e = eb.relerr(a, b)
                assert e < 1e-11, (K, own_gd, name, e)


def test_gn_first_token_cancels_with_every_rounding():
    """Token 0's dq is exactly zero without dden (out_0 = v_0).  With every
    bf16 rounding on, dL/d den formed from the kernels' own sums, sum_s P_Q G,
    keeps it zero to fp64 rounding; formed from the stored bf16 output,
    dO . y_0, it does not."""
    q, k, v, g, _, planes = _gn_case(4, 6, 64, 7, False)
    beta = 3.0
    exact = eb.run_gn(q, k, v, g, None, planes, beta)
    scale = np.abs(exact[2]).max()
    own = eb.run_gn(q, k, v, g, None, planes, beta, on=eb.ROUNDINGS)
    stored = eb.run_gn(q, k, v, g, None, planes, beta, on=eb.ROUNDINGS, own_gd=False)
    assert np.abs(own[2][:, :, 0]).max() <= 1e-12 * scale
    assert np.abs(stored[2][:, :, 0]).max() > 5e-4 * scale  # 1.4e-3 here
