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
