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
