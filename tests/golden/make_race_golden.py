"""Write tests/golden/race_golden.npz: small seeded cases with the fp64 oracle's
outputs and gradients (oracle/race_oracle.c, pinned by tests/test_oracle.py).
The GPU parity test compares the HIP operator against these stored vectors as
well as against the live oracle, so a later change to the oracle cannot move
the target silently.

    python tests/golden/make_race_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))
from helpers import make_case, to64  # noqa: E402
from oracle import race_oracle as ro  # noqa: E402

CASES = {
    # name: (make_case kwargs, causal, inv_temp)
    "causal_bf16": (dict(B=1, T=40, H=1, L=8, K=4, seed=101), True, 0.125),
    "noncausal_fp32": (dict(B=1, T=36, H=1, L=5, K=2, dtype=torch.float32, unit=False, seed=102), False, 1.0),
    "causal_fp32": (dict(B=1, T=33, H=1, L=5, K=2, dtype=torch.float32, unit=False, seed=103), True, 0.8),
}


def main():
    out = {}
    for nm, (kw, causal, it) in CASES.items():
        q, k, v, do, planes = make_case(**kw)
        bf16 = q.dtype == torch.bfloat16
        arrs = {s: x.float().numpy() for s, x in (("q", q), ("k", k), ("v", v), ("do", do))}
        pl = planes.double().numpy()
        o = ro.race_forward(to64(q), to64(k), to64(v), pl, causal=causal, inv_temp=it)
        dq, dk, dv, git, gabs = ro.race_backward(to64(q), to64(k), to64(v), to64(do), pl, causal=causal,
                                                 inv_temp=it, with_l1=True)
        rec = dict(arrs, planes=planes.numpy(), out=o.astype(np.float32), dq=dq.astype(np.float32),
                   dk=dk.astype(np.float32), dv=dv.astype(np.float32), dinv_temp=np.float64(git), dinv_temp_l1=np.float64(gabs),
                   L=np.int64(kw["L"]), K=np.int64(kw["K"]), causal=np.int64(causal),
                   inv_temp=np.float64(it), bf16=np.int64(bf16))
        for key, val in rec.items():
            out[f"{nm}__{key}"] = val
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "race_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
