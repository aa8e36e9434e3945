"""Write tests/golden/prefix_mean_ref.npz: seeded inputs and the outputs of the
reference's own CPU kernel (kernels/cpu/race_pref.cpp, compiled from source by
oracle/build_ref.py) for race_prefix_mean_flat and race_prefix_mean_flat_bw.

Run from the repository root in a tree where oracle/_ref is built:
    python tests/golden/make_prefix_mean_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import race_oracle  # noqa: E402


def main():
    ext = race_oracle.ref_race_pref()
    if ext is None:
        raise SystemExit("oracle/_ref is not built")
    rng = np.random.default_rng(2024)
    NS, T, D, eps = 6, 48, 8, 1e-6
    w = rng.random((NS, T)).astype(np.float32)
    w[0, :5] = 0.0                    # leading zero weights: A_t = 0 -> E = 0
    w[1, 7] = 1e-8                    # tiny weight next to eps
    v = rng.standard_normal((NS, T, D)).astype(np.float32)
    gE = rng.standard_normal((NS, T, D)).astype(np.float32)
    E = ext.race_prefix_mean_flat(torch.from_numpy(w), torch.from_numpy(v), eps).numpy()
    gW, gV = ext.race_prefix_mean_flat_bw(torch.from_numpy(w), torch.from_numpy(v),
                                          torch.from_numpy(gE), eps)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "prefix_mean_ref.npz")
    np.savez_compressed(out, w=w, v=v, gE=gE, eps=np.float64(eps), E=E, gW=gW.numpy(), gV=gV.numpy())
    print("wrote", out)


if __name__ == "__main__":
    main()
