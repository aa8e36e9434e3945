"""Pins for the bucket-probability functions of the CPU oracle
(race_probs / race_probs_bwd; misc/arxiv_64K.py:1580-1644,
misc/vit.py:3193-3262) -- CPU only.

  closed form    P = prod_k sigmoid(2 c_rk u_k) per table; rows sum to 1
  autograd       a torch fp64 restatement of the reference's aten path
                 (projection, tanh, / temperature, corner logits, softmax)
                 pins dx and d inv_temp through torch.autograd
"""
import itertools

import numpy as np
import torch


def test_probs_closed_form_and_normalisation(oracle):
    rng = np.random.default_rng(0)
    M, B, T, H, D, L, K, it = 2, 1, 7, 2, 8, 3, 3, 0.6
    x = rng.standard_normal((M, B, T, H, D))
    pl = rng.standard_normal((M, L, K, D))
    P = oracle.race_probs(x, pl, inv_temp=it)
    assert P.shape == (M, B, H, T, L << K)
    np.testing.assert_allclose(P.reshape(M, B, H, T, L, -1).sum(-1), 1.0, rtol=1e-13)
    c = np.array(list(itertools.product([-1., +1.], repeat=K)))
    for m in range(M):
        for h in range(H):
            u = np.tanh(np.einsum("td,lkd->tlk", x[m, 0, :, h], pl[m])) * it
            ref = np.prod(1 / (1 + np.exp(-2 * c[None, None] * u[:, :, None, :])), axis=-1).reshape(T, -1)
            np.testing.assert_allclose(P[m, 0, h], ref, rtol=1e-12)


def test_probs_backward_autograd(oracle):
    rng = np.random.default_rng(1)
    M, B, T, H, D, L, K, it = 1, 2, 5, 2, 8, 2, 4, 1.3
    x = rng.standard_normal((M, B, T, H, D))
    pl = rng.standard_normal((1, L, K, D))
    dP = rng.standard_normal((M, B, H, T, L << K))
    dx, git = oracle.race_probs_bwd(x, dP, pl, inv_temp=it)
    xt = torch.tensor(x, requires_grad=True)
    itt = torch.tensor(it, dtype=torch.float64, requires_grad=True)
    protos = torch.tensor(list(itertools.product([-1., +1.], repeat=K)), dtype=torch.float64).T  # [K, R]
    planes_T = torch.tensor(pl[0]).reshape(L * K, D).T                                             # [D, L*K]
    proj = xt.permute(0, 1, 3, 2, 4) @ planes_T                                                    # [M,B,H,T,L*K]
    logits = (proj.view(M, B, H, T, L, K).tanh() * itt) @ protos
    P = torch.softmax(logits, dim=-1).reshape(M, B, H, T, -1)
    np.testing.assert_allclose(P.detach().numpy(), oracle.race_probs(x, pl, inv_temp=it), rtol=1e-12)
    (P * torch.tensor(dP)).sum().backward()
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(git, itt.grad.item(), rtol=1e-10)
