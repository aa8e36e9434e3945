"""fp64 checks for full-length causal runs, where the oracle is too slow for
every token (configs C4 at N = 2^20 and 2^22).

Independent restatement of the operator's math for a few heads (torch fp64,
on whatever device the tensors live; contiguous operands only):

  * probs(x): the soft hash P[t, l*2^K + r] = prod_k sigmoid(+-2 tanh(x.w_lk) it),
    sign + iff bit (K-1-k) of r is set (the corner order of
    itertools.product([-1, 1], repeat=K), misc/race.py:54-58);
  * totals(): A_s = sum_t P_K[t, s], B_s = sum_t P_K[t, s] v_t over a token range;
  * suffix_reference(): with dO zero before the last T0 tokens, the backward
    carries of every earlier token are constants of those T0 tokens
    (kernels/cpu/race_pref.cpp:188-216 and the chunked form of the survey's
    Appendix B):  W = P_Q/(A(t)+eps), G = g.B(t), dA = -W G/(A(t)+eps),
    U_s = sum_t W[t,s] g_t, alpha_s = sum_t dA[t,s]; then for tau before the
    last T0 tokens
        dV_tau     = sum_s P_K[tau, s] U_s,
        dP_K[tau,s] = alpha_s + v_tau . U_s,
    and dK_tau through the softmax / tanh / projection backward
    (autograd of misc/race.py:79-105), dQ_tau = 0 exactly.
"""
import math

import torch


def corner_signs(K, dev):
    """c[r, k] = +1 iff bit (K-1-k) of r is set, else -1."""
    R = 1 << K
    return torch.tensor([[1.0 if (r >> (K - 1 - k)) & 1 else -1.0 for k in range(K)] for r in range(R)],
                        dtype=torch.float64, device=dev)


def probs(x, planes, it, L, K):
    """x [n, D] fp64, planes [L, K, D] fp64 -> P [n, L*2^K]."""
    proj = x @ planes.reshape(L * K, -1).T.contiguous()          # [n, L*K]
    u = torch.tanh(proj) * it
    logits = u.reshape(-1, L, 1, K) * corner_signs(K, x.device)  # [n, L, R, K]
    return torch.softmax(logits.sum(-1), dim=-1).reshape(x.shape[0], -1)


def totals(k, v, h, planes, it, L, K, t0, t1, step=1 << 16):
    """A [S], B [S, D] over tokens [t0, t1) of head h of [1,1,T,H,D] tensors."""
    S = L << K
    A = torch.zeros(S, dtype=torch.float64, device=k.device)
    Bs = torch.zeros(S, k.shape[-1], dtype=torch.float64, device=k.device)
    for a in range(t0, t1, step):
        b = min(t1, a + step)
        kc = k[0, 0, a:b, h].double()
        vc = v[0, 0, a:b, h].double()
        P = probs(kc, planes, it, L, K)
        A += P.sum(0)
        Bs += P.T.contiguous() @ vc
    return A, Bs


def suffix_reference(q, k, v, do, h, planes, it, L, K, T0, eps, taus):
    """(dK, dV) [len(taus), D] fp64 of head h at tokens taus < T - T0, for a
    run whose dO is zero before the last T0 tokens."""
    T = q.shape[2]
    dev = q.device
    A, Bsum = totals(k, v, h, planes, it, L, K, 0, T - T0)
    U = torch.zeros_like(Bsum)
    alpha = torch.zeros_like(A)
    sub = 1024
    for a in range(T - T0, T, sub):  # the last T0 tokens, running prefixes
        b = min(T, a + sub)
        kc, vc, qc, gc = [x[0, 0, a:b, h].double() for x in (k, v, q, do)]
        PK, PQ = probs(kc, planes, it, L, K), probs(qc, planes, it, L, K)
        At = A + torch.cumsum(PK, 0)                                         # [n, S]
        Bt = Bsum + torch.cumsum(PK[:, :, None] * vc[:, None, :], 0)         # [n, S, D]
        G = (Bt * gc[:, None, :]).sum(-1)                                    # g_t . B_s(t)
        inv = 1.0 / (At + eps)
        W = PQ * inv
        U += W.T.contiguous() @ gc
        alpha += (-W * G * inv).sum(0)
        A, Bsum = At[-1], Bt[-1]
    ks, vs = k[0, 0, taus, h].double(), v[0, 0, taus, h].double()
    PK = probs(ks, planes, it, L, K)
    dV = PK @ U
    dPK = alpha[None, :] + vs @ U.T.contiguous()
    R = 1 << K
    P3, dP3 = PK.reshape(-1, L, R), dPK.reshape(-1, L, R)
    dlog = P3 * (dP3 - (P3 * dP3).sum(-1, keepdim=True))                    # softmax backward
    du = dlog @ corner_signs(K, dev)                                         # [n, L, K]
    pl2 = planes.reshape(L * K, -1)
    th = torch.tanh(ks @ pl2.T.contiguous())
    dproj = du.reshape(-1, L * K) * it * (1 - th * th)
    dK = dproj @ pl2
    return dK, dV


def sample_taus(T, T0, seed=5, n=24):
    """Early token positions: tile and segment edges plus random ones."""
    g = torch.Generator().manual_seed(seed)
    fixed = [0, 1, 31, 32, 33, 4095, 4096, 65535, 65536, 131071, T // 2, T - T0 - 33, T - T0 - 1]
    rnd = torch.randint(0, T - T0, (n,), generator=g).tolist()
    return sorted(set(t for t in fixed + rnd if 0 <= t < T - T0))


def last_token_reference(q, k, v, h, planes, it, L, K, eps):
    """Causal output of head h at t = T-1: the readout over the whole sequence."""
    T = q.shape[2]
    A, Bs = totals(k, v, h, planes, it, L, K, 0, T)
    pq = probs(q[0, 0, T - 1:T, h].double(), planes, it, L, K)[0]
    return (pq / (A + eps)) @ Bs


def inv_temp_default(D):
    return 1.0 / math.sqrt(D)
