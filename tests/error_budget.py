"""bf16 error budget of the causal RACE operator: which roundings of the bf16
kernels (race_attention_amd/csrc/race_kernels.hip) account for the error of
out, dQ, dK and dV against the exact operator.

A numpy fp64 restatement of the tile algorithm the kernels run (32-token
tiles: the recurrence of kernels/cpu/race_pref.cpp:36-220 cut into tiles), in
which every value the kernels round to bf16 passes through a switchable
rounding:

  P      P_K as an MFMA operand: every sum over tokens of P_K (A, B, the
         in-tile triangles, dV) uses bf16 P_K (P_Q stays fp32 until it is
         part of W);
  W      W = P_Q / (A(t) + eps) as an operand (outputs, U, Sc, Sc2; dP_K's
         in-tile term takes W as an fp32-accurate hi + lo pair in every bf16
         instantiation, so W never rounds there);
  B      the carried B_s at a tile start as a bf16 operand: O's carried part and
         the G of k_bwd_out (for dA).  (k_bwd_reduce's G, which feeds dQ, takes
         B as an fp32-accurate hi + lo pair, so it is never rounded there);
  U      the carried U_s at a tile end as an operand (dP_K's v.U, dV);
  tri    the in-tile 32 x 32 blocks Sc = tril(W P_K^T), Sc2 = triu(P_K W^T)
         and M = tril(v g^T), stored or taken as bf16;
  dproj  d(projection) rows (bf16 in LDS) and planes^T (bf16) in dX = dproj
         planes (8-bit hashes: the rows reach the product as an fp32-accurate
         hi + lo pair, so only planes^T rounds there -- taken as the K <= 4 case
         here, an upper bound);
  out    the bf16 rounding of the outputs themselves (out, dQ, dK, dV).

One more switch is not a rounding of the current kernels: xpart rounds each
128-bucket slice's partial d(projection) of a table wider than a slice (8-bit
hashes, two slices per table) to bf16 before the slices are added, as bf16
partials would.  The partials of a column can cancel (the softmax backward's
mean term), so that rounding is relative to the partials, not the sum; the
kernels keep them fp32 for that reason (race_kernels.hip xpart_f32).
`python tests/error_budget.py --k8` prints the comparison.

Everything else is exact here: the fp32-accurate projection (hi/lo split of
the planes), the sigmoid factors, A's fp64 carries, fp32 accumulation (far
below 2^-9), the softmax backward's hi/lo table sums.  The kernels' carries of
B in fp32 are also taken as exact (their walk error is bounded by the segment
length, see race_capi.hip kMaxSegTiles).

hl=True models the small-table instantiations (race_kernels.hip hl_ops: bf16
with at most 3 hash bits, or 4 bits in at most 64 buckets), which take P_K,
W and the carried U as fp32-accurate hi + lo operand pairs wherever a sum
feeds the gradients' softmax backward: P_K in A, in B and in the in-tile G
term; W in U (and, as in every instantiation, in dP_K's in-tile term); U in
dP_K's v . U term.  P and W keep their rounding in the output triangles and
dV, U in dV.

With every rounding off the restatement equals the oracle (tests/
test_error_budget.py pins it there).  `python tests/error_budget.py [T]`
prints the error of each rounding alone and of all together; with --gpu (on a
GPU) also the HIP operator's own error on the same inputs.
"""
from __future__ import annotations

import itertools
import sys

import numpy as np

TT = 32
ROUNDINGS = ("P", "W", "B", "U", "tri", "dproj", "out")
SLICE = 128  # buckets per bf16 slice


def bf16(x: np.ndarray) -> np.ndarray:
    """Round to the nearest bf16 (ties to even), via fp32."""
    x32 = np.ascontiguousarray(x, dtype=np.float32)
    u = x32.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def corners(K: int) -> np.ndarray:
    """c[r, k] = +1 iff bit (K-1-k) of r is set (itertools.product order, misc/race.py:54-58)."""
    return np.array([[1.0 if (r >> (K - 1 - k)) & 1 else -1.0 for k in range(K)] for r in range(1 << K)])


def soft_hash(x, planes, it):
    """x [T, D], planes [L, K, D] -> P [T, L*R], th [T, L*K] (th = tanh(x . w))."""
    L, K, D = planes.shape
    th = np.tanh(x @ planes.reshape(L * K, D).T)
    u = th.reshape(-1, L, K) * it
    logits = np.einsum("tlk,rk->tlr", u, corners(K))
    logits -= logits.max(-1, keepdims=True)
    P = np.exp(logits)
    P /= P.sum(-1, keepdims=True)
    return P.reshape(x.shape[0], -1), th


def soft_hash_bwd(P, dP, th, planes, it, xpart=None):
    """d(projection) [T, L*K] from dP [T, L*R] through the softmax over corners
    and tanh.  xpart (a rounding): tables wider than SLICE buckets are summed
    from per-slice partials du_z = sum_{r in z} P dP c_r - (sum_{r in z} P dP)
    tanh(u), each passed through xpart before the slices are added."""
    L, K, D = planes.shape
    R = 1 << K
    P3, dP3 = P.reshape(-1, L, R), dP.reshape(-1, L, R)
    dth = it * (1.0 - th * th)
    if xpart is None or R <= SLICE:
        dlog = P3 * (dP3 - (P3 * dP3).sum(-1, keepdims=True))
        du = np.einsum("tlr,rk->tlk", dlog, corners(K)).reshape(-1, L * K)
        return du * dth
    c, tu = corners(K), np.tanh(th.reshape(-1, L, K) * it)
    out = np.zeros((P.shape[0], L, K))
    for z in range(R // SLICE):
        sl = slice(z * SLICE, (z + 1) * SLICE)
        pd = P3[:, :, sl] * dP3[:, :, sl]
        du = np.einsum("tlr,rk->tlk", pd, c[sl]) - pd.sum(-1, keepdims=True) * tu
        out += xpart(du * dth.reshape(-1, L, K))
    return out.reshape(-1, L * K)


def stream(q, k, v, g, planes, it, eps, on=(), hl=False):
    """One causal stream: q, k, v, g [T, D] (bf16-valued fp64), planes [L, K, D].
    Returns out, dq, dk, dv [T, D] with the roundings named in `on` applied
    (hl: the small-table operand pairs)."""
    r = {name: (bf16 if name in on else (lambda x: x)) for name in ROUNDINGS}
    xp = bf16 if "xpart" in on else None
    T, D = q.shape
    L, K, _ = planes.shape
    PQ, thq = soft_hash(q, planes, it)
    PK, thk = soft_hash(k, planes, it)
    PKr = r["P"](PK)
    PKx = PK if hl else PKr  # P_K in A, B and the in-tile G term
    S = PK.shape[1]
    nt = (T + TT - 1) // TT
    A0 = np.zeros((nt, S))      # A, B at each tile start (exact carries)
    B0 = np.zeros((nt, S, D))
    out = np.zeros((T, D))
    W = np.zeros((T, S))
    Wr = np.zeros((T, S))
    Ac = np.zeros(S)
    Bc = np.zeros((S, D))
    for c in range(nt):
        a, b = c * TT, min(T, c * TT + TT)
        A0[c], B0[c] = Ac, Bc
        pk, px, vv = PKr[a:b], PKx[a:b], v[a:b]
        At = Ac + np.cumsum(px, 0)                                   # A_s(t), t in the tile
        W[a:b] = PQ[a:b] / (At + eps)
        w = r["W"](W[a:b])
        Wr[a:b] = w
        Sc = r["tri"](np.tril(w @ pk.T))                             # Sc[t, t'] = sum_s W P_K, t' <= t
        out[a:b] = w @ r["B"](Bc) + Sc @ vv
        Bc = Bc + px.T @ vv
        Ac = Ac + px.sum(0)
    dq_proj = np.zeros((T, L * K))
    dk_proj = np.zeros((T, L * K))
    dv = np.zeros((T, D))
    Uc = np.zeros((S, D))
    alc = np.zeros(S)
    for c in reversed(range(nt)):
        a, b = c * TT, min(T, c * TT + TT)
        pk, px, vv, gg, w = PKr[a:b], PKx[a:b], v[a:b], g[a:b], Wr[a:b]
        wx = W[a:b] if hl else w                                      # W in U
        At = A0[c] + np.cumsum(px, 0)
        inv = 1.0 / (At + eps)
        M = r["tri"](np.triu(vv @ gg.T))                             # M[tau, t] = v_tau . g_t, tau <= t
        tri_g = M.T @ px                                              # in-tile part of G[t, s] = g_t . B_s(t)
        dPQ = (gg @ B0[c].T + tri_g) * inv                            # k_bwd_reduce: hi + lo B
        dA = -W[a:b] * (gg @ r["B"](B0[c]).T + tri_g) * inv           # k_bwd_out: bf16 B; fp32 W
        alpha = alc + np.cumsum(dA[::-1], 0)[::-1]                    # suffix from tau on
        Ur = r["U"](Uc)
        dPK = alpha + vv @ (Uc if hl else Ur).T + M @ W[a:b]          # sum_{t >= tau} M[tau, t] W[t, s]: a pair
        Sc2 = r["tri"](np.triu(pk @ w.T))                             # Sc2[tau, t] = sum_s P_K W, t >= tau
        dv[a:b] = pk @ Ur + Sc2 @ gg
        Uc = Uc + wx.T @ gg
        alc = alc + dA.sum(0)
        dq_proj[a:b] = soft_hash_bwd(PQ[a:b], dPQ, thq[a:b], planes, it, xp)
        dk_proj[a:b] = soft_hash_bwd(PK[a:b], dPK, thk[a:b], planes, it, xp)
    pl = planes.reshape(L * K, D)
    dq = r["dproj"](dq_proj) @ r["dproj"](pl)
    dk = r["dproj"](dk_proj) @ r["dproj"](pl)
    return tuple(r["out"](x) for x in (out, dq, dk, dv))


def stream_gn(q, k, v, g, h, planes, beta, floor, on=(), hl=False, own_gd=True, slice_parts=False):
    """One causal stream of the globally normalised operator (F2): num = sum_s
    P_Q B_s(t), den = sum_s P_Q A_s(t) over all tables, out = num / max(den,
    floor); h [T] is the upstream gradient of den.  The same switches as
    `stream`, placed where the GN kernels round:
      forward   W = P_Q as an operand (outputs, Sc), den from fp32 P_Q and A;
      backward  G with B as a hi + lo pair and the in-tile M rounded (tri);
                gd = h - [den >= floor] rd^2 sum_s P_Q G, as the kernels form
                it (own_gd; own_gd=False: h - [den >= floor] rd dO.y with y the
                stored output, the form the kernels avoid);
                W = P_Q rd as an operand in U, Sc2 and dV, an fp32-accurate
                pair in dP_K's in-tile term for tables up to 7 bits.
    slice_parts: the bucket-slice kernels round each 128-bucket slice's
    numerator and dV (its own Sc, Sc2 blocks) to bf16 (as "out") before the
    slices are summed (and the numerator divided).
    Returns out, den, dq, dk, dv [T, D] ([T] for den)."""
    r = {name: (bf16 if name in on else (lambda x: x)) for name in ROUNDINGS}
    T, D = q.shape
    L, K, _ = planes.shape
    PQ, thq = soft_hash(q, planes, beta)
    PK, thk = soft_hash(k, planes, beta)
    PKr = r["P"](PK)
    PKx = PK if hl else PKr  # P_K in A, B and the in-tile G term
    S = PK.shape[1]
    nt = (T + TT - 1) // TT
    A0 = np.zeros((nt, S))
    B0 = np.zeros((nt, S, D))
    out = np.zeros((T, D))
    den = np.zeros(T)
    Ac = np.zeros(S)
    Bc = np.zeros((S, D))
    nz = (S + SLICE - 1) // SLICE if slice_parts else 1
    for c in range(nt):
        a, b = c * TT, min(T, c * TT + TT)
        A0[c], B0[c] = Ac, Bc
        pk, px, vv = PKr[a:b], PKx[a:b], v[a:b]
        At = Ac + np.cumsum(px, 0)
        den[a:b] = (PQ[a:b] * At).sum(1)
        w = r["W"](PQ[a:b])
        num = np.zeros((b - a, D))
        for z in range(nz):
            sl = slice(z * SLICE, (z + 1) * SLICE) if slice_parts else slice(0, S)
            Sc = r["tri"](np.tril(w[:, sl] @ pk[:, sl].T))
            part = w[:, sl] @ r["B"](Bc[sl]) + Sc @ vv
            num += r["out"](part) if slice_parts else part
        out[a:b] = num / np.maximum(den[a:b], floor)[:, None]
        Bc = Bc + px.T @ vv
        Ac = Ac + px.sum(0)
    y = r["out"](out)
    act = den >= floor
    rd = 1.0 / np.maximum(den, floor)
    dq_proj = np.zeros((T, L * K))
    dk_proj = np.zeros((T, L * K))
    dv = np.zeros((T, D))
    Uc = np.zeros((S, D))
    alc = np.zeros(S)
    for c in reversed(range(nt)):
        a, b = c * TT, min(T, c * TT + TT)
        pk, px, vv, gg = PKr[a:b], PKx[a:b], v[a:b], g[a:b]
        At = A0[c] + np.cumsum(px, 0)
        M = r["tri"](np.triu(vv @ gg.T))
        G = gg @ B0[c].T + M.T @ px
        if own_gd:
            gd = h[a:b] - act[a:b] * rd[a:b] ** 2 * (PQ[a:b] * G).sum(1)
        else:
            gd = h[a:b] - act[a:b] * rd[a:b] * (gg * y[a:b]).sum(1)
        dPQ = G * rd[a:b, None] + gd[:, None] * At
        dA = gd[:, None] * PQ[a:b]
        W = PQ[a:b] * rd[a:b, None]
        w = r["W"](W)
        wx = W if hl else w
        alpha = alc + np.cumsum(dA[::-1], 0)[::-1]
        Ur = r["U"](Uc)
        dPK = alpha + vv @ (Uc if hl else Ur).T + M @ (W if (hl or K < 8) else w)
        for z in range(nz):
            sl = slice(z * SLICE, (z + 1) * SLICE) if slice_parts else slice(0, S)
            Sc2 = r["tri"](np.triu(pk[:, sl] @ w[:, sl].T))
            part = pk[:, sl] @ Ur[sl] + Sc2 @ gg
            dv[a:b] += r["out"](part) if slice_parts else part
        Uc = Uc + wx.T @ gg
        alc = alc + dA.sum(0)
        dq_proj[a:b] = soft_hash_bwd(PQ[a:b], dPQ, thq[a:b], planes, beta)
        dk_proj[a:b] = soft_hash_bwd(PK[a:b], dPK, thk[a:b], planes, beta)
    pl = planes.reshape(L * K, D)
    dq = r["dproj"](dq_proj) @ r["dproj"](pl)
    dk = r["dproj"](dk_proj) @ r["dproj"](pl)
    return y, den, r["out"](dq), r["out"](dk), r["out"](dv)


def run_gn(q, k, v, g, h, planes, beta, floor=1e-6, on=(), hl=False, own_gd=True, slice_parts=False):
    """F2 over [M,B,T,H,D] arrays (h: [M,B,H,T] or None), planes [NP,L,K,D]
    (NP = 1 or M) -> out, den [M,B,H,T], dq, dk, dv."""
    M, B, T, H, D = q.shape
    res = [np.zeros_like(q), np.zeros((M, B, H, T))] + [np.zeros_like(q) for _ in range(3)]
    for m, bb, hh in itertools.product(range(M), range(B), range(H)):
        hv = h[m, bb, hh] if h is not None else np.zeros(T)
        o = stream_gn(q[m, bb, :, hh], k[m, bb, :, hh], v[m, bb, :, hh], g[m, bb, :, hh], hv,
                      planes[m if planes.shape[0] > 1 else 0], beta, floor, on, hl, own_gd, slice_parts)
        res[0][m, bb, :, hh], res[1][m, bb, hh] = o[0], o[1]
        for x, y in zip(res[2:], o[2:]):
            x[m, bb, :, hh] = y
    return tuple(res)


def run(q, k, v, g, planes, it, eps=1e-6, on=(), hl=False):
    """[M,B,T,H,D] arrays (bf16-valued), planes [1,L,K,D] -> out, dq, dk, dv of the same shape."""
    res = [np.zeros_like(q) for _ in range(4)]
    M, B, T, H, D = q.shape
    for m, bb, h in itertools.product(range(M), range(B), range(H)):
        o = stream(q[m, bb, :, h], k[m, bb, :, h], v[m, bb, :, h], g[m, bb, :, h], planes[0], it, eps, on, hl)
        for x, y in zip(res, o):
            x[m, bb, :, h] = y
    return tuple(res)


def relerr(a, b):
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-30))


def inputs(T=1024, H=4, shift=0.0, L=8, K=4, seed=0):
    """Unit-norm Q, K; V = normalize(N(0,1) + shift); dO N(0,1); all bf16-valued."""
    rng = np.random.default_rng(seed)
    nrm = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)  # noqa: E731
    q, k = (bf16(nrm(rng.standard_normal((1, 1, T, H, 64)))) for _ in range(2))
    v = bf16(nrm(rng.standard_normal((1, 1, T, H, 64)) + shift))
    g = bf16(rng.standard_normal((1, 1, T, H, 64)))
    planes = rng.standard_normal((1, L, K, 64)).astype(np.float32).astype(np.float64)
    return q, k, v, g, planes


def gpu_run(q, k, v, g, planes, it, eps=1e-6):
    """The bf16 HIP operator on the same (bf16-valued) inputs."""
    import torch
    from race_attention_amd.functional import race_bwd_raw, race_fwd_raw
    dev = torch.device("cuda:0")
    L, K = planes.shape[1], planes.shape[2]
    t = [torch.from_numpy(x).to(dev, torch.bfloat16) for x in (q, k, v, g)]
    pd = torch.from_numpy(planes).float().to(dev)
    out, st = race_fwd_raw(t[0], t[1], t[2], pd, L=L, K=K, causal=True, inv_temp=it, eps=eps)
    dq, dk, dv, _ = race_bwd_raw(t[0], t[1], t[2], pd, t[3], st, L=L, K=K, causal=True, inv_temp=it, eps=eps)
    torch.cuda.synchronize()
    return tuple(x.double().cpu().numpy() for x in (out, dq, dk, dv))


def table(T=1024, H=4, shifts=(0.0, 0.5), L=8, K=4, gpu=False, sets=None):
    it = 1.0 / 8.0
    rows = []
    for shift in shifts:
        q, k, v, g, planes = inputs(T, H, shift, L, K)
        exact = run(q, k, v, g, planes, it)
        for on in sets or [(x,) for x in ROUNDINGS] + [ROUNDINGS]:
            got = run(q, k, v, g, planes, it, on=on)
            rows.append((shift, "+".join(on) if len(on) > 1 else on[0],
                         [relerr(a, b) for a, b in zip(got, exact)]))
        if gpu:
            got = gpu_run(q, k, v, g, planes, it)
            rows.append((shift, "**GPU kernels**", [relerr(a, b) for a, b in zip(got, exact)]))
    return rows


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    k8 = "--k8" in sys.argv
    T = int(args[0]) if args else (512 if k8 else 1024)
    L, K = (4, 8) if k8 else (8, 4)
    sets = [("dproj",), ("xpart",), ROUNDINGS, ("xpart",) + ROUNDINGS] if k8 else None
    print(f"bf16 roundings, causal K={K} L={L} d=64, T={T}, 4 streams; max|a-b|/max|b| against the exact operator")
    print("| V mean shift | rounding | out | dq | dk | dv |")
    print("|---|---|---|---|---|---|")
    for shift, name, e in table(T=T, L=L, K=K, gpu="--gpu" in sys.argv, sets=sets):
        print(f"| {shift} | {name} | " + " | ".join(f"{x:.1e}" for x in e) + " |", flush=True)
