"""Torch restatement of the reference's globally normalised causal module
(CausalRACEAttention, misc/elsaa_causal_complete.py:438-586) for tests: its
chunked PyTorch path (inter-chunk states + masked intra-chunk products), run
in fp64 on the CPU.  Test infrastructure only."""
import itertools

import torch
import torch.nn.functional as F


def phi(x, planes, beta):
    """[B,H,T,D] -> [B,H,L,T,R]: softmax over corners of beta * (tanh(proj) . c)
    (misc/elsaa_causal_complete.py:483-490)."""
    L, K, D = planes.shape
    c = torch.tensor(list(itertools.product([-1.0, 1.0], repeat=K)), dtype=x.dtype)
    th = torch.tanh(torch.einsum("bhtd,lkd->bhtlk", x, planes))
    z = beta * torch.einsum("bhtlk,rk->bhtlr", th, c)
    return torch.softmax(z, dim=-1).permute(0, 1, 3, 2, 4)


def chunked(Q, K, V, planes, beta, C):
    """The module's chunked causal path: exclusive per-chunk states for the
    inter-chunk part and a masked intra-chunk product, both averaged over L
    (misc/elsaa_causal_complete.py:508-586).  Returns (out, den_sum_over_L)."""
    B, H, T, D = Q.shape
    L = planes.shape[0]
    pQ, pK = phi(Q, planes, beta), phi(K, planes, beta)
    nums, dens = [], []
    SA = torch.zeros(B, H, L, pK.shape[-1], dtype=Q.dtype)
    SB = torch.zeros(B, H, L, pK.shape[-1], D, dtype=Q.dtype)
    for c0 in range(0, T, C):
        c1 = min(T, c0 + C)
        q_c, k_c, v_c = pQ[:, :, :, c0:c1], pK[:, :, :, c0:c1], V[:, :, c0:c1]
        inter_n = torch.einsum("bhlcr,bhlrd->bhcd", q_c, SB) / L
        inter_d = torch.einsum("bhlcr,bhlr->bhc", q_c, SA) / L
        m = torch.einsum("bhlcr,bhlsr->bhcs", q_c, k_c) / L
        m = m * torch.tril(torch.ones(c1 - c0, c1 - c0, dtype=Q.dtype))
        nums.append(inter_n + m @ v_c)
        dens.append(inter_d + m.sum(-1))
        SA = SA + k_c.sum(3)
        SB = SB + torch.einsum("bhlcr,bhcd->bhlrd", k_c, v_c)
    num, den = torch.cat(nums, 2), torch.cat(dens, 2)
    return num / den.clamp_min(1e-6)[..., None], den * L


def module_forward(mod, x, mask=None, C=16):
    """CausalRACEAttention.forward (misc/elsaa_causal_complete.py:492-586) in
    fp64 from the weights of ``mod`` (dropout off): returns (out, d_token) and
    the dict of fp64 leaf tensors (x and every parameter) for gradients."""
    leaves = {n: p.detach().double().cpu().clone().requires_grad_(True) for n, p in mod.named_parameters()}
    xx = x.detach().double().cpu().clone().requires_grad_(True)
    leaves["x"] = xx
    B, T, _ = xx.shape
    H, dk, L = mod.h, mod.dk, mod.num_tables

    def lin(name, z):
        return F.linear(z, leaves[name + ".weight"], leaves.get(name + ".bias"))

    Q, K, V = [lin(nm, xx).view(B, T, H, dk).transpose(1, 2) for nm in ("q", "k", "v")]
    if mask is not None:
        keep = mask.double().cpu()[:, None, :, None]
        K, V = K * keep, V * keep
    beta = leaves["log_beta"].exp().clamp(1e-2, 20.0)
    o, den = chunked(Q, K, V, mod.planes.detach().double().cpu(), beta, C)
    for z in (Q, K, V, o, den):
        z.retain_grad()
    out = lin("o", o.transpose(1, 2).reshape(B, T, H * dk))
    if mask is not None:
        out = out * mask.double().cpu().unsqueeze(-1)
    d_token = (den.mean(dim=1) / L).unsqueeze(-1).clamp_min(1e-6)
    # the attention core's inputs and outputs ([B,H,T,dk], den [B,H,T]):
    # after backward, o.grad and den.grad are its upstream gradients
    leaves["_core"] = (Q, K, V, o, den, float(beta.detach()))
    return out, d_token, leaves

