"""Torch restatement, in fp64 on the CPU, of the reference's padded-batch and
denominator-proxy RACE modules (misc/classification.py:520-683,
misc/vit.py:1441-1543) for the module-level GPU tests.  Test infrastructure
only."""
import torch
import torch.nn.functional as F


def ace_with_denom(Khf, Vhf, Qhf, planes_T, protos_T, logit_temp, mask=None, eps=1e-6, keep=None):
    """Non-causal estimator with the padding mask on P_K, P_Q and V and the
    den proxy (misc/classification.py:543-592, :641-659).  planes_T is
    [d, L*K] (shared) or [M, d, L*K].  Returns (out [M,B,T,H,d], den
    [M,B,T,H]).  keep (a list) receives the corner logits, with retain_grad,
    for the l1 mass of the temperature gradient."""
    M, B, T, H, dk = Khf.shape
    L = planes_T.shape[-1] // protos_T.shape[0]
    Kb = protos_T.shape[0]
    S = L * protos_T.shape[1]
    scale = logit_temp.exp().clamp(1e-2, 20.0)
    N = M * B * H

    def streams(x):
        return x.permute(0, 1, 3, 2, 4).reshape(N, T, dk)

    K2, Q2, V2 = streams(Khf), streams(Qhf), streams(Vhf)
    if planes_T.dim() == 2:
        projK, projQ = K2 @ planes_T, Q2 @ planes_T
    else:
        pl = planes_T.repeat_interleave(B * H, dim=0)            # [N, d, L*K]
        projK, projQ = torch.bmm(K2, pl), torch.bmm(Q2, pl)
    logK = projK.view(N, T, L, Kb).tanh().div(scale) @ protos_T
    logQ = projQ.view(N, T, L, Kb).tanh().div(scale) @ protos_T
    if keep is not None:
        for z in (logK, logQ):
            z.retain_grad()
            keep.append(z)
    probsK = F.softmax(logK, dim=-1).reshape(N, T, S)
    probsQ = F.softmax(logQ, dim=-1).reshape(N, T, S)
    if mask is not None:
        mN = mask.double()[None, :, None, :].expand(M, B, H, T).reshape(N, T, 1)
        probsK, probsQ, V2 = probsK * mN, probsQ * mN, V2 * mN
    num = probsK.transpose(1, 2).bmm(V2)
    den_s = probsK.sum(dim=1)
    out = probsQ.bmm(num / (den_s.unsqueeze(-1) + eps))
    d2 = torch.einsum("nts,ns->nt", probsQ, den_s).clamp_min(eps)
    return (out.view(M, B, H, T, dk).permute(0, 1, 3, 2, 4), d2.view(M, B, H, T).permute(0, 1, 3, 2))


def leaves_of(mod, x):
    leaves = {n: p.detach().double().cpu().clone().requires_grad_(True) for n, p in mod.named_parameters()}
    leaves["x"] = x.detach().double().cpu().clone().requires_grad_(True)
    return leaves


def classification_with_denom(mod, x, mask=None):
    """misc/classification.py:628-683 (RACEAttentionWithDenom.forward), dropout off."""
    L_ = leaves_of(mod, x)
    xx = L_["x"]
    B, T, _ = xx.shape
    h, dk, M = mod.h, mod.dk, mod.M

    def lin(name, z):
        return F.linear(z, L_[name + ".weight"], L_.get(name + ".bias"))

    Q, K, V = [lin(nm, xx).view(B, T, h, dk) for nm in ("q", "k", "v")]
    if mask is not None:
        m = mask.double()[:, :, None, None]
        Q, K, V = Q * m, K * m, V * m
    pack = lambda z: z.unsqueeze(0).expand(M, -1, -1, -1, -1)  # noqa: E731
    L_["_logits"] = []
    out_m, den_m = ace_with_denom(pack(K), pack(V), pack(Q), mod.ace.planes_T.double().cpu(),
                                  mod.ace.protos_T.double().cpu(), L_["ace.logit_temp"], mask=mask, keep=L_["_logits"])
    out = lin("o", out_m.mean(dim=0).contiguous().view(B, T, h * dk))
    d_tok = den_m.mean(dim=0).mean(dim=-1, keepdim=True).clamp_min(1e-6)
    if mask is not None:
        out = out * mask.double().unsqueeze(-1)
    return out, d_tok, L_


def vit_with_denom(mod, x):
    """misc/vit.py:1511-1543 (RACEAttentionWithDenom.forward), dropout off,
    with the reference's head merge."""
    L_ = leaves_of(mod, x)
    xx = L_["x"]
    B, T, _ = xx.shape
    H, dk, M = mod.H, mod.d_k, mod.M

    def lin(name, z):
        return F.linear(z, L_[name + ".weight"], L_.get(name + ".bias"))

    Q, K, V = [lin(nm, xx).view(B, T, H, dk) for nm in ("q_proj", "k_proj", "v_proj")]
    pack = lambda z: z.unsqueeze(0).expand(M, -1, -1, -1, -1)  # noqa: E731
    L_["_logits"] = []
    out_m, den_m = ace_with_denom(pack(K), pack(V), pack(Q), mod.ace.planes_T.double().cpu(),
                                  mod.ace.protos_T.double().cpu(), L_["ace.logit_temp"], keep=L_["_logits"])
    out = lin("out", out_m.mean(dim=0).permute(0, 2, 1, 3).reshape(B, T, H * dk))
    d_tok = den_m.mean(dim=0).mean(dim=-1, keepdim=True).clamp_min(1e-6)
    return out, d_tok, L_


def temp_grad_l1(leaves):
    """l1 mass of d logit_temp's terms: d logit_temp = -sum(dlogits * logits)
    over the K and Q corner logits (logits scale as 1/temperature)."""
    return float(sum((z.grad * z.detach()).abs().sum() for z in leaves["_logits"]))
