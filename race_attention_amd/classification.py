"""Padded-batch RACE modules with the reference API of misc/classification.py.

Drop-in replacements for misc/classification.py's BatchedACE (:520-592, with
the padding mask), RACEAttention (:595-626) and RACEAttentionWithDenom
(:628-683).  Same arguments, buffer/parameter names (planes_T, protos_T,
logit_temp) and shapes; the attention core runs in the HIP library
(race_attention_amd.functional.race_attention_ex).

The reference multiplies P_K, P_Q and V by the [B,T] mask (:580-585).  The
kernels take the mask as key weights on P_K; the V and P_Q factors are
elementwise on the operator's input and output (out_t = m_t (P_Q E)_t,
den_t = m_t sum_s P_Q A_s) and are applied here.
"""
from __future__ import annotations

import torch
from torch import nn

from . import vit as _vit
from .functional import race_attention_ex


def _mask_terms(mask, M, B, T, H):
    """[B,T] mask -> (fp32 [B,T] key weights, [1,B,T,1,1] factor)."""
    m = mask.to(torch.float32)
    return m, m.view(1, B, T, 1, 1)


class BatchedACE(_vit.BatchedACE):
    """Non-causal BatchedACE with a padding mask (misc/classification.py:520-592).

    forward(Khf, Vhf, Qhf, mask=None, eps=1e-6) -> [M,B,T,H,d_k]; mask [B,T]
    (1 = token, 0 = padding, or fractional weights)."""

    def __init__(self, d_k, K, L, M, device="cpu", share_planes=False):
        super().__init__(d_k, K, L, M, device=device, share_planes=share_planes)

    def forward(self, Khf, Vhf, Qhf, mask=None, eps=1e-6):
        return self.forward_with_den(Khf, Vhf, Qhf, mask=mask, eps=eps, with_den=False)

    def forward_with_den(self, Khf, Vhf, Qhf, mask=None, eps=1e-6, with_den=True):
        """(out [M,B,T,H,d_k], den [M,B,T,H]) as _ace_with_denom
        (misc/classification.py:641-659): den = (sum_s P_Q A_s).clamp_min(eps)."""
        M, B, T, H, dk = Khf.shape
        assert M == self.M and dk == self.d_k
        inv_temp = 1.0 / self.scale()
        kw = None
        if mask is not None:
            kw, f = _mask_terms(mask, M, B, T, H)
            Vhf = Vhf * f.to(Vhf.dtype)
        res = race_attention_ex(Qhf, Khf, Vhf, self.planes(), L=self.L, K=self.K, inv_temp=inv_temp, kmask=kw,
                                with_den=with_den, eps=eps)
        out, den = res if with_den else (res, None)
        if mask is not None:
            out = out * f.to(out.dtype)
            if den is not None:
                den = den * kw.view(1, B, 1, T)
        if den is None:
            return out
        return out, den.clamp_min(eps).permute(0, 1, 3, 2)


class RACEAttention(nn.Module):
    """Padded-batch multi-head RACE attention (misc/classification.py:595-626):
    forward(x, mask) with Q, K, V masked before the estimator, the masked
    estimator, the per-token head concatenation and a masked output."""

    def __init__(self, d, h, drop, M=2, K=3, L=2, qkv_bias=False, device="cpu"):
        super().__init__()
        assert d % h == 0
        self.h, self.dk, self.M = h, d // h, M
        self.q = nn.Linear(d, d, bias=qkv_bias)
        self.k = nn.Linear(d, d, bias=qkv_bias)
        self.v = nn.Linear(d, d, bias=qkv_bias)
        self.o = nn.Linear(d, d)
        self.drop = nn.Dropout(drop)
        self.ace = BatchedACE(self.dk, K, L, M, device=device)

    def _qkv(self, x, mask):
        B, T, _ = x.shape
        Q = self.q(x).view(B, T, self.h, self.dk)
        K = self.k(x).view(B, T, self.h, self.dk)
        V = self.v(x).view(B, T, self.h, self.dk)
        if mask is not None:
            m = mask[:, :, None, None].to(Q.dtype)
            Q, K, V = Q * m, K * m, V * m
        pack = lambda z: z.unsqueeze(0).expand(self.M, -1, -1, -1, -1)  # noqa: E731
        return pack(Q), pack(K), pack(V)

    def forward(self, x, mask):
        B, T, _ = x.shape
        Q, K, V = self._qkv(x, mask)
        out = self.ace(K, V, Q, mask=mask).mean(dim=0)
        out = self.drop(self.o(out.contiguous().view(B, T, self.h * self.dk)))
        if mask is not None:
            out = out * mask.unsqueeze(-1).to(out.dtype)
        return out


class RACEAttentionWithDenom(RACEAttention):
    """RACEAttention that also returns the denominator proxy
    (misc/classification.py:628-683): forward(x, mask=None) ->
    (out [B,T,d], d_race_token [B,T,1]), d_race_token = the mean over M and
    heads of (sum_s P_Q A_s).clamp_min(eps), clamped at 1e-6."""

    def forward(self, x, mask=None):
        B, T, _ = x.shape
        Q, K, V = self._qkv(x, mask)
        out_m, den_m = self.ace.forward_with_den(K, V, Q, mask=mask)
        out = self.drop(self.o(out_m.mean(dim=0).contiguous().view(B, T, self.h * self.dk)))
        d_race_token = den_m.mean(dim=0).mean(dim=-1, keepdim=True).clamp_min(1e-6)
        if mask is not None:
            out = out * mask.unsqueeze(-1).to(out.dtype)
        return out, d_race_token
