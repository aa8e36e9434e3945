"""Causal RACE modules with the reference API of misc/race.py.

Drop-in replacements for misc/race.py's RACEPrefixMeanFlatFn (:9-24),
BatchedACE (:26-142), RACEAttention (:144-173) and RACEBlock (:176-206).
Same constructor arguments, buffer names (planes_T, protos_T) and shapes; the
attention core runs in the HIP library (race_attention_amd.functional).
"""
from __future__ import annotations

import itertools
import math

import torch
from torch import nn

from .functional import RACEPrefixMeanFlatFn, race_attention  # noqa: F401  (re-exported)


def _corner_protos(K: int, device) -> torch.Tensor:
    """[K, R] corners of {-1,+1}^K in itertools.product order (misc/race.py:54-58)."""
    corners = torch.tensor(list(itertools.product([-1., +1.], repeat=K)), device=device)
    return corners.T.contiguous()


def planes_from_T(planes_T: torch.Tensor, L: int, K: int) -> torch.Tensor:
    """planes_T [d, L*K] or [M, d, L*K] -> [L,K,d] or [M,L,K,d] (column j = l*K + k)."""
    if planes_T.dim() == 2:
        return planes_T.T.reshape(L, K, planes_T.shape[0])
    return planes_T.transpose(1, 2).reshape(planes_T.shape[0], L, K, planes_T.shape[1])


class BatchedACE(nn.Module):
    """Causal BatchedACE (misc/race.py:26-142).

    Inputs Khf, Vhf, Qhf: [M, B, T, H, d_k] (note the K, V, Q order).  Output
    [M, B, T, H, d_k].  Temperature is sqrt(d_k) (misc/race.py:67); eps 1e-6.
    share_planes=True: one [L, K, d_k] sketch for all M (planes_T [d_k, L*K]);
    False: independent sketches (planes_T [M, d_k, L*K]).
    """

    def __init__(self, d_k, K, L, M, device='cpu', share_planes: bool = True):
        super().__init__()
        self.d_k, self.K, self.L, self.M = d_k, K, L, M
        self.R = 1 << K
        self.share_planes = share_planes
        if share_planes:
            planes = torch.randn(L, K, d_k, device=device)
            self.register_buffer('planes_T', planes.view(L * K, d_k).T)
        else:
            planes = torch.randn(M, L, K, d_k, device=device)
            self.register_buffer('planes_T', planes.view(M, L * K, d_k).transpose(1, 2))
        self.register_buffer('protos_T', _corner_protos(K, device))
        self.eps = 1e-6

    def planes(self) -> torch.Tensor:
        return planes_from_T(self.planes_T, self.L, self.K)

    def forward(self, Khf, Vhf, Qhf):
        M, B, T, H, dk = Khf.shape
        assert M == self.M and dk == self.d_k
        inv_temp = 1.0 / math.sqrt(dk)
        return race_attention(Qhf, Khf, Vhf, self.planes(), L=self.L, K=self.K, causal=True,
                              inv_temp=inv_temp, eps=self.eps)


def merge_heads(out_h: torch.Tensor, reference_head_merge: bool) -> torch.Tensor:
    """[M,B,T,H,d] -> mean over M -> [B,T,H*d].

    reference_head_merge=True reproduces the reference's
    ``.permute(0,2,1,3).contiguous().view(B,T,-1)`` on a [B,T,H,d] tensor
    (misc/race.py:172, misc/vit.py:1034-1035), which re-reads [B,H,T,d]
    memory as [B,T,H*d]; False concatenates heads per token."""
    out = out_h.mean(0) if out_h.shape[0] > 1 else out_h[0]
    B, T = out.shape[0], out.shape[1]
    if reference_head_merge:
        return out.permute(0, 2, 1, 3).contiguous().view(B, T, -1)
    return out.reshape(B, T, -1)


class RACEAttention(nn.Module):
    """Multi-head causal RACE attention (misc/race.py:144-173).

    reference_head_merge (default True) keeps the reference's head merge
    bit-for-bit; see merge_heads.  With share_planes the M estimators see the
    same inputs and sketch, so they are computed once (their mean equals each
    of them)."""

    def __init__(self, d, h, K, L, M, drop=0.1, qkv_bias=False, device='cpu', reference_head_merge=True):
        super().__init__()
        assert d % h == 0
        self.h, self.d_k, self.M = h, d // h, M
        self.q = nn.Linear(d, d, bias=qkv_bias)
        self.k = nn.Linear(d, d, bias=qkv_bias)
        self.v = nn.Linear(d, d, bias=qkv_bias)
        self.o = nn.Linear(d, d)
        self.drop = nn.Dropout(drop)
        self.ace = BatchedACE(self.d_k, K, L, M, device=device)
        self.reference_head_merge = reference_head_merge

    def forward(self, x):
        B, T, _ = x.shape
        Q = self.q(x).view(B, T, self.h, self.d_k)
        K = self.k(x).view(B, T, self.h, self.d_k)
        V = self.v(x).view(B, T, self.h, self.d_k)
        M = 1 if self.ace.share_planes else self.M
        pack = lambda z: z.unsqueeze(0).expand(M, -1, -1, -1, -1)  # noqa: E731
        if M == self.M:
            out_h = self.ace(pack(K), pack(V), pack(Q))
        else:
            out_h = race_attention(pack(Q), pack(K), pack(V), self.ace.planes(), L=self.ace.L, K=self.ace.K,
                                   causal=True, inv_temp=1.0 / math.sqrt(self.d_k), eps=self.ace.eps)
        out = merge_heads(out_h, self.reference_head_merge)
        return self.drop(self.o(out))


class RACEBlock(nn.Module):
    """Pre-norm transformer block with causal RACE attention (misc/race.py:176-206).
    cfg keys: emb_dim, n_heads, K, L, M, drop_rate, qkv_bias."""

    def __init__(self, cfg, device='cpu'):
        super().__init__()
        self.att = RACEAttention(d=cfg["emb_dim"], h=cfg["n_heads"], K=cfg["K"], L=cfg["L"], M=cfg["M"],
                                 drop=cfg["drop_rate"], qkv_bias=cfg["qkv_bias"], device=device,
                                 reference_head_merge=cfg.get("reference_head_merge", True))
        self.norm1 = nn.LayerNorm(cfg["emb_dim"])
        self.norm2 = nn.LayerNorm(cfg["emb_dim"])
        self.ff = nn.Sequential(nn.Linear(cfg["emb_dim"], 4 * cfg["emb_dim"]), nn.GELU(),
                                nn.Linear(4 * cfg["emb_dim"], cfg["emb_dim"]))
        self.drop = nn.Dropout(cfg["drop_rate"])

    def forward(self, x):
        h = x
        x = self.att(self.norm1(x))
        x = self.drop(x) + h
        h = x
        x = self.ff(self.norm2(x))
        return self.drop(x) + h
