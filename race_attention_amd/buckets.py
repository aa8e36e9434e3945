"""Soft bucket probabilities of a RACE module's inputs, for hybrid consumers,
with the reference API of misc/arxiv_64K.py:1580-1644
(race_bucket_probs_from_qk) and misc/vit.py:3193-3262
(race_avg_bucket_probs_from_x).  The probabilities come from the HIP kernel
(race_attention_amd.functional.race_bucket_probs) with the module's own
hyperplanes and learnable temperature, and are differentiable.
"""
from __future__ import annotations

import torch

from .functional import race_bucket_probs


def _planes_and_temp(ace):
    return ace.planes(), 1.0 / ace.scale()


def race_bucket_probs_from_qk(attn, Q: torch.Tensor, K: torch.Tensor):
    """(probsQ, probsK), each [M,B,H,T,L,R], for Q, K [B,T,H,dk] with
    attn.ace's hyperplanes and temperature, the M estimators an expand of
    the inputs (misc/arxiv_64K.py:1580-1644)."""
    ace = attn.ace
    M = attn.M
    planes, it = _planes_and_temp(ace)
    pack = lambda z: z.unsqueeze(0).expand(M, -1, -1, -1, -1)  # noqa: E731
    pQ = race_bucket_probs(pack(Q), planes, L=ace.L, K=ace.K, inv_temp=it)
    pK = race_bucket_probs(pack(K), planes, L=ace.L, K=ace.K, inv_temp=it)
    return pQ, pK


def race_avg_bucket_probs_from_x(race_attn, x: torch.Tensor):
    """(probsQ_S_avg, probsK_S_avg), each [B,H,T,S] (S = L*R), averaged over
    the M estimators, from x [B,T,d] through race_attn's q_proj / k_proj
    (misc/vit.py:3193-3262)."""
    B, T, _ = x.shape
    H, dk = race_attn.H, race_attn.d_k
    Q = race_attn.q_proj(x).view(B, T, H, dk)
    K = race_attn.k_proj(x).view(B, T, H, dk)
    pQ, pK = race_bucket_probs_from_qk(race_attn, Q, K)
    M, B_, H_, T_, L, R = pQ.shape
    return pQ.reshape(M, B, H, T, L * R).mean(dim=0), pK.reshape(M, B, H, T, L * R).mean(dim=0)
