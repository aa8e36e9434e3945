"""The reference's CPU execution path for causal RACE, composed around the
reference kernel compiled from source (oracle/_ref/race_pref*.so).

TEST INFRASTRUCTURE ONLY (tests/ and bench.py's cpu_baseline leg).

This is the causal BatchedACE.forward of misc/race.py:63-141 with its
CPU-kernel branch enabled (the commented block misc/race.py:114-133): aten
projection + soft hash on the CPU, the flat prefix mean through the reference
extension (autograd Function as misc/race.py:9-24), and the bmm readout.  It
runs on the host cores in float32 exactly as the reference would, and serves
as the "reference" kind of CPU baseline.
"""
from __future__ import annotations

import itertools
import math

import torch
import torch.nn.functional as F

from . import race_oracle


class _PrefixMeanFlat(torch.autograd.Function):
    """misc/race.py:9-24 around the compiled reference kernel."""

    @staticmethod
    def forward(ctx, probsK_flat, V_flat, eps, ext):
        E_flat = ext.race_prefix_mean_flat(probsK_flat, V_flat, float(eps))
        ctx.save_for_backward(probsK_flat, V_flat)
        ctx.eps = float(eps)
        ctx.ext = ext
        return E_flat

    @staticmethod
    def backward(ctx, gradE_flat):
        probsK_flat, V_flat = ctx.saved_tensors
        gW, gV = ctx.ext.race_prefix_mean_flat_bw(probsK_flat, V_flat,
                                                   gradE_flat.contiguous(), ctx.eps)
        return gW, gV, None, None


def protos_T(K: int) -> torch.Tensor:
    """[K, R] corner prototypes, misc/race.py:54-58."""
    corners = torch.tensor(list(itertools.product([-1., +1.], repeat=K)))
    return corners.T.contiguous()


def causal_forward(Khf, Vhf, Qhf, planes_T, K: int, L: int, eps: float = 1e-6, scale=None, ext=None):
    """Causal F1 forward on CPU tensors [M,B,T,H,dk] with shared planes_T [dk, L*K]."""
    if ext is None:
        ext = race_oracle.ref_race_pref()
        if ext is None:
            raise RuntimeError("oracle/_ref/race_pref is not built")
    M, B, T, H, dk = Khf.shape
    R = 1 << K
    S = L * R
    if scale is None:
        scale = math.sqrt(dk)                                   # misc/race.py:67
    N = M * B * H
    Kh2 = Khf.permute(0, 1, 3, 2, 4).contiguous().view(N, T, dk)
    Qh2 = Qhf.permute(0, 1, 3, 2, 4).contiguous().view(N, T, dk)
    V2 = Vhf.permute(0, 1, 3, 2, 4).contiguous().view(N, T, dk)
    projK = (Kh2 @ planes_T).view(N, T, L, K)
    projQ = (Qh2 @ planes_T).view(N, T, L, K)
    pT = protos_T(K).to(Khf.dtype)
    probsK = F.softmax(projK.tanh().div(scale) @ pT, dim=-1)
    probsQ = F.softmax(projQ.tanh().div(scale) @ pT, dim=-1)
    probsK_flat = probsK.permute(0, 2, 3, 1).contiguous().view(N * S, T)
    V_flat = (V2.unsqueeze(2).unsqueeze(3).expand(N, T, L, R, dk)
              .permute(0, 2, 3, 1, 4).contiguous().view(N * S, T, dk))
    E_flat = _PrefixMeanFlat.apply(probsK_flat, V_flat, eps, ext)
    E_pref = E_flat.view(N, L, R, T, dk).permute(0, 3, 1, 2, 4).contiguous()
    out2 = torch.bmm(probsQ.reshape(N * T, 1, S), E_pref.view(N * T, S, dk)).view(N, T, dk)
    return out2.view(M, B, H, T, dk).permute(0, 1, 3, 2, 4)
