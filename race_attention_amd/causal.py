"""Globally normalised causal RACE attention ("F2") with the reference API of
misc/elsaa_causal_complete.py.

Drop-in replacement for CausalRACEAttention (misc/elsaa_causal_complete.py:438-586)
and its Triton autograd Function (:384-436): same constructor arguments,
buffer names (planes [L, K, d_k] and corners, both non-persistent), parameter
log_beta, ``last_den`` and forward(x, mask=None, return_den=False).  The
attention core -- probabilities, causal aggregation over all tables and the
per-token normalisation out = num / max(den, 1e-6) -- runs in the HIP library
(race_attention_amd.functional.race_attention_global).

Differences from the reference, all outside the results:
  * chunk_size and chunk_group_size are accepted and kept as attributes, but
    the kernels tile the sequence themselves, so any T works without padding;
  * the reference's PyTorch fallback (taken when T is not a multiple of
    chunk_size) clamps den / L instead of den at 1e-6; this module always
    follows its Triton path (den summed over the L tables, then clamped),
    which differs only where den < L * 1e-6.
"""
from __future__ import annotations

import itertools

import torch
from torch import nn

from .functional import race_attention_global


class CausalRACEAttention(nn.Module):
    """Causal RACE attention with one normaliser per token.

    x [B, T, d] -> [B, T, d].  Per head, with phi(x) = softmax over the 2^K
    corners of beta * (tanh(x planes^T) . corners) per table and
    beta = exp(log_beta).clamp(1e-2, 20):
        out_t = sum_{tau <= t} <phiQ_t, phiK_tau> v_tau / max(sum_{tau <= t} <phiQ_t, phiK_tau>, 1e-6)
    (inner products summed over the L tables).  ``mask`` [B, T] zeroes the
    keys and values of padded tokens before hashing and the outputs after the
    projection, as the reference does (:531-534, :571-572)."""

    def __init__(self, d, h, drop, num_bits=4, num_tables=4, beta_init=1.0,
                 chunk_size=256, qkv_bias=False, device="cpu", chunk_group_size=64):
        super().__init__()
        assert d % h == 0
        self.h = h
        self.dk = d // h
        self.num_bits = num_bits
        self.num_tables = num_tables
        self.R = 1 << num_bits
        self.C = chunk_size
        self.chunk_group_size = chunk_group_size
        self.q = nn.Linear(d, d, bias=qkv_bias)
        self.k = nn.Linear(d, d, bias=qkv_bias)
        self.v = nn.Linear(d, d, bias=qkv_bias)
        self.o = nn.Linear(d, d)
        self.drop = nn.Dropout(drop)
        self.register_buffer('planes', torch.randn(num_tables, num_bits, self.dk, device=device), persistent=False)
        corners = torch.tensor(list(itertools.product([-1.0, 1.0], repeat=num_bits)), device=device,
                               dtype=torch.float32)
        self.register_buffer('corners', corners, persistent=False)
        self.log_beta = nn.Parameter(torch.log(torch.tensor(beta_init, dtype=torch.float32)))
        self.last_den = None

    def beta(self) -> torch.Tensor:
        return self.log_beta.exp().clamp(1e-2, 20.0)

    def forward(self, x, mask=None, return_den=False):
        B, T, _ = x.shape
        H, dk, L = self.h, self.dk, self.num_tables
        # [B, T, H, dk] views of the projections: the operator reads them with
        # their strides (no [B, H, T, dk] copies)
        Q = self.q(x).view(B, T, H, dk)
        K = self.k(x).view(B, T, H, dk)
        V = self.v(x).view(B, T, H, dk)
        if mask is not None:
            keep = mask[:, :, None, None].to(Q.dtype)
            K = K * keep
            V = V * keep
        out_h, den = race_attention_global(Q.unsqueeze(0), K.unsqueeze(0), V.unsqueeze(0), self.planes,
                                           L=L, K=self.num_bits, beta=self.beta())
        out = out_h[0].reshape(B, T, H * dk)          # heads concatenated per token
        out = self.drop(self.o(out))
        if mask is not None:
            out = out * mask.unsqueeze(-1).to(out.dtype)
        d_token = (den[0].mean(dim=1) / L).unsqueeze(-1).clamp_min(1e-6)   # [B, T, 1]
        self.last_den = d_token.detach()
        return (out, d_token) if return_den else out
