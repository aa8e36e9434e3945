"""Non-causal RACE modules with the reference API of misc/vit.py.

Drop-in replacements for misc/vit.py's BatchedACE (:888-979), RACEAttention
(:994-1039), RACEAttentionWithDenom (:1441-1543), RACEBlock (:1040-1068),
PatchEmbedding (:247-256) and VisionTransformer with RACE blocks
(:4918-4982): same arguments, buffer/parameter names
(planes_T, protos_T, logit_temp) and shapes; the attention core runs in the
HIP library.  The learnable temperature is exp(logit_temp) clamped to
[1e-2, temp_max] (temp_max 20 as misc/vit.py:923; the notebooks, misc/mlm.py
and scaling/benchmark_time.py use 10).
"""
from __future__ import annotations

import torch
from torch import nn

from .functional import race_attention, race_attention_ex
from .race import _corner_protos, merge_heads, planes_from_T


class BatchedACE(nn.Module):
    """Non-causal BatchedACE (misc/vit.py:888-979); inputs [M,B,T,H,d_k] in
    K, V, Q order; output [M,B,T,H,d_k]."""

    def __init__(self, d_k, K, L, M, device='cpu', share_planes: bool = False, temp_max: float = 20.0):
        super().__init__()
        self.d_k, self.K, self.L, self.M = d_k, K, L, M
        self.R = 1 << K
        self.share_planes = share_planes
        self.temp_max = temp_max
        if share_planes:
            planes = torch.randn(L, K, d_k, device=device)
            self.register_buffer('planes_T', planes.view(L * K, d_k).T)
        else:
            planes = torch.randn(M, L, K, d_k, device=device)
            self.register_buffer('planes_T', planes.view(M, L * K, d_k).transpose(1, 2))
        self.register_buffer('protos_T', _corner_protos(K, device))
        self.logit_temp = nn.Parameter(torch.log(torch.tensor(1.0)))

    def planes(self) -> torch.Tensor:
        return planes_from_T(self.planes_T, self.L, self.K)

    def scale(self) -> torch.Tensor:
        return self.logit_temp.exp().clamp(1e-2, self.temp_max)

    def forward(self, Khf, Vhf, Qhf, eps: float = 1e-6):
        M, B, T, H, dk = Khf.shape
        assert M == self.M and dk == self.d_k
        inv_temp = 1.0 / self.scale()
        return race_attention(Qhf, Khf, Vhf, self.planes(), L=self.L, K=self.K, causal=False,
                              inv_temp=inv_temp, eps=eps)


class RACEAttention(nn.Module):
    """Multi-head non-causal RACE attention (misc/vit.py:994-1039)."""

    def __init__(self, d_in, d_out, dropout, num_heads, L, K, N_M, qkv_bias=False, device='cpu',
                 reference_head_merge=True):
        super().__init__()
        assert d_in % num_heads == 0
        self.H = num_heads
        self.d_k = d_in // num_heads
        self.M = N_M
        self.L = L
        self.P = K
        self.q_proj = nn.Linear(d_in, d_in, bias=qkv_bias)
        self.k_proj = nn.Linear(d_in, d_in, bias=qkv_bias)
        self.v_proj = nn.Linear(d_in, d_in, bias=qkv_bias)
        self.out = nn.Linear(d_in, d_out)
        self.drop = nn.Dropout(dropout)
        self.ace = BatchedACE(self.d_k, K, L, N_M, device=device)
        self.reference_head_merge = reference_head_merge

    def forward(self, x):
        B, T, _ = x.shape
        H, d_k, M = self.H, self.d_k, self.M
        Q = self.q_proj(x).view(B, T, H, d_k)
        K = self.k_proj(x).view(B, T, H, d_k)
        V = self.v_proj(x).view(B, T, H, d_k)
        pack = lambda z: z.unsqueeze(0).expand(M, -1, -1, -1, -1)  # noqa: E731
        out_hm = self.ace(pack(K), pack(V), pack(Q))
        return self.drop(self.out(merge_heads(out_hm, self.reference_head_merge)))


class RACEAttentionWithDenom(RACEAttention):
    """RACEAttention that also returns the denominator proxy
    (misc/vit.py:1441-1543): forward(x) -> (out [B,T,d_out], d_race_token
    [B,T,1]), d_race(i) = mean over M and heads of sum_s P_Q(i,s) A(s),
    each clamped at eps, then at 1e-6."""

    def _ace_with_denom(self, Khf, Vhf, Qhf, eps: float = 1e-6):
        """(out [M,B,T,H,d_k], den [M,B,T,H]) (misc/vit.py:1452-1510)."""
        ace = self.ace
        out, den = race_attention_ex(Qhf, Khf, Vhf, ace.planes(), L=ace.L, K=ace.K, inv_temp=1.0 / ace.scale(),
                                     with_den=True, eps=eps)
        return out, den.clamp_min(eps).permute(0, 1, 3, 2)

    def forward(self, x):
        B, T, _ = x.shape
        H, d_k, M = self.H, self.d_k, self.M
        Q = self.q_proj(x).view(B, T, H, d_k)
        K = self.k_proj(x).view(B, T, H, d_k)
        V = self.v_proj(x).view(B, T, H, d_k)
        pack = lambda z: z.unsqueeze(0).expand(M, -1, -1, -1, -1)  # noqa: E731
        out_m, den_m = self._ace_with_denom(pack(K), pack(V), pack(Q))
        out = merge_heads(out_m, self.reference_head_merge)
        d_race_token = den_m.mean(dim=0).mean(dim=-1, keepdim=True).clamp_min(1e-6)
        return self.drop(self.out(out)), d_race_token


class RACEBlock(nn.Module):
    """Pre-norm encoder block with non-causal RACE attention (misc/vit.py:1040-1068).
    cfg keys: embed_dim, drop_rate, num_heads, qkv_bias, L, K, M."""

    def __init__(self, cfg, device='cpu'):
        super().__init__()
        self.att = RACEAttention(d_in=cfg["embed_dim"], d_out=cfg["embed_dim"], dropout=cfg["drop_rate"],
                                 num_heads=cfg["num_heads"], qkv_bias=cfg["qkv_bias"], L=cfg["L"], K=cfg["K"],
                                 N_M=cfg["M"], device=device,
                                 reference_head_merge=cfg.get("reference_head_merge", True))
        self.norm1 = nn.LayerNorm(cfg["embed_dim"])
        self.norm2 = nn.LayerNorm(cfg["embed_dim"])
        self.ff = nn.Sequential(nn.Linear(cfg["embed_dim"], 4 * cfg["embed_dim"]), nn.GELU(),
                                nn.Linear(4 * cfg["embed_dim"], cfg["embed_dim"]))
        self.drop = nn.Dropout(cfg["drop_rate"])

    def forward(self, x):
        h = x
        x = self.att(self.norm1(x))
        x = self.drop(x) + h
        h = x
        x = self.ff(self.norm2(x))
        return self.drop(x) + h


class PatchEmbedding(nn.Module):
    """Non-overlapping patches -> tokens (misc/vit.py:247-256): [B,C,H,W] -> [B,N,d]."""

    def __init__(self, cfg):
        super().__init__()
        self.patch_embed = nn.Conv2d(cfg["num_channels"], cfg["embed_dim"], kernel_size=cfg["patch_size"],
                                     stride=cfg["patch_size"])

    def forward(self, x):
        return self.patch_embed(x).flatten(2).transpose(1, 2)


class VisionTransformer(nn.Module):
    """ViT with non-causal RACE blocks (misc/vit.py:4918-4982, attn_type "race"):
    patch embedding, CLS token, learned positions, cfg["transformer_units"]
    RACEBlocks, LayerNorm + Linear head on the CLS token.  cfg keys as the
    reference's VISION_CONFIG: img_size, patch_size, num_channels, embed_dim,
    num_heads, transformer_units, drop_rate, qkv_bias, K, L, M, num_classes."""

    def __init__(self, cfg, attn_type="race", device='cpu'):
        super().__init__()
        if attn_type != "race":
            raise ValueError("this build implements the RACE blocks only (attn_type='race')")
        self.patch_embedding = PatchEmbedding(cfg)
        G = cfg["img_size"] // cfg["patch_size"]
        assert G * cfg["patch_size"] == cfg["img_size"], "img_size must be divisible by patch_size"
        d = cfg["embed_dim"]
        self.cls_token = nn.Parameter(torch.zeros(1, 1, d))
        self.pos_embed = nn.Parameter(torch.zeros(1, G * G + 1, d))
        nn.init.trunc_normal_(self.cls_token, std=0.02)
        nn.init.trunc_normal_(self.pos_embed, std=0.02)
        self.transformer_layers = nn.Sequential(*[RACEBlock(cfg, device) for _ in range(cfg["transformer_units"])])
        self.mlp_head = nn.Sequential(nn.LayerNorm(d), nn.Linear(d, cfg["num_classes"]))

    def forward(self, x):
        x = self.patch_embedding(x)
        B = x.shape[0]
        x = torch.cat([self.cls_token.expand(B, -1, -1), x], dim=1)
        x = x + self.pos_embed[:, :x.size(1), :]
        x = self.transformer_layers(x)
        return self.mlp_head(x[:, 0])

