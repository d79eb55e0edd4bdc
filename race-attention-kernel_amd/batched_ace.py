"""Drop-in BatchedACE (src/race_baseline.py:21-52) running the op on MI355X.

Same constructor and forward signature as the reference module.  Lines 35-44
of the reference (permutes, shared hash planes, tanh, corner softmax) run as
torch ops, exactly as there; lines 45-51 (the cumsum/bmm hot span) are
replaced by race_fused_fwd; line 52 (permute back) is kept.
"""
from __future__ import annotations

import itertools
import math

import torch
import torch.nn.functional as F
from torch import nn

from .ops import race_fused_fwd


class BatchedACE(nn.Module):
    def __init__(self, d_k, K, L, M, device="cpu", share_planes=True, causal=True):
        super().__init__()
        assert share_planes, "reference config uses shared planes"
        self.d_k, self.K, self.L, self.M = d_k, K, L, M
        self.R = 1 << K
        self.causal = causal
        planes = torch.randn(L, K, d_k, device=device)
        self.register_buffer("planes_T", planes.view(L * K, d_k).T)  # [d_k, L*K]
        corners = torch.tensor(list(itertools.product([-1.0, 1.0], repeat=K)), device=device)
        self.register_buffer("protos_T", corners.T)  # [K, R]

    def bucket_probs(self, x2: torch.Tensor) -> torch.Tensor:
        """[N, T, d] -> [N, T, L, R] corner probabilities (reference lines 41-44)."""
        N, T, dk = x2.shape
        proj = (x2 @ self.planes_T).view(N, T, self.L, self.K)
        return F.softmax(proj.tanh().div(math.sqrt(dk)) @ self.protos_T, dim=-1)

    def forward(self, Khf, Vhf, Qhf):
        M, B, T, H, dk = Khf.shape
        N = M * B * H
        Kh2 = Khf.permute(0, 1, 3, 2, 4).contiguous().view(N, T, dk)
        Qh2 = Qhf.permute(0, 1, 3, 2, 4).contiguous().view(N, T, dk)
        V2 = Vhf.permute(0, 1, 3, 2, 4).contiguous().view(N, T, dk)
        probsK = self.bucket_probs(Kh2).contiguous()
        probsQ = self.bucket_probs(Qh2).contiguous()
        out2 = race_fused_fwd(probsQ, probsK, V2, self.causal)
        return out2.view(M, B, H, T, dk).permute(0, 1, 3, 2, 4)
