"""Unfused causal attention baseline (the CLI's `unfused` backend).

Same three steps and precisions as the reference's unfused baseline
(attention/fused/unfused.py:1-17, :92-116), run as PyTorch-ROCm eager ops:
  1. S = causal_mask(Q K^T * scale)   fp32, materialised as B*H*N*N
  2. P = row_softmax(S)               rounded to the input dtype, materialised
  3. O = P V                          fp32 accumulation, cast to the input dtype
It is a comparison baseline, not a hot path: it allocates the full S and P.
tile_m / tile_n are accepted for the backend signature and unused (eager ops
have no tiles), so any N works, like the fused backends.
"""

import math

import torch


def _unfused(q, k, v, tile_m, tile_n, return_intermediates):
    B, H, N, D = q.shape
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    scale = 1.0 / math.sqrt(D)
    S = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * scale
    future = torch.triu(torch.ones(N, N, dtype=torch.bool, device=q.device), diagonal=1)
    S.masked_fill_(future, float("-inf"))
    P = torch.softmax(S, dim=-1).to(q.dtype)
    O = torch.matmul(P.float(), v.float()).to(q.dtype)
    if return_intermediates:
        return O, S, P
    return O


def unfused_attention(q, k, v, tile_m=64, tile_n=64, return_intermediates=False):
    return _unfused(q, k, v, tile_m, tile_n, return_intermediates)
