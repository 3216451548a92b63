"""Fused causal GQA/MQA forward on MI355X: drop-in for attention/gqa/fused_gqa.py:70-82.

    O = fused_gqa_attention(q, k, v, tile_m=64, tile_n=64)

q: [B, H, N, D]; k, v: [B, H_kv, N, D] with H_kv dividing H; query head h reads
K/V head h // (H // H_kv).  One workgroup serves up to four query heads of the
same K/V group, so each K/V tile staged in LDS is reused across those heads.
"""

import torch

from attention import _lib


def fused_gqa_attention(q, k, v, tile_m=64, tile_n=64):
    B, H, N, D = q.shape
    H_kv = k.shape[1]
    if tuple(k.shape) != (B, H_kv, N, D) or v.shape != k.shape or H % H_kv != 0:
        raise ValueError(
            f"GQA needs K, V of shape [B, H_kv, N, D] with H_kv dividing H; got Q {tuple(q.shape)}, "
            f"K {tuple(k.shape)}, V {tuple(v.shape)}")
    if N % tile_m != 0 or N % tile_n != 0:
        raise ValueError(f"N={N} must be divisible by tile_m={tile_m} and tile_n={tile_n}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share one dtype; got {q.dtype}, {k.dtype}, {v.dtype}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    o = torch.empty_like(q)
    _lib.fwd(q, k, v, o, None, tile_m, tile_n)
    return o
