"""Fused causal MHA forward on MI355X: drop-in for attention/fused/fused.py:68-76.

    O = fused_attention(q, k, v, tile_m=64, tile_n=64)

q, k, v: [B, H, N, D] float16 or bfloat16 GPU tensors.  Returns O with q's
shape and dtype, enqueued on the current stream without synchronising (as the
reference's ct.launch).  tile_m / tile_n select the kernel's query rows per
workgroup and keys per LDS tile (each 64 or 128, each dividing N).
"""

import torch

from attention import _lib


def fused_attention(q, k, v, tile_m=64, tile_n=64):
    B, H, N, D = q.shape
    if N % tile_m != 0 or N % tile_n != 0:
        raise ValueError(f"N={N} must be divisible by tile_m={tile_m} and tile_n={tile_n}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must all be (B, H, N, D); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share one dtype; got {q.dtype}, {k.dtype}, {v.dtype}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    o = torch.empty_like(q)
    _lib.fwd(q, k, v, o, None, tile_m, tile_n)
    return o
