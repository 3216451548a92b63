"""Fused causal GQA/MQA forward on MI355X: drop-in for attention/gqa/fused_gqa.py:70-82.

    O = fused_gqa_attention(q, k, v, tile_m=64, tile_n=64)

q: [B, H, N, D]; k, v: [B, H_kv, N, D] with H_kv dividing H; query head h reads
K/V head h // (H // H_kv).  One workgroup serves up to four query heads of the
same K/V group, so each K/V tile staged in LDS is reused across those heads.

Beyond the reference (whose backward is MHA-only): the same attention with
autograd, whose backward runs dQ (which also leaves each row's Delta and LSE term
for the next kernel) then dK/dV (one workgroup per K/V-head key tile, summing the
group's query heads in registers, no atomics; split over several workgroups with
fp32 partial sums when the key tiles alone leave the GPU idle):

    O = fused_gqa_attention_autograd(q, k, v, tile_m=64, tile_n=64); O.backward(dO)
"""

import torch

from attention import _lib

_DTYPES = (torch.float16, torch.bfloat16)


def _check_gqa(q, k, v, tile_m, tile_n):
    B, H, N, D = q.shape
    H_kv = k.shape[1]
    if tuple(k.shape) != (B, H_kv, N, D) or v.shape != k.shape or H % H_kv != 0:
        raise ValueError(
            f"GQA needs K, V of shape [B, H_kv, N, D] with H_kv dividing H; got Q {tuple(q.shape)}, "
            f"K {tuple(k.shape)}, V {tuple(v.shape)}")
    _lib.check_tiles(tile_m, tile_n)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share one dtype; got {q.dtype}, {k.dtype}, {v.dtype}")


def fused_gqa_attention(q, k, v, tile_m=64, tile_n=64):
    _check_gqa(q, k, v, tile_m, tile_n)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    o = torch.empty_like(q)
    _lib.fwd(q, k, v, o, None, tile_m, tile_n)
    return o


class FusedGQAAttentionFn(torch.autograd.Function):
    """Forward with LSE, then the recompute backward with dK/dV summed per K/V head."""

    @staticmethod
    def forward(ctx, q, k, v, tile_m=64, tile_n=64):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        if q.dim() != 4:
            raise ValueError(f"q must be (B, H, N, D); got {tuple(q.shape)}")
        _check_gqa(q, k, v, tile_m, tile_n)
        if q.dtype not in _DTYPES:
            raise TypeError("q, k, v must all be float16 or all be bfloat16")
        B, H, N, D = q.shape
        o = torch.empty_like(q)
        lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
        _lib.fwd(q, k, v, o, lse, tile_m, tile_n)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.tiles = (tile_m, tile_n)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        _lib.bwd(q, k, v, o, do.contiguous().to(q.dtype), lse, dq, dk, dv, *ctx.tiles)
        return dq, dk, dv, None, None


def fused_gqa_attention_autograd(q, k, v, tile_m=64, tile_n=64):
    """Causal GQA/MQA attention, q (B, H, N, D), k/v (B, H_kv, N, D), with autograd.

    The checks of FusedGQAAttentionFn, then the same forward and backward as a C++ autograd
    node (csrc/fa_autograd.cpp), bitwise equal to FusedGQAAttentionFn.apply."""
    if q.dim() != 4:
        raise ValueError(f"q must be (B, H, N, D); got {tuple(q.shape)}")
    _check_gqa(q, k, v, tile_m, tile_n)
    if q.dtype not in _DTYPES:
        raise TypeError("q, k, v must all be float16 or all be bfloat16")
    _lib._require_device(q, k, v)
    return _lib.autograd().fused_attention(q, k, v, int(tile_m), int(tile_n))
