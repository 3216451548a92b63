"""Fused causal attention with a recompute backward and autograd, on MI355X.

Drop-in for attention/backward/fused_backward.py:151-206 of the reference.

Forward  = the fused forward kernel with the LSE output switched on: it writes
           lse = m + log2(l) (base-2 log-sum-exp of the scores pre-multiplied by
           log2(e)/sqrt(D)) directly, where the reference stores m and l and adds
           them with a torch op (:61-62, :169).
Backward = two atomic-free kernels on the same stream:
  dQ kernel:    one workgroup per query tile; loops over the visible key tiles;
                dQ = scale * dS K.  Forms Delta = rowsum(dO * O) from the O and dO
                rows it holds in registers (the reference runs it as a separate torch
                op, :175) and leaves each row's -LSE/c and -Delta in a small workspace.
  dK/dV kernel: one workgroup per key tile; loops over the query tiles that see it,
                recomputing P from the LSE; dV = P^T dO, dK = scale * dS^T Q, reading
                the per-row terms instead of forming Delta in every key tile.
  with dS = P * (dP - Delta) and dP = dO V^T.  (The C entry fa_bwd keeps the
  reference's order with no workspace: a row pass writes the same per-row terms
  into dQ's buffer, dK/dV reads them, then dQ runs; the results are the same.)

Shapes: q, k, v are (B, H, N, D) float16 or bfloat16, any N (a partial last tile
is masked), tiles 64 or 128.
Use:    o = fused_attention_autograd(q, k, v, tile_m=64, tile_n=64); o.backward(do)
"""

import torch

from attention import _lib

_DTYPES = (torch.float16, torch.bfloat16)


def _check(q, k, v, tile_m, tile_n):
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k, v must all be float16 or all be bfloat16")
    if q.shape != k.shape or q.shape != v.shape or q.dim() != 4:
        raise ValueError(f"q, k, v must all be (B, H, N, D); got {q.shape}, {k.shape}, {v.shape}")
    _lib.check_tiles(tile_m, tile_n)


def _forward(q, k, v, tile_m, tile_n):
    """Returns (o, lse) with lse [B, H, N] float32 in the reference's base-2 units."""
    B, H, N, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    _lib.fwd(q, k, v, o, lse, tile_m, tile_n)
    return o, lse


def _backward(q, k, v, o, lse, do, tile_m, tile_n):
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    _lib.bwd(q, k, v, o, do, lse, dq, dk, dv, tile_m, tile_n)
    return dq, dk, dv


class FusedAttentionFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, tile_m=64, tile_n=64):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        _check(q, k, v, tile_m, tile_n)
        o, lse = _forward(q, k, v, tile_m, tile_n)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.tiles = (tile_m, tile_n)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _backward(q, k, v, o, lse, do.contiguous().to(q.dtype), *ctx.tiles)
        return dq, dk, dv, None, None


def fused_attention_autograd(q, k, v, tile_m=64, tile_n=64):
    """Causal attention (B, H, N, D) float16/bfloat16 with autograd support.

    The checks of FusedAttentionFn, then the same forward and backward as a C++ autograd node
    (csrc/fa_autograd.cpp): results bitwise equal to FusedAttentionFn.apply, without Python in
    the backward (the host path is what bounds short sequences)."""
    _check(q, k, v, tile_m, tile_n)
    _lib._require_device(q, k, v)
    return _lib.autograd().fused_attention(q, k, v, int(tile_m), int(tile_n))
