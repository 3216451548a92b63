"""Unfused causal GQA/MQA baseline (the GQA CLI's `unfused` backend).

The reference's attention/gqa/unfused_gqa.py:99-128 as PyTorch-ROCm eager ops:
K/V heads are repeated across their query group, then the three unfused steps
of attention/fused/unfused.py run unchanged.
"""

from attention.fused.unfused import _unfused


def unfused_gqa_attention(q, k, v, tile_m=64, tile_n=64, return_intermediates=False):
    B, H, N, D = q.shape
    H_kv = k.shape[1]
    if tuple(k.shape) != (B, H_kv, N, D) or v.shape != k.shape or H % H_kv != 0:
        raise ValueError(f"GQA needs K, V of shape [B, H_kv, N, D] with H_kv dividing H; got "
                         f"Q {tuple(q.shape)}, K {tuple(k.shape)}, V {tuple(v.shape)}")
    group = H // H_kv
    if group > 1:
        k = k.repeat_interleave(group, dim=1)
        v = v.repeat_interleave(group, dim=1)
    return _unfused(q, k, v, tile_m, tile_n, return_intermediates)
