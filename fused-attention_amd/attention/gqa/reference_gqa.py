"""PyTorch fp32 causal GQA/MQA attention: the GQA CLI's `reference` backend.

Same formula as attention/gqa/reference_gqa.py:15-47 of the reference: each
K/V head is repeated H // H_kv times along the head axis so query head h uses
K/V head h // (H // H_kv), then softmax(Q K^T / sqrt(D) + causal) V in fp32.
"""

import torch.nn.functional as F

from attention.fused.reference import reference_attention_explicit


def _group_size(num_q_heads, k, v):
    """Query heads per K/V head.  K and V must agree on their head count and it must divide H;
    the two error messages are the GQA CLI's user-visible contract (kept word for word)."""
    H_kv = k.shape[1]
    if v.shape[1] != H_kv:
        raise ValueError(f"K/V head count mismatch: K={H_kv}, V={v.shape[1]}")
    if H_kv < 1 or num_q_heads % H_kv != 0:
        raise ValueError(f"H={num_q_heads} not divisible by H_kv={H_kv}")
    return num_q_heads // H_kv


def _per_query_head(x, group):
    """[B, H_kv, N, D] -> [B, H_kv * group, N, D] where head h is K/V head h // group."""
    return x if group == 1 else x.repeat_interleave(group, dim=1)


def _expand_kv(k32, v32, num_q_heads):
    group = _group_size(num_q_heads, k32, v32)
    return _per_query_head(k32, group), _per_query_head(v32, group)


def reference_gqa_attention(q, k, v):
    q32, k32, v32 = q.float(), k.float(), v.float()
    k32, v32 = _expand_kv(k32, v32, q32.shape[1])
    return F.scaled_dot_product_attention(q32, k32, v32, is_causal=True)


def reference_gqa_attention_explicit(q, k, v):
    q32, k32, v32 = q.float(), k.float(), v.float()
    k32, v32 = _expand_kv(k32, v32, q32.shape[1])
    return reference_attention_explicit(q32, k32, v32)


# name used by run_attention_gqa.py (reference attention/gqa/reference_gqa.py:47)
causal_attention_reference_gqa = reference_gqa_attention_explicit
