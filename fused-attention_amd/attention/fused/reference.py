"""PyTorch fp32 causal attention: the library's `reference` backend.

Same formula as the reference's ground truth (attention/fused/reference.py:12-27):
softmax(Q K^T / sqrt(D) + causal mask) V with every intermediate in fp32.  It
runs on whatever device the inputs live on, so the CLI's reference backend also
works on a machine without a GPU.
"""

import math

import torch
import torch.nn.functional as F


def reference_attention(q, k, v):
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)


def reference_attention_explicit(q, k, v):
    q32, k32, v32 = q.float(), k.float(), v.float()
    N, D = q32.shape[-2], q32.shape[-1]
    S = (q32 @ k32.transpose(-1, -2).contiguous()) / math.sqrt(D)
    future = torch.triu(torch.ones(N, N, dtype=torch.bool, device=q.device), diagonal=1)
    S = S.masked_fill(future, float("-inf"))
    P = torch.softmax(S, dim=-1)
    return P @ v32


# name used by run_attention.py and the tests (reference attention/fused/reference.py:27)
causal_attention_reference = reference_attention_explicit
