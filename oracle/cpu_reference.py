"""The reference's PyTorch fp32 path on the CPU -- TEST INFRASTRUCTURE ONLY (CPU baseline).

Restates the reference's ground truth as it runs in its harness:
reference_attention_explicit (attention/fused/reference.py:16-23), head-chunked so the
N x N fp32 scores of one chunk stay under 2 GiB (tests/fused/run_correctness.py:36,57-67),
and fp32 autograd of the same formula for the backward
(tests/backward/run_correctness_backward.py:25-44).  bench.py times these on the
host cores as the reported CPU baseline.
"""

import math

import torch

REFERENCE_BUDGET_BYTES = 2 * 1024**3


def reference_attention_explicit(q, k, v):
    q32, k32, v32 = q.float(), k.float(), v.float()
    if k32.shape[1] != q32.shape[1]:
        g = q32.shape[1] // k32.shape[1]
        k32, v32 = k32.repeat_interleave(g, dim=1), v32.repeat_interleave(g, dim=1)
    N, D = q32.shape[-2], q32.shape[-1]
    S = (q32 @ k32.transpose(-1, -2).contiguous()) / math.sqrt(D)
    future = torch.triu(torch.ones(N, N, dtype=torch.bool, device=q.device), diagonal=1)
    S = S.masked_fill(future, float("-inf"))
    P = torch.softmax(S, dim=-1)
    return P @ v32


def reference_chunked(q, k, v):
    """Run the fp32 reference over head chunks within the 2 GiB score budget."""
    B, H, N, _ = q.shape
    g = H // k.shape[1]
    per_head = N * N * 4 * 2
    chunk = max(1, min(H, REFERENCE_BUDGET_BYTES // per_head))
    chunk = max(g, chunk - chunk % g) if g > 1 else chunk  # whole GQA groups per chunk
    out = torch.empty(q.shape[:3] + (v.shape[3],), dtype=torch.float32, device=q.device)
    for b in range(B):
        for h0 in range(0, H, chunk):
            hk0, hk1 = h0 // g, (min(H, h0 + chunk) + g - 1) // g
            out[b:b + 1, h0:h0 + chunk] = reference_attention_explicit(
                q[b:b + 1, h0:h0 + chunk], k[b:b + 1, hk0:hk1], v[b:b + 1, hk0:hk1])
    return out


def reference_grads(q, k, v, do):
    """(O, dQ, dK, dV) from fp32 autograd of the explicit formula (MHA)."""
    q, k, v = (t.detach().float().clone().requires_grad_(True) for t in (q, k, v))
    o = reference_attention_explicit(q, k, v)
    o.backward(do.float())
    return o.detach(), q.grad, k.grad, v.grad


def reference_grads_gqa(q, k, v, do):
    """(O, dQ, dK, dV) from fp32 autograd of the explicit formula on K/V repeated to the
    query heads (attention/gqa/reference_gqa.py:15-26): autograd of repeat_interleave sums
    each group's gradients onto its K/V head."""
    q, k, v = (t.detach().float().clone().requires_grad_(True) for t in (q, k, v))
    g = q.shape[1] // k.shape[1]
    o = reference_attention_explicit(q, k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1))
    o.backward(do.float())
    return o.detach(), q.grad, k.grad, v.grad
