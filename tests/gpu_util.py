"""Helpers for the GPU parity tests: device inputs, the two checks, reporting.

Every fused output is checked twice:
  * against the float64 oracle on sampled (batch, head) slices and sampled query rows
    (rows are independent, so the oracle can evaluate any subset exactly);
  * element by element against the reference's fp32 PyTorch formula on the GPU,
    head-chunked under 2 GiB as the reference harness does, with the reference's
    mixed tolerance |out - ref| <= 2e-2 + 2e-2 |ref| and max-abs <= 2e-2.
"""

import sys

import numpy as np
import torch

from oracle import attention_oracle as orc
from oracle import cpu_reference

ATOL = 2e-2
RTOL = 2e-2
MAX_ABS = 2e-2


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype).contiguous()


def compare_full(out, ref):
    """(max_abs, tol_ratio) of out vs ref; both must pass."""
    out = out.float()
    assert torch.isfinite(out).all(), "non-finite values in the fused output"
    err = (out - ref).abs()
    return float(err.max()), float((err / (ATOL + RTOL * ref.abs())).max())


def head_samples(B, H):
    picks = {(0, 0), (B - 1, H - 1), (B // 2, H // 2)}
    return sorted(picks)


def check_forward(out, q, k, v, rows_count=40, label=""):
    """Assert out (GPU) matches the oracle on sampled rows and the fp32 reference everywhere."""
    B, H, N, D = q.shape
    g = H // k.shape[1]
    ref = cpu_reference.reference_chunked(q, k, v)
    max_abs, ratio = compare_full(out, ref)
    del ref
    rows = orc.sample_rows(N, count=rows_count)
    worst = 0.0
    for b, h in head_samples(B, H):
        hk = h // g
        qs = q[b:b + 1, h:h + 1].double().cpu().numpy()
        ks = k[b:b + 1, hk:hk + 1].double().cpu().numpy()
        vs = v[b:b + 1, hk:hk + 1].double().cpu().numpy()
        want = orc.forward(qs, ks, vs, rows)
        got = out[b:b + 1, h:h + 1, rows].double().cpu().numpy()
        worst = max(worst, float(np.abs(got - want).max()))
    log(f"{label} max_abs={max_abs:.3e} tol_ratio={ratio:.3f} oracle_rows_max_abs={worst:.3e}")
    assert max_abs <= MAX_ABS and ratio <= 1.0, (label, max_abs, ratio)
    assert worst <= MAX_ABS, (label, worst)
    return max_abs, ratio, worst
