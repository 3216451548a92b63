"""Seeded random shapes through the whole path: forward (MHA and GQA/MQA) against the fp32
reference and the float64 oracle, and the grouped backward against fp32 autograd.

Each case draws B, H_kv, the group size, N (any length, partial tiles included), D, the
dtype and the tiles from a fixed seed, so the dispatch choices the shapes drive (heads per
workgroup, 64-row tiles run as 128-row workgroups, the dK/dV split and the per-row terms of
the backward workspace) meet one another in combinations the structured suites do not list.
Bars as in the structured suites: forward max-abs <= 2e-2 (and the reference's mixed
tolerance), backward O/dQ max-abs <= 2e-2, dK/dV mixed tolerance 2e-2 + 2e-2 |ref|, all with
relative Frobenius error <= 2e-2.
"""

import numpy as np
import pytest
import torch

from attention.gqa.fused_gqa import fused_gqa_attention
from tests.gpu_util import check_forward, dev, log
from tests.test_gqa_bwd_gpu import check, make

pytestmark = pytest.mark.gpu

DTYPES = (torch.float16, torch.bfloat16)
TILES = ((64, 64), (64, 128), (128, 64), (128, 128))


def draw(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 4))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    N = int(rng.integers(1, 700))
    D = int(rng.choice([32, 64, 128]))
    dt = DTYPES[int(rng.integers(0, 2))]
    tiles = TILES[int(rng.integers(0, 4))]
    return B, Hkv * G, Hkv, N, D, dt, tiles


@pytest.mark.parametrize("seed", range(24))
def test_random_forward(seed):
    B, H, Hkv, N, D, dt, tiles = draw(1000 + seed)
    label = f"random fwd seed={seed} B{B} H{H} Hkv{Hkv} N{N} D{D} {str(dt)[6:]} {tiles}"
    log(label)
    q, k, v, _ = make(B, H, Hkv, N, D, dt, seed=2000 + seed)
    out = fused_gqa_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    check_forward(out, q, k, v, rows_count=min(N, 24), label=label)


@pytest.mark.parametrize("seed", range(16))
def test_random_backward(seed):
    B, H, Hkv, N, D, dt, tiles = draw(5000 + seed)
    label = f"random bwd seed={seed} B{B} H{H} Hkv{Hkv} N{N} D{D} {str(dt)[6:]} {tiles}"
    log(label)
    q, k, v, do = make(B, H, Hkv, N, D, dt, seed=6000 + seed)
    check(q, k, v, do, tiles, label)
