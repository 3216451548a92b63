"""GPU parity of the fused causal forward (MHA) and the forward with LSE.

Cases:
  * small shapes over every dtype x head dim x tile combination;
  * the reference's 84-case MHA suite (tests/fused/cases.py), fp16, at each tile config;
  * the full-size workload: B=4, H=32, S=4096, D=128 bf16 (tiles {64,128}^2);
  * LSE of the forward against the oracle's base-2 log-sum-exp.
"""

import math
import time

import numpy as np
import pytest
import torch

from attention.backward.fused_backward import _forward
from attention.fused.fused import fused_attention
from oracle import attention_oracle as orc
from oracle import cases
from tests.gpu_util import check_forward, dev, log, margin

LOG2E = 1.4426950408889634

pytestmark = pytest.mark.gpu

TILES = [(64, 64), (64, 128), (128, 64), (128, 128)]
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("tiles", TILES, ids=lambda t: f"{t[0]}x{t[1]}")
def test_small_shapes(dt, D, tiles):
    B, H, N = 2, 3, 384 if tiles == (128, 128) else 256
    if N % tiles[0] or N % tiles[1]:
        N = 256
    q, k, v = (dev(x, DTYPES[dt]) for x in cases.normal_inputs([(B, H, N, D)] * 3, seed=D + tiles[0]))
    log(f"small dt={dt} D={D} tiles={tiles} N={N}")
    o = fused_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    assert o.dtype == q.dtype and o.shape == q.shape
    # row 0 attends to key 0 only: O[0] == V[0] exactly
    assert torch.equal(o[:, :, 0], v[:, :, 0])
    check_forward(o, q, k, v, label=f"small {dt} D{D} {tiles}")


def test_row0_exact_and_prefix_mean_with_zero_q():
    B, H, N, D = 1, 2, 512, 64
    _, _, v = cases.normal_inputs([(B, H, N, D)] * 3, seed=3)
    vd = dev(v, torch.float16)
    q = torch.zeros_like(vd)
    k = dev(cases.normal_inputs([(B, H, N, D)], seed=4)[0], torch.float16)
    o = fused_attention(q, k, vd, 64, 64)
    torch.cuda.synchronize()
    prefix = torch.cumsum(vd.double(), dim=2) / torch.arange(1, N + 1, device="cuda").double()[:, None]
    assert float((o.double() - prefix).abs().max()) <= 2e-3


@pytest.mark.parametrize("tiles", TILES, ids=lambda t: f"{t[0]}x{t[1]}")
@pytest.mark.parametrize("case", cases.all_cases(), ids=lambda c: c.id)
def test_reference_suite_fp16(case, tiles):
    """The reference's 84 MHA cases (fp16, sigma tiny/large) at each tile config (a case whose N
    is not a multiple of a tile runs with a partial last tile, where the reference rejects it)."""
    q, k, v = (dev(x, torch.float16) for x in cases.make_inputs(case))
    log(f"suite {case.id} tiles={tiles}")
    t0 = time.perf_counter()
    o = fused_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    check_forward(o, q, k, v, rows_count=24, label=f"{case.id} {tiles}", case=case, tiles=tiles, seconds=seconds)


@pytest.mark.parametrize("case", [c for c in cases.all_cases() if c.N <= 2048][::3], ids=lambda c: c.id)
def test_reference_suite_bf16(case):
    """A third of the MHA suite with the same seeded values cast to bfloat16."""
    q, k, v = (dev(x, torch.bfloat16) for x in cases.make_inputs(case, dtype=np.float32))
    log(f"suite-bf16 {case.id}")
    o = fused_attention(q, k, v, 64, 64)
    torch.cuda.synchronize()
    check_forward(o, q, k, v, rows_count=24, label=f"bf16 {case.id}")


@pytest.mark.parametrize("tiles", TILES, ids=lambda t: f"{t[0]}x{t[1]}")
def test_full_size_bf16_B4_H32_S4096_D128(tiles):
    shape = (4, 32, 4096, 128)
    q, k, v = (dev(x, torch.bfloat16) for x in cases.normal_inputs([shape] * 3, seed=0))
    log(f"full-size MHA bf16 {shape} tiles={tiles}")
    o = fused_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    check_forward(o, q, k, v, rows_count=32, label=f"MHA {shape} {tiles}", tiles=tiles,
                  margin_test="fwd B4 H32 S4096 D128")
    # the forward that saves LSE (the training step's), every row against fp32 on the GPU
    o2, lse = _forward(q, k, v, *tiles)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    S, D = shape[2], shape[3]
    mask = torch.triu(torch.ones(S, S, device="cuda", dtype=torch.bool), 1)
    err = 0.0
    for b in range(shape[0]):
        for h in range(shape[1]):
            s = (q[b, h].float() @ k[b, h].float().t().contiguous()) / math.sqrt(D)
            s.masked_fill_(mask, float("-inf"))
            err = max(err, float((lse[b, h] - torch.logsumexp(s, -1) * LOG2E).abs().max()))
    log(f"MHA {shape} {tiles} LSE max_abs={err:.3e} (bar {LSE_ABS['bf16']})")
    margin("fwd+LSE B4 H32 S4096 D128", q, k, tiles, "LSE", err, LSE_ABS["bf16"])
    assert err <= LSE_ABS["bf16"]


# LSE bars: l sums P rounded to the input type, whose relative rounding error is at most
# 2^-8 (bf16, 8-bit significand) or 2^-11 (fp16), so log2(l) is off by at most
# 2^-8 / ln 2 = 5.6e-3 or 2^-11 / ln 2 = 7.0e-4, plus fp32 noise
LSE_ABS = {"bf16": 6e-3, "fp16": 1e-3}


@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("tiles", [(64, 64), (128, 64), (64, 128)], ids=lambda t: f"{t[0]}x{t[1]}")
def test_forward_lse(dt, tiles):
    B, H, N, D = 2, 4, 512, 64
    q, k = (dev(x, DTYPES[dt]) for x in cases.normal_inputs([(B, H, N, D)] * 2, seed=11, scale=2.0))
    v = dev(cases.normal_inputs([(B, H, N, D)], seed=12)[0], DTYPES[dt])  # V unscaled, as the reference cases
    log(f"lse dt={dt} tiles={tiles}")
    o, lse = _forward(q, k, v, *tiles)
    torch.cuda.synchronize()
    assert lse.dtype == torch.float32 and lse.shape == (B, H, N)
    want = orc.lse_log2(q.double().cpu().numpy(), k.double().cpu().numpy())
    err = float(np.abs(lse.cpu().numpy() - want).max())
    log(f"  lse max_abs={err:.3e}")
    assert err <= LSE_ABS[dt], (dt, tiles, err)
    check_forward(o, q, k, v, label=f"lse-fwd {dt} {tiles}")
    # the forward with LSE must equal the plain forward bit for bit
    assert torch.equal(o, fused_attention(q, k, v, *tiles))


def test_non_default_stream_and_repeatability():
    B, H, N, D = 1, 4, 1024, 128
    q, k, v = (dev(x, torch.bfloat16) for x in cases.normal_inputs([(B, H, N, D)] * 3, seed=5))
    o1 = fused_attention(q, k, v)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        o2 = fused_attention(q, k, v)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("tn", [64, 128])
def test_tile_m_does_not_change_results(D, tn):
    """tile_m sets how many 32-row waves share a workgroup; every 32-row group runs the same
    arithmetic over the same key tiles either way, so O, LSE, dQ, dK and dV of tile_m = 64 and
    tile_m = 128 are bitwise equal (partial tiles included)."""
    from attention.backward.fused_backward import _backward, _forward
    g = torch.Generator(device="cuda").manual_seed(D + tn)
    q, k, v, do = (torch.randn(1, 4, 1000, D, device="cuda", generator=g).bfloat16() for _ in range(4))
    log(f"tile_m invariance D{D} tile_n {tn}")
    o64, l64 = _forward(q, k, v, 64, tn)
    o128, l128 = _forward(q, k, v, 128, tn)
    torch.cuda.synchronize()
    assert torch.equal(o64, o128) and torch.equal(l64, l128)
    g64 = _backward(q, k, v, o64, l64, do, 64, tn)
    g128 = _backward(q, k, v, o128, l128, do, 128, tn)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(g64, g128))
