"""GPU parity of the fused causal GQA/MQA forward.

Cases:
  * the reference's 96-case GQA suite (tests/gqa/cases_gqa.py), fp16, at each tile config;
  * full-size GQA: B=2, H=32, H_kv=8, S=8192, D=128 bf16;
  * full-size MQA: B=1, H=32, H_kv=1, S=16384, D=64 fp16, inputs N(0,1) * 0.5;
  * H_kv == H must reproduce the MHA kernel's output bit for bit.
"""

import time

import numpy as np
import pytest
import torch

from attention.fused.fused import fused_attention
from attention.gqa.fused_gqa import fused_gqa_attention
from oracle import cases
from tests.gpu_util import check_forward, dev, log

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tiles", [(64, 64), (64, 128), (128, 64), (128, 128)], ids=lambda t: f"{t[0]}x{t[1]}")
@pytest.mark.parametrize("case", cases.all_gqa_cases(), ids=lambda c: c.id)
def test_reference_gqa_suite_fp16(case, tiles):
    q, k, v = (dev(x, torch.float16) for x in cases.make_gqa_inputs(case))
    assert k.shape[1] == case.H_kv  # never pre-expanded
    log(f"gqa-suite {case.id} tiles={tiles}")
    t0 = time.perf_counter()
    o = fused_gqa_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    check_forward(o, q, k, v, rows_count=24, label=f"{case.id} {tiles}", case=case, tiles=tiles, seconds=seconds)


@pytest.mark.parametrize("tiles", [(64, 64), (128, 64)], ids=lambda t: f"{t[0]}x{t[1]}")
def test_full_size_gqa_bf16_B2_H32_Hkv8_S8192_D128(tiles):
    q, k, v = cases.normal_inputs([(2, 32, 8192, 128), (2, 8, 8192, 128), (2, 8, 8192, 128)], seed=1)
    q, k, v = (dev(x, torch.bfloat16) for x in (q, k, v))
    log(f"full-size GQA tiles={tiles}")
    o = fused_gqa_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    check_forward(o, q, k, v, rows_count=24, label=f"GQA B2H32Hkv8 S8192 {tiles}", tiles=tiles,
                  margin_test="GQA fwd B2 H32 Hkv8 S8192 D128")


@pytest.mark.parametrize("tiles", [(64, 64), (128, 128)], ids=lambda t: f"{t[0]}x{t[1]}")
def test_full_size_mqa_fp16_B1_H32_Hkv1_S16384_D64(tiles):
    q, k, v = cases.normal_inputs([(1, 32, 16384, 64), (1, 1, 16384, 64), (1, 1, 16384, 64)],
                                  seed=2, scale=0.5)
    q, k, v = (dev(x, torch.float16) for x in (q, k, v))
    log(f"full-size MQA tiles={tiles}")
    o = fused_gqa_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    check_forward(o, q, k, v, rows_count=24, label=f"MQA S16384 {tiles}", tiles=tiles,
                  margin_test="MQA fwd B1 H32 Hkv1 S16384 D64")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_group_one_equals_mha(dt):
    q, k, v = (dev(x, dt) for x in cases.normal_inputs([(2, 4, 512, 64)] * 3, seed=9))
    a = fused_gqa_attention(q, k, v, 64, 64)
    b = fused_attention(q, k, v, 64, 64)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("group", [2, 4, 8])
def test_gqa_equals_mha_on_repeated_kv(group):
    """Packing several query heads per workgroup must not change any head's result."""
    H = 8
    q, k, v = cases.normal_inputs([(1, H, 512, 128), (1, H // group, 512, 128), (1, H // group, 512, 128)], seed=group)
    q, k, v = (dev(x, torch.bfloat16) for x in (q, k, v))
    a = fused_gqa_attention(q, k, v, 64, 64)
    b = fused_attention(q, k.repeat_interleave(group, 1).contiguous(), v.repeat_interleave(group, 1).contiguous(), 64, 64)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("D", [32, 128])
def test_heads_per_workgroup_do_not_change_results(D):
    """With 64-row tiles a workgroup serves four heads of a K/V group when the grid is large
    (B=1 H=32 H_kv=4 S=8192: 1024 workgroups) and two when it is small (the same heads 0..7
    alone: 256 workgroups).  Each row's arithmetic is the same either way: bitwise equal."""
    g = torch.Generator(device="cuda").manual_seed(D)
    q = torch.randn(1, 32, 8192, D, device="cuda", generator=g).half()
    k, v = (torch.randn(1, 4, 8192, D, device="cuda", generator=g).half() for _ in range(2))
    log(f"gqa heads-per-workgroup B1 H32 Hkv4 S8192 D{D}")
    big = fused_gqa_attention(q, k, v, 64, 64)
    small = fused_gqa_attention(q[:, :8].contiguous(), k[:, :1].contiguous(), v[:, :1].contiguous(), 64, 64)
    torch.cuda.synchronize()
    assert torch.isfinite(big).all()
    assert torch.equal(big[:, :8], small)
