"""Any sequence length: partial last query and key tiles (beyond the reference, which requires
N to be a multiple of both tiles and lists partial edge tiles as future work).

Forward, forward with LSE, GQA and the backward at lengths that are not multiples of 64 or 128,
each against the fp32 reference formula on the GPU and the float64 oracle; outputs written
through the C ABI into buffers with a guard region behind them, which must stay untouched.
"""

import math

import numpy as np
import pytest
import torch

from attention import _lib
from attention.backward.fused_backward import _forward, fused_attention_autograd
from attention.fused.fused import fused_attention
from attention.gqa.fused_gqa import fused_gqa_attention, fused_gqa_attention_autograd
from oracle import attention_oracle as orc
from oracle import cases
from oracle.cpu_reference import reference_grads, reference_grads_gqa
from tests.gpu_util import check_forward, dev, log

pytestmark = pytest.mark.gpu

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}
TILES = [(64, 64), (128, 64), (64, 128), (128, 128)]
ODD_N = [1, 17, 63, 100, 130, 257, 1000]


@pytest.mark.parametrize("N", ODD_N)
@pytest.mark.parametrize("tiles", TILES, ids=lambda t: f"{t[0]}x{t[1]}")
def test_forward_any_length(N, tiles):
    q, k, v = (dev(x, torch.bfloat16) for x in cases.normal_inputs([(2, 3, N, 64)] * 3, seed=N + tiles[0]))
    log(f"partial fwd N={N} tiles={tiles}")
    o = fused_attention(q, k, v, *tiles)
    torch.cuda.synchronize()
    assert torch.equal(o[:, :, 0], v[:, :, 0])  # row 0 sees key 0 only
    check_forward(o, q, k, v, rows_count=min(N, 40), label=f"partial fwd N{N} {tiles}")


@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("D", [32, 64, 128])
def test_forward_lse_any_length(dt, D):
    N = 321
    q, k, v = (dev(x, DTYPES[dt]) for x in cases.normal_inputs([(1, 2, N, D)] * 3, seed=D))
    o, lse = _forward(q, k, v, 128, 64)
    torch.cuda.synchronize()
    check_forward(o, q, k, v, label=f"partial fwd+lse {dt} D{D}")
    want = orc.lse_log2(q.double().cpu().numpy(), k.double().cpu().numpy())
    # l sums P rounded to the element type: at most 2^-8 (bf16) / 2^-11 (fp16) relative,
    # i.e. 2^-8 / ln 2 = 5.6e-3 / 2^-11 / ln 2 = 7.0e-4 in log2 units
    tol = 6e-3 if dt == "bf16" else 1e-3
    assert float(np.abs(lse.cpu().numpy() - want).max()) <= tol


@pytest.mark.parametrize("group", [2, 4])
def test_gqa_forward_any_length(group):
    N = 1000
    q = dev(cases.normal_inputs([(1, 8, N, 128)], seed=group)[0], torch.bfloat16)
    k, v = (dev(x, torch.bfloat16) for x in cases.normal_inputs([(1, 8 // group, N, 128)] * 2, seed=group + 1))
    o = fused_gqa_attention(q, k, v, 128, 64)
    torch.cuda.synchronize()
    check_forward(o, q, k, v, label=f"partial gqa fwd g{group}")


def test_forward_full_size_odd_length_bf16():
    """The headline shape at S = 4097 (one row past a tile multiple)."""
    q, k, v = (dev(x, torch.bfloat16) for x in cases.normal_inputs([(4, 32, 4097, 128)] * 3, seed=9))
    o = fused_attention(q, k, v, 128, 64)
    torch.cuda.synchronize()
    check_forward(o, q, k, v, label="partial fwd B4 H32 S4097 D128")


def _grads_ok(got, ref, label, mixed_for_kv=False):
    msg = []
    for name, g, r in zip(("O", "dQ", "dK", "dV"), got, ref):
        assert torch.isfinite(g).all(), (label, name)
        err = (g.float() - r).abs()
        a = float(err.max())
        # relative to the reference's norm, floored at the absolute tolerance's scale: at
        # N = 1 the exact dQ and dK are zero (a single key: P = 1, dP = Delta)
        rel = float((g.float() - r).norm() / max(float(r.norm()), 2e-2 * math.sqrt(r.numel())))
        ratio = float((err / (2e-2 + 2e-2 * r.abs())).max())
        msg.append(f"{name}:abs={a:.2e},rel={rel:.1e}")
        assert rel <= 2e-2, (label, name, rel)
        assert (ratio <= 1.0) if (mixed_for_kv and name in ("dK", "dV")) else (a <= 2e-2), (label, name, a)
    log(f"{label} " + " ".join(msg))


@pytest.mark.parametrize("N", [1, 33, 100, 200, 321, 1000])
@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("D", [64, 128])
def test_backward_any_length(N, dt, D):
    q, k, v, do = (dev(x, DTYPES[dt]) for x in cases.normal_inputs([(1, 2, N, D)] * 4, seed=N + D))
    log(f"partial bwd N={N} {dt} D={D}")
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = fused_attention_autograd(qg, kg, vg, 128, 64)
    o.backward(do)
    torch.cuda.synchronize()
    got = (o.detach(), qg.grad, kg.grad, vg.grad)
    _grads_ok(got, reference_grads(q, k, v, do), f"partial bwd N{N} {dt} D{D}")
    if N <= 200:
        want = orc.backward(*(t.double().cpu().numpy() for t in (q, k, v, do)))
        worst = max(float(np.abs(g.double().cpu().numpy() - w).max()) for g, w in zip(got, want))
        assert worst <= 2e-2, worst


@pytest.mark.parametrize("tiles", [(64, 128), (128, 128)], ids=lambda t: f"{t[0]}x{t[1]}")
def test_gqa_backward_any_length(tiles):
    N = 777
    q, do = (dev(x, torch.float16) for x in cases.normal_inputs([(1, 8, N, 64)] * 2, seed=7))
    k, v = (dev(x, torch.float16) for x in cases.normal_inputs([(1, 2, N, 64)] * 2, seed=8))
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = fused_gqa_attention_autograd(qg, kg, vg, *tiles)
    o.backward(do)
    torch.cuda.synchronize()
    _grads_ok((o.detach(), qg.grad, kg.grad, vg.grad), reference_grads_gqa(q, k, v, do),
              f"partial gqa bwd {tiles}", mixed_for_kv=True)


def _guarded(shape, dtype, guard=4096):
    """A tensor of `shape` at the front of a larger buffer whose tail holds a sentinel."""
    n = math.prod(shape)
    buf = torch.full((n + guard,), -12345.0, device="cuda", dtype=dtype)
    return buf[:n].view(shape), buf[n:]


@pytest.mark.parametrize("N", [1, 65, 200])
def test_no_writes_past_the_outputs(N):
    B, H, D = 1, 2, 64
    dt = torch.bfloat16
    q, k, v, do = (dev(x, dt) for x in cases.normal_inputs([(B, H, N, D)] * 4, seed=N))
    o, o_tail = _guarded((B, H, N, D), dt)
    lse, l_tail = _guarded((B, H, N), torch.float32)
    _lib.fwd(q, k, v, o, lse, 128, 64)
    dq, q_tail = _guarded((B, H, N, D), dt)
    dk, k_tail = _guarded((B, H, N, D), dt)
    dv, v_tail = _guarded((B, H, N, D), dt)
    _lib.bwd(q, k, v, o, do, lse, dq, dk, dv, 128, 64)
    torch.cuda.synchronize()
    for name, tail in (("O", o_tail), ("LSE", l_tail), ("dQ", q_tail), ("dK", k_tail), ("dV", v_tail)):
        assert bool((tail == -12345.0).all()), f"{name}: write past the end at N={N}"
    check_forward(o, q, k, v, rows_count=min(N, 40), label=f"guarded fwd N{N}")
