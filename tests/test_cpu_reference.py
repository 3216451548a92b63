"""Pins oracle/cpu_reference.py -- the fp32 PyTorch checker -- against the float64 oracle (CPU only).

cpu_reference restates the reference's fp32 ground truth as its harness runs it:
the explicit formula (attention/fused/reference.py:16-23), the head chunking under a
2 GiB score budget (tests/fused/run_correctness.py:36,57-67, whole GQA groups per chunk
as tests/gqa/run_correctness_gqa.py:63-80) and fp32 autograd of the formula
(tests/backward/run_correctness_backward.py:25-44).  Several GPU tests use it as the
element-wise checker, so each function is compared here with the float64 oracle
(which tests/test_oracle.py pins against torch SDPA, loops and finite differences),
and mutated copies of the chunking show that a wrong head index is caught.
"""

import inspect
import math

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from oracle import cpu_reference as cref

# fp32 formula vs float64: a few ulp of fp32 on O(1) outputs
TOL_O = dict(rtol=2e-5, atol=2e-5)
TOL_GRAD = dict(rtol=1e-4, atol=1e-4)


def rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * np.float32(scale)


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x))


@pytest.mark.parametrize("B,H,Hkv,N,D", [(2, 4, 4, 64, 32), (1, 8, 2, 96, 64), (1, 4, 1, 48, 16), (1, 3, 3, 1, 8)])
def test_explicit_formula_matches_float64_oracle(B, H, Hkv, N, D):
    q, k, v = rand((B, H, N, D), 1, 2.0), rand((B, Hkv, N, D), 2, 2.0), rand((B, Hkv, N, D), 3)
    got = cref.reference_attention_explicit(t(q), t(k), t(v))
    assert got.dtype == torch.float32 and tuple(got.shape) == (B, H, N, D)
    np.testing.assert_allclose(got.numpy(), orc.forward(q, k, v), **TOL_O)


def test_explicit_formula_special_cases():
    # row 0 sees only key 0: O[0] = V[0]; Q = 0 gives the prefix means of V
    B, H, N, D = 1, 2, 40, 8
    q, k, v = rand((B, H, N, D), 4, 5.0), rand((B, H, N, D), 5, 5.0), rand((B, H, N, D), 6)
    o = cref.reference_attention_explicit(t(q), t(k), t(v)).numpy()
    np.testing.assert_array_equal(o[:, :, 0], v[:, :, 0])
    o0 = cref.reference_attention_explicit(t(np.zeros_like(q)), t(k), t(v)).numpy()
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, N + 1)[None, None, :, None]
    np.testing.assert_allclose(o0, prefix, **TOL_O)


def _budget_for_heads(N, heads):
    """A score budget that admits exactly `heads` heads of N x N per chunk."""
    return heads * N * N * 4 * 2


@pytest.mark.parametrize("H,Hkv,heads", [
    (8, 8, 3),    # MHA, chunks of 3, 3, 2 (H not a multiple of the chunk)
    (8, 8, 1),    # one head per chunk
    (12, 6, 3),   # g = 2: a 3-head budget rounds down to whole groups (2 heads)
    (12, 3, 6),   # g = 4: budget of 6 heads -> chunks of 4 (one group each)
    (16, 4, 9),   # g = 4: budget of 9 heads -> chunks of 8, two groups each
    (8, 2, 1),    # g = 4, budget below one group: chunk = one whole group
    (8, 1, 5),    # MQA (g = 8): every chunk is the whole group
])
def test_chunked_reference_matches_oracle_across_chunk_boundaries(monkeypatch, H, Hkv, heads):
    B, N, D = 2, 32, 16
    monkeypatch.setattr(cref, "REFERENCE_BUDGET_BYTES", _budget_for_heads(N, heads))
    q, k, v = rand((B, H, N, D), 7, 2.0), rand((B, Hkv, N, D), 8, 2.0), rand((B, Hkv, N, D), 9)
    got = cref.reference_chunked(t(q), t(k), t(v))
    np.testing.assert_allclose(got.numpy(), orc.forward(q, k, v), **TOL_O)
    # and one chunk holding every head gives the same values
    monkeypatch.setattr(cref, "REFERENCE_BUDGET_BYTES", _budget_for_heads(N, H))
    whole = cref.reference_chunked(t(q), t(k), t(v))
    np.testing.assert_allclose(got.numpy(), whole.numpy(), rtol=0, atol=1e-6)


def _mutated_chunked(edits):
    """reference_chunked with source edits applied, built in cpu_reference's namespace
    (it reads the module's REFERENCE_BUDGET_BYTES, which the tests monkeypatch)."""
    src = inspect.getsource(cref.reference_chunked)
    for old, new in edits:
        assert src.count(old) == 1, f"mutation anchor not found once: {old!r}"
        src = src.replace(old, new)
    ns = {}
    exec(compile(src, "<mutant>", "exec"), cref.__dict__, ns)
    return ns["reference_chunked"]


_NO_GROUP_ROUNDING = ("chunk = max(g, chunk - chunk % g) if g > 1 else chunk", "chunk = chunk")


@pytest.mark.parametrize("edits", [
    # query head h0 mapped to K/V head h0 instead of h0 // g
    [("hk0, hk1 = h0 // g,", "hk0, hk1 = h0,")],
    # chunks that are not whole groups
    [_NO_GROUP_ROUNDING],
    # ... and the last K/V head index rounded down (dropping "+ g - 1"); with whole-group
    # chunks the two roundings agree, so this mistake needs a straddling chunk to show
    [_NO_GROUP_ROUNDING, ("(min(H, h0 + chunk) + g - 1) // g", "min(H, h0 + chunk) // g")],
    # output written one head past the chunk
    [("out[b:b + 1, h0:h0 + chunk]", "out[b:b + 1, h0 + 1:h0 + chunk + 1]")],
], ids=["kv-head-index", "straddling-chunks", "kv-head-floor", "output-offset"])
def test_planted_chunking_mistakes_are_caught(monkeypatch, edits):
    B, H, Hkv, N, D = 1, 12, 3, 24, 8   # g = 4
    monkeypatch.setattr(cref, "REFERENCE_BUDGET_BYTES", _budget_for_heads(N, 5))  # 5 heads: straddles a group
    q, k, v = rand((B, H, N, D), 10, 2.0), rand((B, Hkv, N, D), 11, 2.0), rand((B, Hkv, N, D), 12)
    want = orc.forward(q, k, v)
    np.testing.assert_allclose(cref.reference_chunked(t(q), t(k), t(v)).numpy(), want, **TOL_O)
    mutant = _mutated_chunked(edits)
    try:
        got = mutant(t(q), t(k), t(v)).numpy()
    except (RuntimeError, ValueError, IndexError, ZeroDivisionError):
        return  # the mutant cannot even run on this shape: caught
    assert not np.allclose(got, want, rtol=1e-3, atol=1e-3), f"mutant {edits} went unnoticed"


@pytest.mark.parametrize("B,H,N,D,sigma", [(1, 2, 16, 8, 1.0), (2, 3, 48, 16, 1.0), (1, 2, 33, 32, 3.0)])
def test_fp32_autograd_matches_float64_gradients(B, H, N, D, sigma):
    q, k, v = (rand((B, H, N, D), s, sigma) for s in (21, 22, 23))
    do = rand((B, H, N, D), 24)
    o, dq, dk, dv = cref.reference_grads(t(q), t(k), t(v), t(do))
    o64, dq64, dk64, dv64 = orc.backward(q, k, v, do)
    tol = TOL_GRAD if sigma == 1.0 else dict(rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(o.numpy(), o64, **TOL_O)
    for got, want in ((dq, dq64), (dk, dk64), (dv, dv64)):
        assert got.dtype == torch.float32
        np.testing.assert_allclose(got.numpy(), want, **tol)


@pytest.mark.parametrize("H,Hkv", [(4, 2), (8, 2), (4, 1), (6, 6)])
def test_fp32_autograd_gqa_sums_group_gradients(H, Hkv):
    B, N, D = 2, 40, 16
    q = rand((B, H, N, D), 31)
    k, v = rand((B, Hkv, N, D), 32), rand((B, Hkv, N, D), 33)
    do = rand((B, H, N, D), 34)
    o, dq, dk, dv = cref.reference_grads_gqa(t(q), t(k), t(v), t(do))
    o64, dq64, dk64, dv64 = orc.backward(q, k, v, do)
    assert tuple(dk.shape) == (B, Hkv, N, D) and tuple(dv.shape) == (B, Hkv, N, D)
    np.testing.assert_allclose(o.numpy(), o64, **TOL_O)
    for got, want in ((dq, dq64), (dk, dk64), (dv, dv64)):
        np.testing.assert_allclose(got.numpy(), want, **TOL_GRAD)
    # a planted head mapping (query head h on K/V head h % H_kv instead of h // g) fails the bar
    if Hkv not in (1, H):
        perm = [h % Hkv for h in range(H)]
        o_bad = cref.reference_attention_explicit(t(q), t(k[:, perm]), t(v[:, perm]))
        assert not np.allclose(o_bad.numpy(), o64, **TOL_GRAD)


def test_gradient_scale_is_one_over_sqrt_d():
    # dQ and dK carry exactly one factor 1/sqrt(D): scaling Q by a and K by 1/a leaves
    # the scores unchanged, so dQ scales by 1/a and dK by a
    B, H, N, D = 1, 2, 24, 16
    q, k, v, do = (rand((B, H, N, D), s) for s in (41, 42, 43, 44))
    _, dq, dk, _ = cref.reference_grads(t(q), t(k), t(v), t(do))
    a = 2.0
    _, dq2, dk2, _ = cref.reference_grads(t(q * a), t(k / a), t(v), t(do))
    np.testing.assert_allclose(dq2.numpy() * a, dq.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dk2.numpy() / a, dk.numpy(), rtol=1e-4, atol=1e-5)
    _, dq64, _, _ = orc.backward(q, k, v, do)
    assert math.isclose(float(np.abs(dq.numpy()).max()), float(np.abs(dq64).max()), rel_tol=1e-4)
