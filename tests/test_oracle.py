"""Pins the oracle against independent checks (CPU only).

Each oracle function is compared with something other than a retyped copy of its
formula: a pure-Python loop version, torch's SDPA in float64, scipy's logsumexp,
finite differences, closed-form special cases and algebraic identities.  The
planted-mistake tests at the end show these checks catch a wrong sign, a dropped
scale and a transposed operand.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.special import logsumexp

from oracle import attention_oracle as orc
from oracle import cases


def rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def sdpa64(q, k, v):
    q, k, v = (torch.from_numpy(np.ascontiguousarray(x)).double() for x in (q, k, v))
    if k.shape[1] != q.shape[1]:
        g = q.shape[1] // k.shape[1]
        k, v = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True).numpy()


# ---------------------------------------------------------------- forward
@pytest.mark.parametrize("shape", [(1, 1, 5, 3), (2, 2, 7, 4), (1, 3, 9, 2)])
def test_forward_matches_pure_python_loops(shape):
    q, k, v = (rand(shape, s) for s in (1, 2, 3))
    np.testing.assert_allclose(orc.forward(q, k, v), orc.naive_loops(q, k, v), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shape,hkv", [((2, 4, 64, 32), 4), ((1, 8, 96, 64), 2), ((1, 4, 48, 16), 1)])
def test_forward_matches_torch_sdpa_float64(shape, hkv):
    B, H, N, D = shape
    q = rand(shape, 10)
    k, v = rand((B, hkv, N, D), 11), rand((B, hkv, N, D), 12)
    np.testing.assert_allclose(orc.forward(q, k, v), sdpa64(q, k, v), rtol=1e-10, atol=1e-12)


def test_forward_row0_is_v0_and_zero_q_gives_prefix_mean():
    B, H, N, D = 2, 3, 40, 8
    q, k, v = rand((B, H, N, D), 4, 5.0), rand((B, H, N, D), 5, 5.0), rand((B, H, N, D), 6)
    o = orc.forward(q, k, v)
    np.testing.assert_array_equal(o[:, :, 0, :], v[:, :, 0, :])
    o0 = orc.forward(np.zeros_like(q), k, v)
    prefix_mean = np.cumsum(v, axis=2) / np.arange(1, N + 1)[None, None, :, None]
    np.testing.assert_allclose(o0, prefix_mean, rtol=1e-12, atol=1e-12)


def test_forward_large_scores_stay_finite():
    q, k, v = (x.astype(np.float16).astype(np.float64) for x in cases.make_inputs(cases.Case(1, 2, 128, 64, "large")))
    o = orc.forward(q, k, v)
    assert np.isfinite(o).all()
    np.testing.assert_allclose(o, sdpa64(q, k, v), rtol=1e-9, atol=1e-9)


def test_row_sampling_equals_full_rows():
    q, k, v = rand((1, 2, 256, 32), 7), rand((1, 2, 256, 32), 8), rand((1, 2, 256, 32), 9)
    rows = orc.sample_rows(256, count=20)
    np.testing.assert_allclose(orc.forward(q, k, v, rows), orc.forward(q, k, v)[:, :, rows], rtol=0, atol=1e-13)
    assert rows[0] == 0 and rows[-1] == 255 and 63 in rows and 64 in rows


def test_gqa_equals_mha_on_repeated_kv():
    B, H, Hkv, N, D = 2, 8, 2, 48, 16
    q, k, v = rand((B, H, N, D), 1), rand((B, Hkv, N, D), 2), rand((B, Hkv, N, D), 3)
    k_rep, v_rep = np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1)
    # query head h must use K/V head h // 4: check head 5 against K/V head 1 directly
    o = orc.forward(q, k, v)
    o5 = orc.forward(q[:, 5:6], k[:, 1:2], v[:, 1:2])
    np.testing.assert_allclose(o[:, 5:6], o5, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(o, orc.forward(q, k_rep, v_rep), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("tm,tn", [(64, 64), (64, 128), (128, 64), (128, 128), (32, 16)])
def test_online_softmax_tiling_matches_closed_form(tm, tn):
    q, k, v = rand((1, 2, 256, 32), 21, 2.0), rand((1, 2, 256, 32), 22, 2.0), rand((1, 2, 256, 32), 23)
    o, lse = orc.online_softmax_forward(q, k, v, tm, tn)
    np.testing.assert_allclose(o, orc.forward(q, k, v), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(lse, orc.lse_log2(q, k), rtol=1e-12, atol=1e-11)


# ---------------------------------------------------------------- LSE / Delta
def test_lse_matches_scipy_logsumexp_and_normalises():
    B, H, N, D = 1, 2, 64, 16
    q, k = rand((B, H, N, D), 31, 3.0), rand((B, H, N, D), 32, 3.0)
    s = np.einsum("bhid,bhjd->bhij", q, k) / math.sqrt(D)
    s[..., np.triu(np.ones((N, N), bool), 1)] = -np.inf
    np.testing.assert_allclose(orc.lse_log2(q, k), logsumexp(s, axis=-1) * orc.LOG2E, rtol=1e-12, atol=1e-12)
    c = orc.LOG2E / math.sqrt(D)
    p = np.exp2(orc.masked_scores(q, k) * math.sqrt(D) * c - orc.lse_log2(q, k)[..., None])
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-12)


def test_delta_identity_rowsum_p_dp():
    B, H, N, D = 1, 2, 32, 8
    q, k, v, do = (rand((B, H, N, D), s) for s in (41, 42, 43, 44))
    o = orc.forward(q, k, v)
    p = orc.probs(q, k)
    dp = do @ np.swapaxes(v, -1, -2)
    np.testing.assert_allclose(orc.delta(do, o), (p * dp).sum(-1), rtol=1e-11, atol=1e-12)


# ---------------------------------------------------------------- gradients
def _loss(q, k, v, do):
    return float((orc.forward(q, k, v) * do).sum())


def test_backward_matches_finite_differences():
    B, H, N, D = 1, 1, 8, 4
    q, k, v, do = (rand((B, H, N, D), s) for s in (51, 52, 53, 54))
    _, dq, dk, dv = orc.backward(q, k, v, do)
    eps = 1e-6
    for x, g in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args = [xp if a is x else a for a in (q, k, v)]
            argm = [xm if a is x else a for a in (q, k, v)]
            num[idx] = (_loss(*args, do) - _loss(*argm, do)) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("hkv", [4, 2, 1])
def test_backward_matches_torch_autograd_float64(hkv):
    B, H, N, D = 2, 4, 40, 16
    q = rand((B, H, N, D), 61)
    k, v = rand((B, hkv, N, D), 62), rand((B, hkv, N, D), 63)
    do = rand((B, H, N, D), 64)
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    g = H // hkv
    o = F.scaled_dot_product_attention(tq, tk.repeat_interleave(g, 1), tv.repeat_interleave(g, 1), is_causal=True)
    o.backward(torch.from_numpy(do))
    o_orc, dq, dk, dv = orc.backward(q, k, v, do)
    np.testing.assert_allclose(o_orc, o.detach().numpy(), rtol=1e-10, atol=1e-12)
    for a, b in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        np.testing.assert_allclose(a, b.numpy(), rtol=1e-9, atol=1e-11)


def test_dq_rows_equals_full_dq():
    q, k, v, do = (rand((1, 2, 96, 16), s) for s in (71, 72, 73, 74))
    rows = orc.sample_rows(96, count=12)
    np.testing.assert_allclose(orc.dq_rows(q, k, v, do, rows), orc.backward(q, k, v, do)[1][:, :, rows],
                               rtol=1e-11, atol=1e-13)


# ---------------------------------------------------------------- cases
def test_case_lists_match_reference_counts_and_order():
    mha, gqa, bwd = cases.all_cases(), cases.all_gqa_cases(), cases.all_bwd_cases()
    assert len(mha) == 84 and len(gqa) == 96 and len(bwd) == 7
    assert mha[0].id == "B1_H1_N128_D32_tiny" and mha[-1].id == "B16_H32_N512_D128_large"
    assert gqa[0].id == "B4_H8_Hkv1_N128_D32_tiny" and gqa[-1].id == "B4_H8_Hkv8_N8192_D128_large"
    assert bwd[0].id == "B1_H1_N128_D64_s1" and bwd[0].seed == 192


def test_case_inputs_are_crc32_seeded_and_deterministic():
    import zlib
    c = cases.Case(2, 8, 128, 64, "large")
    assert c.seed == zlib.crc32(b"B2_H8_N128_D64_large")
    q1, k1, v1 = cases.make_inputs(c)
    q2, _, _ = cases.make_inputs(c)
    assert q1.dtype == np.float16 and q1.shape == (2, 8, 128, 64)
    np.testing.assert_array_equal(q1, q2)
    # the draw order is Q, K, V from one generator: V is unscaled N(0,1)
    assert 0.8 < float(np.std(v1.astype(np.float32))) < 1.2
    assert 5.5 < float(np.std(q1.astype(np.float32))) < 8.5
    gq, gk, gv = cases.make_gqa_inputs(cases.GqaCase(4, 8, 2, 128, 32, "tiny"))
    assert gq.shape == (4, 8, 128, 32) and gk.shape == gv.shape == (4, 2, 128, 32)


# ---------------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught():
    """A wrong mask direction, a dropped 1/sqrt(D) or a transposed operand must fail the pins."""
    B, H, N, D = 1, 2, 24, 8
    q, k, v = rand((B, H, N, D), 81, 2.0), rand((B, H, N, D), 82, 2.0), rand((B, H, N, D), 83)
    ref = sdpa64(q, k, v)

    def wrong_mask(q, k, v):
        s = np.einsum("bhid,bhjd->bhij", q, k) / math.sqrt(D)
        s[..., np.tril(np.ones((N, N), bool), -1)] = -np.inf  # masks the past instead
        p = np.exp(s - s.max(-1, keepdims=True))
        return (p / p.sum(-1, keepdims=True)) @ v

    def no_scale(q, k, v):
        return orc.forward(q * math.sqrt(D), k, v)

    def transposed_v(q, k, v):
        return orc.forward(q, k, np.swapaxes(v, -1, -2)[..., :N, :D] if N == D else v[..., ::-1, :])

    for bad in (wrong_mask, no_scale, transposed_v):
        assert not np.allclose(bad(q, k, v), ref, rtol=1e-6, atol=1e-6), bad.__name__
