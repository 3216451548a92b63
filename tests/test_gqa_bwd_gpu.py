"""GPU parity of fused_gqa_attention_autograd: the GQA/MQA recompute backward.

The reference's backward is MHA-only; this extends it to grouped K/V heads with
the same math: dK and dV of a K/V head are the sums over its query heads
(attention/gqa/reference_gqa.py:15-26 repeats K/V to the query heads, so autograd
of that reference sums each group's gradients).  Every case checks O, dQ, dK, dV
  * against fp32 autograd of the reference formula on repeated K/V, on the GPU:
    O and dQ (per query head, as in the MHA backward) with max-abs <= 2e-2; dK and
    dV, which sum G query heads and so grow up to G-fold, with the reference's mixed
    tolerance |err| <= 2e-2 + 2e-2 |ref| (tests/fused/run_correctness.py:33-34) — a
    16-bit output's own rounding (half an ulp, up to 2^-8 |x| in bf16) exceeds 2e-2
    absolute once |x| >= 8 — and all four with relative Frobenius error <= 2e-2;
  * on small shapes, against the float64 closed-form gradients of the oracle;
  * against the MHA backward run on explicitly repeated K/V, whose per-head dK/dV
    summed over each group must agree with the grouped result.
"""

import numpy as np
import pytest
import torch

from attention.backward.fused_backward import fused_attention_autograd
from attention.gqa.fused_gqa import fused_gqa_attention_autograd
from oracle import attention_oracle as orc
from oracle import cases
from oracle.cpu_reference import reference_grads_gqa
from tests.gpu_util import dev, log, margin

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL = 2e-2
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def run(fn, q, k, v, do, tiles):
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = fn(q, k, v, *tiles)
    o.backward(do)
    torch.cuda.synchronize()
    return o.detach(), q.grad, k.grad, v.grad


def make(B, H, Hkv, N, D, dtype, seed):
    q, do = cases.normal_inputs([(B, H, N, D)] * 2, seed=seed)
    k, v = cases.normal_inputs([(B, Hkv, N, D)] * 2, seed=seed + 1)
    return [dev(x, dtype) for x in (q, k, v, do)]


def check(q, k, v, do, tiles, label, oracle=False, margin_test=None):
    got = run(fused_gqa_attention_autograd, q, k, v, do, tiles)
    for name, g, ref_t in zip(("O", "dQ", "dK", "dV"), got, (q, q, k, v)):
        assert g.dtype == q.dtype and g.shape == ref_t.shape, name
        assert torch.isfinite(g).all(), f"{label}: non-finite {name}"
    ref = reference_grads_gqa(q, k, v, do)
    msg = []
    for name, g, r in zip(("O", "dQ", "dK", "dV"), got, ref):
        err = (g.float() - r).abs()
        a = float(err.max())
        ratio = float((err / (MAX_ABS + REL * r.abs())).max())
        # relative to the reference's norm, floored at the absolute tolerance's scale: at
        # N = 1 the exact dQ and dK are zero (a single key: P = 1, dP = Delta)
        rel = float((g.float() - r).norm() / max(float(r.norm()), MAX_ABS * r.numel() ** 0.5))
        msg.append(f"{name}:abs={a:.2e},ratio={ratio:.2f},rel={rel:.1e}")
        if margin_test is not None:
            margin(margin_test, q, k, tiles, name, a, MAX_ABS, mixed=ratio, rel=rel)
        assert rel <= REL, (label, name, a, rel)
        if name in ("O", "dQ"):
            assert a <= MAX_ABS, (label, name, a)
        else:
            assert ratio <= 1.0, (label, name, a, ratio)
    del ref
    if oracle:
        want = orc.backward(*(t[:1].double().cpu().numpy() for t in (q, k, v, do)))
        worst = 0.0
        for g, w in zip(got, want):
            d = np.abs(g[:1].double().cpu().numpy() - w)
            worst = max(worst, float((d / (MAX_ABS + REL * np.abs(w))).max()))
        msg.append(f"oracle_ratio={worst:.2f}")
        assert worst <= 1.0, (label, worst)
    log(f"{label} " + " ".join(msg))
    return got


@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_gqa_backward_small(dt, D, group):
    H = 8
    q, k, v, do = make(1, H, H // group, 256, D, DTYPES[dt], seed=10 * D + group)
    log(f"gqa-bwd {dt} D={D} group={group}")
    check(q, k, v, do, (64, 64), f"gqa-bwd {dt} D{D} g{group}", oracle=True)


@pytest.mark.parametrize("tiles", [(64, 128), (128, 64), (128, 128)], ids=lambda t: f"{t[0]}x{t[1]}")
def test_gqa_backward_tiles(tiles):
    q, k, v, do = make(2, 8, 2, 384 if 128 not in tiles else 512, 128, torch.bfloat16, seed=sum(tiles))
    check(q, k, v, do, tiles, f"gqa-bwd tiles {tiles}")


def test_gqa_backward_partial_key_tile():
    """S = 320: the dK/dV workgroup's last 128-key tile is partial for every head of the group."""
    q, k, v, do = make(1, 4, 1, 320, 64, torch.float16, seed=3)
    check(q, k, v, do, (64, 64), "gqa-bwd partial N320", oracle=True)


@pytest.mark.parametrize("group", [2, 4])
def test_gqa_backward_equals_group_sum_of_mha(group):
    H, D, N = 8, 64, 512
    q, k, v, do = make(1, H, H // group, N, D, torch.float16, seed=40 + group)
    g_o, g_dq, g_dk, g_dv = run(fused_gqa_attention_autograd, q, k, v, do, (64, 64))
    ke, ve = k.repeat_interleave(group, 1).contiguous(), v.repeat_interleave(group, 1).contiguous()
    m_o, m_dq, m_dk, m_dv = run(fused_attention_autograd, q, ke, ve, do, (64, 64))
    assert torch.equal(g_o, m_o)
    assert torch.equal(g_dq, m_dq)
    for g, m in ((g_dk, m_dk), (g_dv, m_dv)):
        summed = m.float().reshape(1, H // group, group, N, D).sum(2)
        assert float((g.float() - summed).abs().max()) <= 1e-2


def test_gqa_backward_full_size_B2_H32_Hkv8_S4096_D128_bf16():
    q, k, v, do = make(2, 32, 8, 4096, 128, torch.bfloat16, seed=11)
    log("gqa-bwd full-size B2 H32 Hkv8 S4096 D128 bf16")
    check(q, k, v, do, (128, 64), "gqa-bwd B2H32Hkv8 S4096 D128", margin_test="GQA fwd+bwd B2 H32 Hkv8 S4096 D128")


def test_mqa_backward_full_size_B1_H32_Hkv1_S4096_D64_fp16():
    q, k, v, do = make(1, 32, 1, 4096, 64, torch.float16, seed=12)
    q = q * 0.5
    k = k * 0.5
    v = v * 0.5
    log("mqa-bwd full-size B1 H32 Hkv1 S4096 D64 fp16")
    check(q, k, v, do, (128, 64), "mqa-bwd B1H32Hkv1 S4096 D64", margin_test="MQA fwd+bwd B1 H32 Hkv1 S4096 D64")


def _bwd_through_abi(q, k, v, o, do, lse, ws_bytes):
    """dQ, dK, dV from fa_bwd_gqa with a workspace of ws_bytes (0: NULL: dK/dV first, no split)."""
    import ctypes
    import math
    from attention import _lib
    lib = _lib.load()
    B, H, S, D = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    code = lib.fa_bwd_gqa(*(ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, o, do, lse, dq, dk, dv)),
                          B, H, k.shape[1], S, D, _lib.dtype_code(q.dtype), _lib.scale_log2(D),
                          1.0 / math.sqrt(D), 128, 64, _lib._ptr(ws), ws_bytes,
                          _lib._stream(q.device))
    _lib.check(code, "fa_bwd_gqa")
    torch.cuda.synchronize()
    return dq, dk, dv


@pytest.mark.parametrize("shape", [(1, 32, 1, 1000, 64), (1, 8, 2, 2000, 128), (2, 12, 4, 1500, 32),
                                   (1, 4, 4, 4200, 128), (1, 2, 2, 4097, 64)],
                         ids=lambda s: "B%dH%dHkv%dS%dD%d" % s)
def test_dkdv_split_matches_register_sums(shape):
    """The split of each key tile's (query tile, query head) pairs over several workgroups (fp32
    partials + reduction; MHA and GQA) against one workgroup summing every pair in registers:
    dQ identical, dK/dV equal up to fp32 summation order; a smaller workspace takes a smaller
    split; repeated calls are bitwise reproducible."""
    from attention import _lib
    from attention.backward.fused_backward import _forward
    B, H, Hkv, S, D = shape
    q, k, v, do = make(B, H, Hkv, S, D, torch.bfloat16, seed=S + D)
    o, lse = _forward(q, k, v, 128, 64)
    need = _lib.load().fa_bwd_gqa_workspace_size(B, H, Hkv, S, D)
    rows = (8 * B * H * S + 255) // 256 * 256   # the per-row terms; the rest holds the partials
    assert need > rows, "these shapes leave the GPU idle without a split"
    if Hkv == H:  # MHA: also the Python backward, which takes the same workspace
        from attention.backward.fused_backward import _backward
        mha = _backward(q, k, v, o, lse, do, 128, 64)
        torch.cuda.synchronize()
    log(f"gqa head split {shape} workspace {need} B")
    ref = _bwd_through_abi(q, k, v, o, do, lse, 0)
    got = _bwd_through_abi(q, k, v, o, do, lse, need)
    assert torch.equal(got[0], ref[0])
    if Hkv == H:  # the Python layer takes the split for this shape
        assert all(torch.equal(a, b) for a, b in zip(mha, got))
    for g, r in zip(got[1:], ref[1:]):
        assert float((g.float() - r.float()).abs().max()) <= 2e-2 + 1e-2 * float(r.float().abs().max())
    again = _bwd_through_abi(q, k, v, o, do, lse, need)
    assert all(torch.equal(a, b) for a, b in zip(got, again))
    half = _bwd_through_abi(q, k, v, o, do, lse, need // 2)
    rows_only = _bwd_through_abi(q, k, v, o, do, lse, rows)  # dQ first, no split
    too_small = _bwd_through_abi(q, k, v, o, do, lse, rows - 256)  # holds neither part: as NULL
    assert all(torch.equal(a, b) for a, b in zip(too_small, ref))
    for out in (half, rows_only):
        assert torch.equal(out[0], ref[0])
        for g, r in zip(out[1:], ref[1:]):
            assert float((g.float() - r.float()).abs().max()) <= 2e-2 + 1e-2 * float(r.float().abs().max())


@pytest.mark.parametrize("shape", [(1, 8, 1, 1100, 128, "bf16"), (1, 16, 2, 2049, 128, "bf16"),
                                   (2, 8, 2, 3000, 128, "bf16"), (1, 8, 1, 1100, 128, "fp16")],
                         ids=lambda s: "B%dH%dHkv%dS%dD%d-%s" % s)
def test_dkdv_alternating_walk(shape):
    """The dK/dV walk (every D = 128 backward with a workspace takes it), whose even rounds run
    from the last query tile down, with the split's chunks interleaved (partial last
    tiles, splits of 57, 16 and 6 chunks here, bf16 and fp16; the unsplit walk is the full-size
    B2 H32 Hkv8 case): against the fp32 reference, against one workgroup summing each key tile's pairs in registers
    (no workspace), with a smaller split, and bitwise reproducible."""
    from attention import _lib
    from attention.backward.fused_backward import _forward
    B, H, Hkv, S, D, dt = shape
    q, k, v, do = make(B, H, Hkv, S, D, DTYPES[dt], seed=S + H)
    log(f"dkdv alternating walk {shape}")
    check(q, k, v, do, (128, 64), f"dkdv walk {shape}")
    o, lse = _forward(q, k, v, 128, 64)
    need = _lib.load().fa_bwd_gqa_workspace_size(B, H, Hkv, S, D)
    ref = _bwd_through_abi(q, k, v, o, do, lse, 0)
    got = _bwd_through_abi(q, k, v, o, do, lse, need)
    half = _bwd_through_abi(q, k, v, o, do, lse, need // 2)
    for out in (got, half):
        assert torch.equal(out[0], ref[0])
        for g, r in zip(out[1:], ref[1:]):
            assert float((g.float() - r.float()).abs().max()) <= 2e-2 + 1e-2 * float(r.float().abs().max())
    again = _bwd_through_abi(q, k, v, o, do, lse, need)
    assert all(torch.equal(a, b) for a, b in zip(got, again))


@pytest.mark.parametrize("shape", [(1, 4, 1, 2200), (3, 8, 2, 2500), (1, 32, 2, 700), (2, 24, 3, 1500),
                                   (1, 64, 1, 200), (1, 2, 1, 8193), (1, 1, 1, 9000), (4, 16, 4, 2100),
                                   (1, 2, 2, 8192), (1, 4, 2, 4096), (2, 8, 8, 1000), (1, 2, 2, 4096),
                                   (3, 4, 4, 333), (1, 1, 1, 64)],
                         ids=lambda s: "B%dH%dHkv%dS%d" % s)
def test_dkdv_alternating_walk_sweep(shape):
    """More shapes of the alternating dK/dV walk (D = 128 bf16, G from 1 to 64, S from 64 to 9000,
    splits of 2 to 64 chunks, MHA shapes small and large): equal to one workgroup summing each key
    tile's pairs in registers up to fp32 summation order, dQ identical."""
    from attention import _lib
    from attention.backward.fused_backward import _forward
    B, H, Hkv, S = shape
    D = 128
    q, k, v, do = make(B, H, Hkv, S, D, torch.bfloat16, seed=7 * S + H)
    log(f"dkdv alternating walk sweep {shape}")
    o, lse = _forward(q, k, v, 128, 64)
    need = _lib.load().fa_bwd_gqa_workspace_size(B, H, Hkv, S, D)
    ref = _bwd_through_abi(q, k, v, o, do, lse, 0)
    got = _bwd_through_abi(q, k, v, o, do, lse, need)
    assert torch.equal(got[0], ref[0])
    for g, r in zip(got[1:], ref[1:]):
        assert float((g.float() - r.float()).abs().max()) <= 2e-2 + 1e-2 * float(r.float().abs().max())
