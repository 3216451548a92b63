"""Host-side contract of the drop-in modules, on the CPU: validation, wrappers' argument
errors (raised before any device work), the unfused and reference backends."""

import math

import numpy as np
import pytest
import torch

from attention.fused.validation import ValidationError, validate_qkv, MAX_SEQ_LEN
from attention.gqa.validation_gqa import validate_qkv as validate_gqa
from attention.fused.fused import fused_attention
from attention.gqa.fused_gqa import fused_gqa_attention
from attention.backward.fused_backward import fused_attention_autograd, _check
from attention.fused.reference import causal_attention_reference, reference_attention
from attention.gqa.reference_gqa import causal_attention_reference_gqa
from attention.fused.unfused import unfused_attention
from attention.gqa.unfused_gqa import unfused_gqa_attention
from oracle import attention_oracle as orc


def arr(shape, dtype=np.float16):
    return np.zeros(shape, dtype=dtype)


def test_validate_accepts_widened_contract():
    validate_qkv(arr((1, 4, 256, 64)), arr((1, 4, 256, 64)), arr((1, 4, 256, 64)), 64, 64)
    validate_qkv(*(arr((1, 1, 16384, 64), np.float32),) * 3, 64, 128)
    q = torch.zeros(2, 2, 128, 128, dtype=torch.bfloat16)
    validate_qkv(q, q, q, 128, 64)
    assert MAX_SEQ_LEN >= 16384


@pytest.mark.parametrize("mutate,msg", [
    (lambda q, k, v: (q.astype(np.float64), k, v), "dtype"),
    (lambda q, k, v: (q, k.astype(np.float32), v), "share one dtype"),
    (lambda q, k, v: (q[0], k, v), "4-D"),
    (lambda q, k, v: (q, np.asfortranarray(k), v), "contiguous"),
    (lambda q, k, v: (q, np.ascontiguousarray(k[:, :2]), v), "head count"),
    (lambda q, k, v: (q, k, np.ascontiguousarray(v[:, :, :128])), "sequence length mismatch"),
    (lambda q, k, v: (q, k, np.ascontiguousarray(v[..., :32])), "head dim mismatch"),
])
def test_validate_rejections(mutate, msg):
    base = [arr((1, 4, 256, 64)) for _ in range(3)]
    with pytest.raises(ValidationError, match=msg):
        validate_qkv(*mutate(*base), 64, 64)


@pytest.mark.parametrize("shape,bm,bn,msg", [
    ((17, 1, 128, 64), 64, 64, "batch size"),
    ((1, 33, 128, 64), 64, 64, "head count"),
    ((1, 1, 128, 96), 64, 64, "head dim"),
    ((1, 1, 192, 64), 96, 64, "not supported"),
    ((1, 1, 128, 64), 0, 64, "not supported"),
    ((1, 1, 128, 64), 64, 32, "not supported"),
    ((1, 1, 2 * 65536, 32), 64, 64, "out of range"),
])
def test_validate_bounds(shape, bm, bn, msg):
    q = type("T", (), {"shape": shape, "dtype": np.dtype(np.float16), "flags": {"C_CONTIGUOUS": True}})()
    with pytest.raises(ValidationError, match=msg):
        validate_qkv(q, q, q, bm, bn)


def test_validate_accepts_any_sequence_length():
    # partial edge tiles: N need not be a multiple of either tile (the reference required it)
    for N in (1, 63, 100, 192, 4097):
        validate_qkv(arr((1, 2, N, 64)), arr((1, 2, N, 64)), arr((1, 2, N, 64)), 128, 64)
    assert validate_gqa(arr((1, 4, 100, 32)), arr((1, 2, 100, 32)), arr((1, 2, 100, 32)), 64, 128) == 2


def test_validate_gqa_group_and_errors():
    q = arr((2, 8, 128, 32))
    assert validate_gqa(q, arr((2, 2, 128, 32)), arr((2, 2, 128, 32)), 64, 64) == 4
    assert validate_gqa(q, arr((2, 8, 128, 32)), arr((2, 8, 128, 32)), 64, 64) == 1
    with pytest.raises(ValidationError, match="not divisible"):
        validate_gqa(q, arr((2, 3, 128, 32)), arr((2, 3, 128, 32)), 64, 64)
    with pytest.raises(ValidationError, match="K/V head count mismatch"):
        validate_gqa(q, arr((2, 2, 128, 32)), arr((2, 4, 128, 32)), 64, 64)
    with pytest.raises(ValidationError, match="out of range"):
        validate_gqa(arr((2, 2, 128, 32)), arr((2, 4, 128, 32)), arr((2, 4, 128, 32)), 64, 64)


def test_wrappers_raise_reference_errors_before_launch():
    q = torch.zeros(1, 2, 96, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="64 or 128"):
        fused_attention(q, q, q, 96, 64)
    with pytest.raises(ValueError, match="64 or 128"):
        fused_gqa_attention(q, q[:, :1], q[:, :1], 64, 32)
    with pytest.raises(ValueError, match="GQA needs"):
        fused_gqa_attention(q, q[:, :, :64], q[:, :, :64], 64, 64)
    with pytest.raises(TypeError):
        _check(q.float(), q.float(), q.float(), 64, 64)
    with pytest.raises(ValueError, match="64 or 128"):
        _check(q, q, q, 64, 256)
    _check(q, q, q, 128, 64)  # N = 96 is not a multiple of 128: fine, the edge tile is masked
    # on a CPU tensor the fused path refuses loudly instead of falling back
    q = torch.zeros(1, 2, 128, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        fused_attention(q, q, q, 64, 64)
    with pytest.raises(ValueError, match="GPU"):
        fused_attention_autograd(q, q, q, 64, 64)


def test_gqa_autograd_checks_before_launch():
    from attention.gqa.fused_gqa import fused_gqa_attention_autograd
    q = torch.zeros(1, 4, 128, 64, dtype=torch.float16)
    kv = torch.zeros(1, 2, 128, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="GQA needs"):
        fused_gqa_attention_autograd(q, q[:, :3].contiguous(), q[:, :3].contiguous(), 64, 64)
    with pytest.raises(ValueError, match="64 or 128"):
        fused_gqa_attention_autograd(q, kv, kv, 128, 256)
    with pytest.raises(TypeError):
        fused_gqa_attention_autograd(q.float(), kv.float(), kv.float(), 64, 64)
    with pytest.raises(ValueError, match="GPU"):
        fused_gqa_attention_autograd(q, kv, kv, 64, 64)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from attention import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(_lib.LibraryError, match="not found"):
        _lib.load()


def _inputs(B, H, Hkv, N, D, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, D, generator=g) * scale
    k = torch.randn(B, Hkv, N, D, generator=g) * scale
    v = torch.randn(B, Hkv, N, D, generator=g)
    return q, k, v


def test_reference_backends_match_oracle_on_cpu():
    q, k, v = _inputs(1, 4, 4, 128, 32, scale=2.0)
    want = orc.forward(q.numpy(), k.numpy(), v.numpy())
    np.testing.assert_allclose(causal_attention_reference(q, k, v).numpy(), want, atol=2e-5)
    np.testing.assert_allclose(reference_attention(q, k, v).numpy(), want, atol=2e-5)
    q, k, v = _inputs(2, 8, 2, 64, 16, seed=3)
    np.testing.assert_allclose(causal_attention_reference_gqa(q, k, v).numpy(),
                               orc.forward(q.numpy(), k.numpy(), v.numpy()), atol=2e-5)


def test_unfused_backends_match_oracle_on_cpu():
    q, k, v = _inputs(1, 2, 2, 128, 64, seed=5)
    o, S, P = unfused_attention(q.half(), k.half(), v.half(), 64, 64, return_intermediates=True)
    qh, kh, vh = (t.half().double().numpy() for t in (q, k, v))
    np.testing.assert_allclose(o.float().numpy(), orc.forward(qh, kh, vh), atol=2e-2)
    assert S.dtype == torch.float32 and P.dtype == torch.float16 and S.shape == (1, 2, 128, 128)
    assert torch.isinf(S[0, 0, 0, 1]) and float(P[0, 0, 0, 1]) == 0.0
    q, k, v = _inputs(1, 4, 1, 64, 32, seed=6)
    np.testing.assert_allclose(unfused_gqa_attention(q, k, v, 64, 64).numpy(),
                               orc.forward(q.numpy(), k.numpy(), v.numpy()), atol=2e-5)
    # the eager baseline has no tiles: any N, like the fused backends (here N = 64, tile 48)
    np.testing.assert_allclose(unfused_attention(q, q, q, 48, 64).numpy(),
                               orc.forward(q.numpy(), q.numpy(), q.numpy()), atol=2e-5)


def test_autograd_node_loads_without_a_gpu():
    """The C++ autograd node (fa_autograd, over libfa.so) is built in-tree and imports on a host
    without a GPU; the Python wrappers check their arguments before reaching it."""
    from attention import _lib
    mod = _lib.autograd()
    assert callable(mod.fused_attention)
    assert _lib.autograd() is mod
