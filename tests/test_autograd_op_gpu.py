"""The C++ autograd node behind fused_attention_autograd / fused_gqa_attention_autograd.

It runs the forward and backward of the Python autograd Functions (FusedAttentionFn,
FusedGQAAttentionFn: the reference's interface, attention/backward/fused_backward.py:151-206)
through the same C entry points with the same arguments, so O and every gradient must equal
theirs bitwise; the gradients' accuracy against the fp32 reference is what the backward suites
(tests/test_bwd_gpu.py, tests/test_gqa_bwd_gpu.py) check through the same node.
"""

import pytest
import torch

from attention import _lib
from attention.backward.fused_backward import FusedAttentionFn, fused_attention_autograd
from attention.gqa.fused_gqa import FusedGQAAttentionFn, fused_gqa_attention_autograd
from oracle import cases
from tests.gpu_util import log

pytestmark = pytest.mark.gpu


def _inputs(B, H, Hkv, S, D, dtype, seed):
    q, do = (torch.from_numpy(x).cuda().to(dtype) for x in cases.normal_inputs([(B, H, S, D)] * 2, seed=seed))
    k, v = (torch.from_numpy(x).cuda().to(dtype) for x in cases.normal_inputs([(B, Hkv, S, D)] * 2, seed=seed + 1))
    return q, k, v, do


def _grads(fn, q, k, v, do, tiles):
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    o = fn(*leaves, *tiles)
    o.backward(do)
    torch.cuda.synchronize()
    return [o.detach()] + [t.grad for t in leaves]


CASES = [  # (B, H, H_kv, S, D, dtype, tiles)
    (2, 8, 8, 128, 64, torch.float16, (64, 64)),
    (1, 4, 4, 1000, 128, torch.bfloat16, (128, 64)),
    (2, 3, 3, 257, 32, torch.float16, (64, 128)),
    (1, 8, 2, 700, 128, torch.bfloat16, (64, 64)),     # GQA
    (1, 16, 1, 513, 64, torch.float16, (128, 128)),    # MQA, dK/dV split
    (4, 32, 32, 4096, 128, torch.bfloat16, (128, 64)), # the headline shape
]


@pytest.mark.parametrize("B,H,Hkv,S,D,dtype,tiles", CASES)
def test_node_equals_python_function_bitwise(B, H, Hkv, S, D, dtype, tiles):
    q, k, v, do = _inputs(B, H, Hkv, S, D, dtype, seed=S + D + H)
    log(f"autograd node vs Python Function B={B} H={H} H_kv={Hkv} S={S} D={D} {dtype} tiles={tiles}")
    if Hkv == H:
        want = _grads(FusedAttentionFn.apply, q, k, v, do, tiles)
        got = _grads(fused_attention_autograd, q, k, v, do, tiles)
    else:
        want = _grads(FusedGQAAttentionFn.apply, q, k, v, do, tiles)
        got = _grads(fused_gqa_attention_autograd, q, k, v, do, tiles)
    for name, g, w in zip(("O", "dQ", "dK", "dV"), got, want):
        assert g.dtype == w.dtype and g.shape == w.shape, name
        assert torch.equal(g, w), f"{name} of the C++ node differs from the Python Function's"


def test_node_on_a_side_stream_and_non_contiguous_inputs():
    """Work goes to the caller's current stream; inputs that are views (a transposed layout made
    contiguous by the node) give the results of their contiguous copies; gradients accumulate
    over two backward passes into the same leaves."""
    B, H, S, D = 1, 4, 300, 64
    q, k, v, do = _inputs(B, H, H, S, D, torch.float16, seed=5)
    want = _grads(FusedAttentionFn.apply, q, k, v, do, (64, 64))
    # the same values held as [B, S, H, D] and viewed as [B, H, S, D]
    views = [t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v)]
    assert not views[0].is_contiguous()
    leaves = [t.detach().requires_grad_(True) for t in views]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        o = fused_attention_autograd(*leaves, 64, 64)
        o.backward(do)
        o2 = fused_attention_autograd(*leaves, 64, 64)
        o2.backward(do)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(o.detach(), want[0])
    for name, leaf, w in zip(("dQ", "dK", "dV"), leaves, want[1:]):
        assert torch.equal(leaf.grad, (w.float() + w.float()).to(w.dtype)), name


def test_node_keeps_the_reference_errors():
    q = torch.zeros(1, 4, 128, 64, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError):
        fused_attention_autograd(q, q[:, :2].contiguous(), q[:, :2].contiguous())
    with pytest.raises(TypeError):
        fused_attention_autograd(q.float(), q.float(), q.float())
    with pytest.raises(ValueError):
        fused_attention_autograd(q, q, q, 96, 64)
    with pytest.raises(ValueError):
        fused_gqa_attention_autograd(q, q[:, :3].contiguous(), q[:, :3].contiguous())
    assert hasattr(_lib.autograd(), "fused_attention")
