"""The longest sequences the validated contract admits (N up to 65536; the reference stops at
8192): forward and GQA forward at N = 65536, checked row by row against the float64 oracle on
sampled rows (the full fp32 reference would need 16 GiB per score matrix), and the backward at
N = 32768 against fp32 autograd of the reference formula.  Odd lengths one past a tile multiple
are included, so the partial last tiles are exercised at full scale too."""

import numpy as np
import pytest
import torch

from attention.backward.fused_backward import fused_attention_autograd
from attention.fused.fused import fused_attention
from attention.gqa.fused_gqa import fused_gqa_attention
from oracle import attention_oracle as orc
from oracle import cases
from oracle.cpu_reference import reference_grads
from tests.gpu_util import dev, log

pytestmark = pytest.mark.gpu


def _oracle_rows(out, q, k, v, heads, rows):
    g = q.shape[1] // k.shape[1]
    worst = 0.0
    for h in heads:
        want = orc.forward(q[:1, h:h + 1].double().cpu().numpy(), k[:1, h // g:h // g + 1].double().cpu().numpy(),
                           v[:1, h // g:h // g + 1].double().cpu().numpy(), rows)
        got = out[:1, h:h + 1, rows].double().cpu().numpy()
        worst = max(worst, float(np.abs(got - want).max()))
    return worst


@pytest.mark.parametrize("N", [65536, 65535])
def test_forward_max_length(N):
    q, k, v = (dev(x, torch.bfloat16) for x in cases.normal_inputs([(1, 2, N, 128)] * 3, seed=5))
    log(f"max-length forward N={N}")
    o = fused_attention(q, k, v, 128, 64)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    assert torch.equal(o[:, :, 0], v[:, :, 0])
    rows = orc.sample_rows(N, count=24)
    worst = _oracle_rows(o, q, k, v, (0, 1), rows)
    log(f"  oracle rows max_abs={worst:.3e}")
    assert worst <= 2e-2


def test_gqa_forward_max_length():
    N = 65536
    q = dev(cases.normal_inputs([(1, 4, N, 64)], seed=6)[0], torch.float16)
    k, v = (dev(x, torch.float16) for x in cases.normal_inputs([(1, 1, N, 64)] * 2, seed=7))
    log("max-length MQA forward N=65536")
    o = fused_gqa_attention(q, k, v, 128, 64)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    worst = _oracle_rows(o, q, k, v, (0, 3), orc.sample_rows(N, count=16))
    log(f"  oracle rows max_abs={worst:.3e}")
    assert worst <= 2e-2


@pytest.mark.parametrize("N", [32768, 32769])
def test_backward_long(N):
    q, k, v, do = (dev(x, torch.bfloat16) for x in cases.normal_inputs([(1, 1, N, 64)] * 4, seed=N))
    log(f"long backward N={N}")
    qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = fused_attention_autograd(qg, kg, vg, 128, 64)
    o.backward(do)
    torch.cuda.synchronize()
    ref = reference_grads(q, k, v, do)
    for name, g, r in zip(("O", "dQ", "dK", "dV"), (o.detach(), qg.grad, kg.grad, vg.grad), ref):
        assert torch.isfinite(g).all(), name
        a = float((g.float() - r).abs().max())
        rel = float((g.float() - r).norm() / r.norm())
        log(f"  {name}: max_abs={a:.3e} rel={rel:.2e}")
        assert a <= 2e-2 and rel <= 2e-2, (name, a, rel)
    del ref
    torch.cuda.empty_cache()
