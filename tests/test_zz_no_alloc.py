"""fa_bwd_gqa_noalloc: the backward with the library's own device scratch, through the C ABI.

The entry point has no counterpart in the reference; it serves callers that cannot
allocate device memory.  Its results must equal fa_bwd_gqa's given a caller workspace of
the scratch's size (fa_noalloc_scratch_bytes(), 64 MiB) -- bitwise, since both run the same
kernels with the same split -- on consecutive calls that reuse the scratch, one of them
smaller, including a shape whose full dK/dV split needs more than 64 MiB (it then runs the
largest split that fits, as fa_bwd_gqa does with that workspace).
"""

import ctypes
import math

import pytest
import torch

from attention import _lib
from gpu_util import log
from oracle import cases

pytestmark = pytest.mark.gpu

VP = ctypes.c_void_p


def ptr(t):
    return VP(t.data_ptr()) if t is not None else VP(0)


def make_case(B, H, Hkv, S, D, dtype, seed):
    q, do = (torch.from_numpy(x).cuda().to(dtype) for x in cases.normal_inputs([(B, H, S, D)] * 2, seed=seed))
    k, v = (torch.from_numpy(x).cuda().to(dtype) for x in cases.normal_inputs([(B, Hkv, S, D)] * 2, seed=seed + 1))
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device="cuda", dtype=torch.float32)
    _lib.fwd(q, k, v, o, lse, 64, 64)
    return q, k, v, o, do, lse


def run_bwd(lib, entry, case, tiles, workspace=None):
    q, k, v, o, do, lse = case
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    args = [ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse), ptr(dq), ptr(dk), ptr(dv),
            B, H, Hkv, S, D, _lib.dtype_code(q.dtype), _lib.scale_log2(D), 1.0 / math.sqrt(D), tiles[0], tiles[1]]
    stream = VP(torch.cuda.current_stream().cuda_stream)
    if entry == "noalloc":
        code = lib.fa_bwd_gqa_noalloc(*args, stream)
    else:
        code = lib.fa_bwd_gqa(*args, ptr(workspace), workspace.numel() if workspace is not None else 0, stream)
    assert code == _lib.FA_OK, _lib.strerror(code)
    return dq, dk, dv


# (B, H, H_kv, S, D, dtype, tiles), in call order: GQA whose full dK/dV split asks for more
# than 64 MiB of partial sums on a 256-CU device (per-row terms 1 MiB + 8 x 2 x 4096 x 128 x 4
# bytes per chunk), a smaller GQA shape that splits into many chunks, a small MHA shape, and
# the second one again after the small one
CALLS = [(1, 32, 8, 4096, 128, torch.bfloat16, (64, 64)), (2, 8, 2, 1000, 128, torch.bfloat16, (64, 64)),
         (1, 4, 4, 300, 64, torch.float16, (128, 64)), (2, 8, 2, 1000, 128, torch.bfloat16, (64, 64))]


def test_noalloc_backward_equals_workspace_backward_on_consecutive_calls():
    lib = _lib.load()
    cap = lib.fa_noalloc_scratch_bytes()
    assert cap == 64 << 20
    ws = torch.empty(cap, dtype=torch.uint8, device="cuda")  # the caller workspace of the same size
    for i, (B, H, Hkv, S, D, dtype, tiles) in enumerate(CALLS):
        split = lib.fa_bwd_dkdv_split(B, H, Hkv, S, D)
        need = lib.fa_bwd_gqa_workspace_size(B, H, Hkv, S, D)
        log(f"noalloc call {i}: B={B} H={H} H_kv={Hkv} S={S} D={D} {dtype} tiles={tiles} split={split} "
            f"full workspace {need} bytes ({'fits' if need <= cap else 'exceeds'} the {cap}-byte scratch)")
        case = make_case(B, H, Hkv, S, D, dtype, seed=10 + i % 3)
        want = run_bwd(lib, "workspace", case, tiles, ws)
        got = run_bwd(lib, "noalloc", case, tiles)
        torch.cuda.synchronize()
        for name, g, w in zip(("dQ", "dK", "dV"), got, want):
            assert torch.isfinite(g.float()).all(), name
            assert torch.equal(g, w), f"{name} differs from fa_bwd_gqa's with a {cap}-byte workspace (call {i})"
        log(f"noalloc call {i}: bitwise equal to fa_bwd_gqa with a {cap}-byte workspace")


def test_noalloc_runs_shapes_past_the_full_split():
    """The first call's shape asks for more workspace than the scratch holds (the premise of
    the test above); its results still match the fp32 autograd of the reference formula."""
    from oracle.cpu_reference import reference_grads_gqa
    lib = _lib.load()
    B, H, Hkv, S, D, dtype, tiles = CALLS[0]
    assert lib.fa_bwd_gqa_workspace_size(B, H, Hkv, S, D) > lib.fa_noalloc_scratch_bytes()
    case = make_case(B, H, Hkv, S, D, dtype, seed=10)
    dq, dk, dv = run_bwd(lib, "noalloc", case, tiles)
    torch.cuda.synchronize()
    q, k, v, o, do, lse = case
    g = H // Hkv
    # the first and the last K/V head with their query heads: fp32 autograd on the CPU
    for kh in (0, Hkv - 1):
        hs = slice(kh * g, (kh + 1) * g)
        _, rq, rk, rv = reference_grads_gqa(*(t.float().cpu() for t in (q[:, hs], k[:, kh:kh + 1],
                                                                         v[:, kh:kh + 1], do[:, hs])))
        gq, gk, gv = (t.float().cpu() for t in (dq[:, hs], dk[:, kh:kh + 1], dv[:, kh:kh + 1]))
        eq, ek, ev = (float((x - r).abs().max()) for x, r in ((gq, rq), (gk, rk), (gv, rv)))
        log(f"noalloc past the full split, K/V head {kh}: dQ {eq:.3e} dK {ek:.3e} dV {ev:.3e}")
        assert eq <= 2e-2
        # dK / dV of a K/V head sum G heads' bf16 gradients: the reference's mixed bar
        # (tests/fused/run_correctness.py:33-34), as in the GQA backward suite
        assert bool(((gk - rk).abs() <= 2e-2 + 2e-2 * rk.abs()).all())
        assert bool(((gv - rv).abs() <= 2e-2 + 2e-2 * rv.abs()).all())
