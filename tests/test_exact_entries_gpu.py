"""fa_fwd_exact and fa_bwd_gqa_exact on the GPU, through the C ABI.

These entry points (used by the tile study, no reference counterpart) run kernel instances
the dispatch rules never reach: 64-row forward workgroups of one head, one, two or four GQA
heads per workgroup where the rule picks another count (two heads of 128 rows where it takes
four of 64), 64-row dQ workgroups, and any dK/dV split from 1 to 64 -- including more chunks
than the heaviest key tile has (query tile, head) pairs, where some chunks are empty and store
zero partial sums.

Claims checked:
* the workgroup shape does not change a result: a 32-row wave runs the same arithmetic over
  the same key tiles whatever its workgroup holds, so O, LSE and dQ equal the dispatching
  entries' bitwise, and so do dK and dV at the same split;
* a split changes only the fp32 summation order of dK and dV: every split matches the
  unsplit result to that order (a few bf16 / fp16 units) and the fp32 reference within the
  suites' bars;
* without a workspace the exact entry runs the dK/dV kernel that forms Delta itself (no other
  entry point reaches it): dQ unchanged, dK and dV within the same bars.
"""

import ctypes
import math

import pytest
import torch

from attention import _lib
from gpu_util import log
from oracle import cases
from oracle.cpu_reference import reference_grads_gqa

pytestmark = pytest.mark.gpu

VP = ctypes.c_void_p


def ptr(t):
    return VP(t.data_ptr()) if t is not None else VP(0)


def stream():
    return VP(torch.cuda.current_stream().cuda_stream)


def inputs(B, H, Hkv, S, D, dtype, seed):
    q, do = (torch.from_numpy(x).cuda().to(dtype) for x in cases.normal_inputs([(B, H, S, D)] * 2, seed=seed))
    k, v = (torch.from_numpy(x).cuda().to(dtype) for x in cases.normal_inputs([(B, Hkv, S, D)] * 2, seed=seed + 1))
    return q, k, v, do


def fwd(lib, q, k, v, bm, bn, gh=None):
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    o = torch.full_like(q, float("nan"))
    lse = torch.full((B, H, S), float("nan"), device="cuda")
    args = [ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, H, Hkv, S, D, _lib.dtype_code(q.dtype), _lib.scale_log2(D),
            bm, bn]
    code = lib.fa_fwd(*args, stream()) if gh is None else lib.fa_fwd_exact(*args, gh, stream())
    assert code == _lib.FA_OK, _lib.strerror(code)
    return o, lse


def rowb_bytes(B, H, S):
    return (8 * B * H * S + 255) // 256 * 256


def bwd(lib, q, k, v, o, do, lse, bm, bn, nsplit=None, workspace=True):
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
    args = [ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse), ptr(dq), ptr(dk), ptr(dv), B, H, Hkv, S, D,
            _lib.dtype_code(q.dtype), _lib.scale_log2(D), 1.0 / math.sqrt(D), bm, bn]
    if nsplit is None:
        n = lib.fa_bwd_gqa_workspace_size(B, H, Hkv, S, D)
        ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        code = lib.fa_bwd_gqa(*args, ptr(ws), n, stream())
    else:
        n = rowb_bytes(B, H, S) + (8 * B * Hkv * nsplit * S * D if nsplit > 1 else 0) if workspace else 0
        ws = torch.empty(n, dtype=torch.uint8, device="cuda") if workspace else None
        code = lib.fa_bwd_gqa_exact(*args, nsplit, ptr(ws), n, stream())
    assert code == _lib.FA_OK, _lib.strerror(code)
    torch.cuda.synchronize()
    return dq, dk, dv


FWD_CASES = [  # (B, H, H_kv, S, D, dtype)
    (1, 4, 4, 1000, 128, torch.bfloat16), (2, 2, 2, 777, 64, torch.float16),
    (1, 8, 2, 1000, 128, torch.bfloat16), (1, 8, 2, 333, 64, torch.float16), (1, 8, 1, 500, 32, torch.bfloat16),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,dtype", FWD_CASES)
def test_forward_exact_shapes_equal_dispatch_bitwise(B, H, Hkv, S, D, dtype):
    lib = _lib.load()
    q, k, v, _ = inputs(B, H, Hkv, S, D, dtype, seed=S + D)
    o_ref, lse_ref = fwd(lib, q, k, v, 64, 64)
    g = H // Hkv
    shapes = [(64, 64, gh) for gh in (1, 2, 4) if g % gh == 0] + [(128, 64, gh) for gh in (1, 2) if g % gh == 0]
    shapes += [(64, 128, 1)]
    for bm, bn, gh in shapes:
        if bn == 128 and not lib.fa_supported(_lib.dtype_code(dtype), D, bm, bn, 1, 1, 0):
            continue
        if bn != 64:  # a different key tile sums P over other blocks: compare to the 64-key tile's tiles
            o_b, lse_b = fwd(lib, q, k, v, 64, bn)
        else:
            o_b, lse_b = o_ref, lse_ref
        o, lse = fwd(lib, q, k, v, bm, bn, gh)
        torch.cuda.synchronize()
        log(f"fwd exact {bm}x{bn} gh={gh} B={B} H={H} H_kv={Hkv} S={S} D={D}: "
            f"O maxdiff {float((o.float() - o_b.float()).abs().max()):.3g}")
        assert torch.equal(o, o_b), f"O of {bm}x{bn} with {gh} heads per workgroup"
        assert torch.equal(lse, lse_b), f"LSE of {bm}x{bn} with {gh} heads per workgroup"


@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.float16)])
def test_forward_gqa_tile_as_four_heads_bitwise(D, dtype):
    """A 128-row, 64-key GQA tile runs as 64-row workgroups of four heads where the grid is large
    enough (512 workgroups here, two per CU on a 256-CU device): the same O and LSE as two heads
    of 128 rows and as four heads of 64."""
    lib = _lib.load()
    B, H, Hkv, S = 2, 8, 2, 8192
    q, k, v, _ = inputs(B, H, Hkv, S, D, dtype, seed=D)
    gh = lib.fa_fwd_heads_per_wg(B, H, Hkv, S, D, 128, 64)
    rows = lib.fa_fwd_rows_per_wg(128, 64, D, gh)
    o, lse = fwd(lib, q, k, v, 128, 64)
    for bm, g in ((128, 2), (64, 4)):
        o_x, lse_x = fwd(lib, q, k, v, bm, 64, g)
        torch.cuda.synchronize()
        log(f"fwd 128x64 dispatch ({gh} heads of {rows} rows) vs exact {g} heads of {bm} rows, D={D}: "
            f"O maxdiff {float((o.float() - o_x.float()).abs().max()):.3g}")
        assert torch.equal(o, o_x) and torch.equal(lse, lse_x), f"{g} heads of {bm} rows"


BWD_CASES = [  # (B, H, H_kv, S, D, dtype): paired dK/dV at D = 128, one-wave at D <= 64
    (1, 4, 2, 1000, 128, torch.bfloat16), (1, 4, 1, 700, 64, torch.float16), (1, 4, 2, 600, 32, torch.bfloat16),
]


@pytest.mark.parametrize("B,H,Hkv,S,D,dtype", BWD_CASES)
def test_backward_exact_shapes_and_splits(B, H, Hkv, S, D, dtype):
    lib = _lib.load()
    q, k, v, do = inputs(B, H, Hkv, S, D, dtype, seed=3 * S + D)
    o, lse = fwd(lib, q, k, v, 64, 64)
    base_split = lib.fa_bwd_dkdv_split(B, H, Hkv, S, D)
    want = bwd(lib, q, k, v, o, do, lse, 64, 64)
    # dQ rows per workgroup: the exact 64-row dQ against the dispatch's (128 rows)
    got = bwd(lib, q, k, v, o, do, lse, 64, 64, nsplit=base_split)
    for name, g_, w in zip(("dQ", "dK", "dV"), got, want):
        assert torch.equal(g_, w), f"{name}: 64-row dQ workgroups at the dispatch's split {base_split}"
    # the fp32 reference (autograd of the formula on repeated K/V, group sums)
    _, rq, rk, rv = reference_grads_gqa(*(t.float().cpu() for t in (q, k, v, do)))
    g = H // Hkv
    pairs = g * ((S + 63) // 64)  # the heaviest key tile's (query tile, head) pairs
    for nsplit in (1, 2, 7, pairs, min(64, pairs + 5), 64):
        dq, dk, dv = bwd(lib, q, k, v, o, do, lse, 64, 64, nsplit=nsplit)
        assert torch.equal(dq, want[0]), "dQ does not depend on the dK/dV split"
        dd = max(float((dk.float() - want[1].float()).abs().max()), float((dv.float() - want[2].float()).abs().max()))
        ek = float((dk.float().cpu() - rk).abs().max())
        ev = float((dv.float().cpu() - rv).abs().max())
        log(f"bwd exact split {nsplit} (heaviest tile {pairs} pairs) B={B} H={H} H_kv={Hkv} S={S} D={D} {dtype}: "
            f"vs unsplit {dd:.3g}, vs fp32 dK {ek:.3g} dV {ev:.3g}")
        # only the fp32 order of the partial sums changes: a few units of the 16-bit output
        assert dd <= 8 * 2.0 ** -7 * max(1.0, float(rk.abs().max()), float(rv.abs().max()))
        for got_t, ref in ((dk, rk), (dv, rv)):
            err = (got_t.float().cpu() - ref).abs()
            assert bool((err <= 2e-2 + 2e-2 * ref.abs()).all()), f"split {nsplit} against the fp32 reference"
    assert float((dq.float().cpu() - rq).abs().max()) <= 2e-2
    # no workspace: the dK/dV kernel forms each row's Delta from the O and dO tiles of every key
    # tile it meets, in another fp32 order than the dQ kernel's (and, at D = 128, from dP
    # rounded once more); dQ runs after it and is unchanged
    dq, dk, dv = bwd(lib, q, k, v, o, do, lse, 64, 64, nsplit=1, workspace=False)
    assert torch.equal(dq, want[0]), "dQ with the Delta-forming dK/dV"
    dd = max(float((dk.float() - want[1].float()).abs().max()), float((dv.float() - want[2].float()).abs().max()))
    log(f"bwd exact, no workspace B={B} H={H} H_kv={Hkv} S={S} D={D} {dtype}: vs unsplit {dd:.3g}")
    assert dd <= 8 * 2.0 ** -7 * max(1.0, float(rk.abs().max()), float(rv.abs().max()))
    for got_t, ref in ((dk, rk), (dv, rv)):
        err = (got_t.float().cpu() - ref).abs()
        assert bool((err <= 2e-2 + 2e-2 * ref.abs()).all()), "Delta-forming dK/dV against the fp32 reference"
