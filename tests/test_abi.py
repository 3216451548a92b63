"""The C ABI of libfa.so, checked without a GPU.

The library must load, export every function include/fa.h declares, and reject
bad arguments with the documented status codes before touching the device.
"""

import ctypes
import os
import re

import pytest

from attention import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "fa.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z_]+)\s*\(", text)))


def test_header_declares_the_bound_signatures():
    assert header_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_header_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name
    assert lib.fa_version() >= 100


def test_no_internal_symbols_leak():
    out = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert {"fa_fwd", "fa_bwd", "fa_bwd_gqa", "fa_supported", "fa_strerror", "fa_version"} <= exported
    assert not any(s.startswith("fa_fwd_table") or s.startswith("fa_bwd_table") for s in exported)


def test_strerror_covers_every_status(lib):
    for code in range(0, -10, -1):
        assert lib.fa_strerror(code).decode() not in ("", "unknown status")
    assert lib.fa_strerror(-99).decode() == "unknown status"


NULL = ctypes.c_void_p(0)
# never dereferenced: every case below fails argument validation before any launch (any S
# is valid, so none of them may rely on S alone being rejected)
FAKE = ctypes.c_void_p(0x1000)


def fwd(lib, B=1, H=2, Hkv=2, S=256, D=64, dtype=1, bm=64, bn=64, ptr=FAKE, lse=NULL):
    return lib.fa_fwd(ptr, ptr, ptr, ptr, lse, B, H, Hkv, S, D, dtype, 0.1, bm, bn, NULL)


def bwd(lib, B=1, H=2, S=256, D=64, dtype=0, bm=64, bn=64, ptr=FAKE):
    return lib.fa_bwd(ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, B, H, S, D, dtype, 0.1, 0.1, bm, bn, NULL)


@pytest.mark.parametrize("kw,code", [
    (dict(B=0), _lib.FA_ERR_DIMS),
    (dict(S=-64), _lib.FA_ERR_DIMS),
    (dict(Hkv=3), _lib.FA_ERR_DIMS),
    (dict(Hkv=4), _lib.FA_ERR_DIMS),
    (dict(dtype=2), _lib.FA_ERR_DTYPE),
    (dict(D=48), _lib.FA_ERR_HEADDIM),
    (dict(D=256), _lib.FA_ERR_HEADDIM),
    (dict(bm=32), _lib.FA_ERR_TILE),
    (dict(bn=256), _lib.FA_ERR_TILE),
    (dict(bm=96), _lib.FA_ERR_TILE),
    (dict(ptr=NULL), _lib.FA_ERR_NULL),
])
def test_fwd_rejects_bad_arguments(lib, kw, code):
    assert fwd(lib, **kw) == code


@pytest.mark.parametrize("S,D", [(1 << 23, 128), (1 << 24, 64), (1 << 25, 32), ((1 << 23) + 5, 128)])
def test_rows_of_one_head_past_2gib_are_rejected(lib, S, D):
    """S * D * 2 bytes of one (batch, head) slice must stay below 2^31: the kernels form
    byte offsets and tile sizes inside a slice in 32-bit int.  B = H = 1 keeps B*H*S legal."""
    assert fwd(lib, B=1, H=1, Hkv=1, S=S, D=D) == _lib.FA_ERR_DIMS
    assert bwd(lib, B=1, H=1, S=S, D=D) == _lib.FA_ERR_DIMS
    assert bwd_gqa(lib, B=1, H=1, Hkv=1, S=S, D=D) == _lib.FA_ERR_DIMS


@pytest.mark.parametrize("kw,code", [
    (dict(H=0), _lib.FA_ERR_DIMS),
    (dict(dtype=7), _lib.FA_ERR_DTYPE),
    (dict(D=96), _lib.FA_ERR_HEADDIM),
    (dict(bn=192), _lib.FA_ERR_TILE),
    (dict(ptr=NULL), _lib.FA_ERR_NULL),
])
def test_bwd_rejects_bad_arguments(lib, kw, code):
    assert bwd(lib, **kw) == code


def bwd_gqa(lib, B=1, H=4, Hkv=2, S=256, D=64, dtype=1, bm=64, bn=64, ptr=FAKE, ws=NULL, ws_bytes=0):
    return lib.fa_bwd_gqa(ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, B, H, Hkv, S, D, dtype, 0.1, 0.1,
                          bm, bn, ws, ws_bytes, NULL)


@pytest.mark.parametrize("kw,code", [
    (dict(Hkv=3), _lib.FA_ERR_DIMS),
    (dict(Hkv=0), _lib.FA_ERR_DIMS),
    (dict(Hkv=8), _lib.FA_ERR_DIMS),
    (dict(B=-1), _lib.FA_ERR_DIMS),
    (dict(dtype=5), _lib.FA_ERR_DTYPE),
    (dict(D=80), _lib.FA_ERR_HEADDIM),
    (dict(bm=256), _lib.FA_ERR_TILE),
    (dict(ptr=NULL), _lib.FA_ERR_NULL),
    (dict(ws=ctypes.c_void_p(0x1004), ws_bytes=1 << 20), _lib.FA_ERR_WORKSPACE),
])
def test_bwd_gqa_rejects_bad_arguments(lib, kw, code):
    assert bwd_gqa(lib, **kw) == code


def rowb(B, H, S):
    """-LSE/c and -Delta per query row: 8 * B * H * S bytes rounded up to 256."""
    return (8 * B * H * S + 255) // 256 * 256


def test_bwd_gqa_workspace_size(lib):
    """The per-row terms, then fp32 partial dK and dV per chunk: 2 * B * H_kv * nsplit * S * D * 4
    bytes, with nsplit the chunks per 128-key tile that give two work items per dK/dV workgroup
    slot (the paired D = 128 kernel: one per CU, 256; the one-wave kernel at D <= 64: two per CU)
    times ceil(S / 8192), at most the heaviest key tile's (query tile, query head) pairs and 64
    (no split below 64 pairs)."""
    ws = lib.fa_bwd_gqa_workspace_size
    assert ws(2, 32, 32, 4096, 128) == rowb(2, 32, 4096)              # 2*32*32 key tiles: no split
    assert ws(2, 32, 8, 4096, 128) == rowb(2, 32, 4096)               # 2*8*32 = 512 items already
    assert ws(1, 8, 8, 4096, 128) == rowb(1, 8, 4096) + 2 * 8 * 2 * 4096 * 128 * 4  # MHA, 256 key tiles: 2 chunks
    assert ws(1, 32, 1, 4096, 64) == rowb(1, 32, 4096) + 2 * 32 * 4096 * 64 * 4   # MQA: 32 key tiles x 32 chunks
    # S = 8192, D = 128: target 512, 4 x 64 key tiles -> 2 chunks
    assert ws(1, 32, 4, 8192, 128) == rowb(1, 32, 8192) + 2 * 4 * 2 * 8192 * 128 * 4
    # S = 16384: target 2 x 512 (D = 128), 8 x 128 key tiles -> 8 chunks
    assert ws(1, 8, 1, 16384, 128) == rowb(1, 8, 16384) + 2 * 8 * 16384 * 128 * 4
    assert ws(1, 6, 2, 100, 32) == rowb(1, 6, 100)                    # 3 heads x 2 query tiles: too short to split
    assert ws(1, 32, 1, 200, 32) == rowb(1, 32, 200) + 2 * 64 * 200 * 32 * 4  # 2 key tiles of 32 x 4 pairs: 64 chunks (the cap)
    assert ws(2, 8, 8, 2048, 128) == rowb(2, 8, 2048)                 # 32 pairs per key tile: not worth a split
    assert ws(1, 1, 1, 64, 64) == rowb(1, 1, 64)                      # one pair: nothing to split
    for bad in ((0, 4, 2, 256, 64), (1, 4, 3, 256, 64), (1, 4, 2, 0, 64), (1, 4, 2, 256, 48)):
        assert ws(*bad) == 0


def test_supported_table(lib):
    for dtype in (0, 1):
        for D in (32, 64, 128):
            for bm in (64, 128):
                for bn in (64, 128):
                    assert lib.fa_supported(dtype, D, bm, bn, 1, 0, 0) == 1
                    assert lib.fa_supported(dtype, D, bm, bn, 1, 1, 0) == 1
                    for group in (2, 4, 8, 32):
                        assert lib.fa_supported(dtype, D, bm, bn, group, 0, 0) == 1
                        assert lib.fa_supported(dtype, D, bm, bn, group, 1, 1) == 1
    assert lib.fa_supported(1, 128, 64, 64, 0, 0, 0) == 0
    assert lib.fa_supported(1, 96, 64, 64, 1, 0, 0) == 0


def test_error_mapping_to_reference_exceptions():
    with pytest.raises(TypeError):
        _lib.check(_lib.FA_ERR_DTYPE, "x")
    for code in (_lib.FA_ERR_DIMS, _lib.FA_ERR_HEADDIM, _lib.FA_ERR_TILE, _lib.FA_ERR_UNSUPPORTED):
        with pytest.raises(ValueError):
            _lib.check(code, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.FA_ERR_LAUNCH, "x")
    _lib.check(_lib.FA_OK, "x")


def test_no_unresolved_library_symbols():
    """Every kernel launch stub is defined inside the library (none left for the loader)."""
    out = os.popen(f"nm -D --undefined-only {_lib.LIB_PATH}").read()
    missing = [line.split()[-1] for line in out.splitlines() if "_ZN2fa" in line]
    assert not missing, missing[:5]


def test_noalloc_entry_rejects_shapes_past_its_scratch(lib):
    """fa_bwd_gqa_noalloc: argument errors as fa_bwd_gqa, and FA_ERR_SCRATCH -- before any
    launch -- when the shape's per-row terms (8 * B * H * S bytes) exceed the library's 64 MiB
    device scratch.  A shape whose full dK/dV split would not fit behind them is accepted
    and runs a smaller split (tests/test_zz_no_alloc.py, on the GPU)."""
    assert lib.fa_noalloc_scratch_bytes() == 64 << 20

    def noalloc(B=1, H=4, Hkv=2, S=256, D=64, dtype=1, bm=64, bn=64, ptr=FAKE):
        return lib.fa_bwd_gqa_noalloc(ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, B, H, Hkv, S, D, dtype,
                                      0.1, 0.1, bm, bn, NULL)
    assert noalloc(Hkv=3) == _lib.FA_ERR_DIMS
    assert noalloc(dtype=4) == _lib.FA_ERR_DTYPE
    assert noalloc(D=40) == _lib.FA_ERR_HEADDIM
    assert noalloc(bn=32) == _lib.FA_ERR_TILE
    assert noalloc(ptr=NULL) == _lib.FA_ERR_NULL
    assert noalloc(S=1 << 25, D=32, H=1, Hkv=1) == _lib.FA_ERR_DIMS
    # 4 * 32 * 65537 rows: 67,109,888 bytes of per-row terms, one row past the 8M that fit
    assert noalloc(B=4, H=32, Hkv=32, S=65537) == _lib.FA_ERR_SCRATCH
    assert noalloc(B=4, H=32, Hkv=32, S=65537, D=128) == _lib.FA_ERR_SCRATCH
    assert "scratch" in lib.fa_strerror(_lib.FA_ERR_SCRATCH).decode()


def test_exact_shape_entries_and_rule_queries(lib):
    """The study entry points reject what their kernels cannot run, before any launch, and the
    rule queries return the dispatch choices of fa_fwd / fa_bwd_gqa."""
    def fwd_exact(B=1, H=8, Hkv=2, S=256, D=64, dtype=1, bm=64, bn=64, gh=1, ptr=FAKE):
        return lib.fa_fwd_exact(ptr, ptr, ptr, ptr, NULL, B, H, Hkv, S, D, dtype, 0.1, bm, bn, gh, NULL)
    assert fwd_exact(gh=0) == _lib.FA_ERR_DIMS
    assert fwd_exact(gh=3) == _lib.FA_ERR_DIMS       # does not divide the group of 4
    assert fwd_exact(H=8, Hkv=4, gh=4) == _lib.FA_ERR_DIMS  # group of 2
    assert fwd_exact(bm=128, bn=128, gh=2) == _lib.FA_ERR_UNSUPPORTED
    assert fwd_exact(bm=128, bn=64, gh=4) == _lib.FA_ERR_UNSUPPORTED
    assert fwd_exact(bn=96) == _lib.FA_ERR_TILE
    assert fwd_exact(ptr=NULL) == _lib.FA_ERR_NULL

    def bwd_exact(B=1, H=4, Hkv=2, S=256, D=64, dtype=1, bm=64, bn=64, nsplit=1, ws=NULL, ws_bytes=0, ptr=FAKE):
        return lib.fa_bwd_gqa_exact(ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, B, H, Hkv, S, D, dtype, 0.1, 0.1,
                                    bm, bn, nsplit, ws, ws_bytes, NULL)
    assert bwd_exact(nsplit=0) == _lib.FA_ERR_DIMS
    assert bwd_exact(nsplit=65) == _lib.FA_ERR_DIMS
    assert bwd_exact(nsplit=2) == _lib.FA_ERR_WORKSPACE          # a split needs its partial sums
    need = rowb(1, 4, 256) + 2 * 1 * 2 * 2 * 256 * 64 * 4
    assert bwd_exact(nsplit=2, ws=ctypes.c_void_p(0x10000), ws_bytes=need - 16) == _lib.FA_ERR_WORKSPACE
    assert bwd_exact(bm=96) == _lib.FA_ERR_TILE
    assert bwd_exact(ptr=NULL) == _lib.FA_ERR_NULL

    # the rules, as documented beside them in fa_api.hip
    assert lib.fa_fwd_rows_per_wg(64, 64, 128, 1) == 128 and lib.fa_fwd_rows_per_wg(64, 128, 128, 1) == 128
    assert lib.fa_fwd_rows_per_wg(64, 128, 64, 1) == 128 and lib.fa_fwd_rows_per_wg(64, 64, 32, 2) == 64
    assert lib.fa_bwd_dq_rows_per_wg(64, 128) == 128 and lib.fa_bwd_dq_rows_per_wg(64, 64) == 128
    assert lib.fa_bwd_dq_rows_per_wg(64, 32) == 128 and lib.fa_bwd_dq_rows_per_wg(128, 32) == 128
    assert lib.fa_fwd_heads_per_wg(4, 32, 32, 4096, 128, 128, 64) == 1
    assert lib.fa_fwd_heads_per_wg(2, 32, 8, 8192, 128, 64, 64) == 4
    assert lib.fa_fwd_heads_per_wg(2, 32, 8, 8192, 128, 128, 64) == 4   # 128-row tile as four 64-row heads
    assert lib.fa_fwd_rows_per_wg(128, 64, 128, 4) == 64
    assert lib.fa_fwd_heads_per_wg(1, 32, 1, 16384, 64, 128, 64) == 4
    assert lib.fa_fwd_heads_per_wg(2, 8, 1, 2048, 128, 128, 64) == 2    # four would leave CUs short
    assert lib.fa_fwd_heads_per_wg(2, 8, 1, 1024, 128, 64, 64) == 2   # 4 -> 2: under 2 workgroups per CU
    assert lib.fa_fwd_heads_per_wg(1, 16, 4, 4096, 128, 64, 64) == 2  # one per CU at four heads
    assert lib.fa_fwd_heads_per_wg(2, 8, 1, 8192, 128, 64, 64) == 4   # two per CU: four stay
    assert lib.fa_fwd_heads_per_wg(2, 8, 1, 8192, 64, 64, 64) == 4
    assert lib.fa_fwd_heads_per_wg(2, 8, 1, 8192, 32, 64, 64) == 2    # D = 32: under 4 per CU
    assert lib.fa_fwd_heads_per_wg(1, 32, 1, 16384, 64, 64, 128) == 2
    # dK/dV split: two items per workgroup slot (the paired D = 128 kernel one slot per CU, the
    # one-wave kernel two), one round more per 8192 keys; no split under 64 pairs per key tile
    assert lib.fa_bwd_dkdv_split(4, 32, 32, 4096, 128) == 1
    assert lib.fa_bwd_dkdv_split(1, 32, 1, 4096, 128) == 16    # 32 key tiles, target 512
    assert lib.fa_bwd_dkdv_split(1, 32, 1, 4096, 64) == 32     # target 1024
    assert lib.fa_bwd_dkdv_split(1, 32, 1, 16384, 64) == 16    # 128 key tiles, target 2 x 1024
    assert lib.fa_bwd_dkdv_split(1, 8, 1, 16384, 128) == 8     # target 2 x 512
    assert lib.fa_bwd_dkdv_split(1, 8, 8, 4096, 128) == 2
    assert lib.fa_bwd_dkdv_split(1, 4, 4, 8192, 128) == 2      # 256 key tiles, target 512
    assert lib.fa_bwd_dkdv_split(1, 16, 16, 4096, 64) == 2     # 512 key tiles, target 1024
    assert lib.fa_bwd_dkdv_split(2, 16, 16, 4096, 64) == 1
    assert lib.fa_bwd_dkdv_split(2, 8, 8, 2048, 128) == 1      # 32 pairs per key tile
    assert lib.fa_fwd_heads_per_wg(0, 32, 8, 4096, 128, 64, 64) == 0 and lib.fa_bwd_dkdv_split(1, 4, 3, 64, 128) == 0
    assert lib.fa_fwd_heads_per_wg(2, 32, 8, 4096, 48, 64, 64) == 0
    assert lib.fa_bwd_dkdv_split(1, 4, 4, 64, 48) == 0
