"""ctypes binding of libfa.so, the gfx950 HIP library behind every fused backend.

The library exports the C ABI declared in include/fa.h.  It is built in-tree
(``make -C fused-attention_amd/csrc``) and loaded from the package root.  There
is no fallback: if the library is missing, every fused entry point raises.
"""

import ctypes
import math
import os

import torch

LOG2E = 1.4426950408889634  # log2(e), folded with 1/sqrt(D) as in attention/fused/fused.py:74

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("FA_LIB_PATH", os.path.join(_PKG_ROOT, "libfa.so"))

FA_F16, FA_BF16 = 0, 1
_DTYPE_CODE = {torch.float16: FA_F16, torch.bfloat16: FA_BF16}

FA_OK = 0
FA_ERR_DIMS = -1
FA_ERR_DTYPE = -2
FA_ERR_HEADDIM = -3
FA_ERR_TILE = -4
FA_ERR_NULL = -5
FA_ERR_LAUNCH = -6
FA_ERR_UNSUPPORTED = -7
FA_ERR_WORKSPACE = -8
FA_ERR_SCRATCH = -9

# (name, restype, argtypes) for every symbol of include/fa.h
_VP, _I, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "fa_fwd": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _F, _I, _I, _VP]),
    "fa_bwd": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                    _I, _I, _I, _I, _I, _F, _F, _I, _I, _VP]),
    "fa_bwd_gqa": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                        _I, _I, _I, _I, _I, _I, _F, _F, _I, _I, _VP, ctypes.c_size_t, _VP]),
    "fa_bwd_gqa_noalloc": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                _I, _I, _I, _I, _I, _I, _F, _F, _I, _I, _VP]),
    "fa_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "fa_fwd_exact": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I, _VP]),
    "fa_bwd_gqa_exact": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                              _I, _I, _I, _I, _I, _I, _F, _F, _I, _I, _I, _VP, ctypes.c_size_t, _VP]),
    "fa_fwd_heads_per_wg": (_I, [_I, _I, _I, _I, _I, _I, _I]),
    "fa_fwd_rows_per_wg": (_I, [_I, _I, _I, _I]),
    "fa_bwd_dq_rows_per_wg": (_I, [_I, _I]),
    "fa_bwd_dkdv_split": (_I, [_I, _I, _I, _I, _I]),
    "fa_bwd_gqa_workspace_size": (ctypes.c_size_t, [_I, _I, _I, _I, _I]),
    "fa_supported": (_I, [_I, _I, _I, _I, _I, _I, _I]),
    "fa_strerror": (ctypes.c_char_p, [_I]),
    "fa_version": (_I, []),
}

_lib = None


class LibraryError(RuntimeError):
    """libfa.so is missing or could not be loaded."""


def load():
    """Load libfa.so once; raise LibraryError (never fall back) if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryError(
            f"{LIB_PATH} not found; build it with `make -C fused-attention_amd/csrc` "
            f"(or __graft_entry__.build()) before using the fused backends")
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:
        raise LibraryError(f"could not load {LIB_PATH}: {e}") from e
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


_autograd = None


def autograd():
    """The C++ autograd op (fa_autograd, built by csrc/build_autograd.py next to libfa.so);
    raise LibraryError (never fall back) if it is absent."""
    global _autograd
    if _autograd is not None:
        return _autograd
    load()  # the op calls into libfa.so; load (and check) it first
    import importlib.util
    import sysconfig
    path = os.path.join(_PKG_ROOT, "fa_autograd" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.exists(path):
        raise LibraryError(
            f"{path} not found; build it with `python3 fused-attention_amd/csrc/build_autograd.py` "
            f"(or __graft_entry__.build()) before using the fused autograd entry points")
    spec = importlib.util.spec_from_file_location("fa_autograd", path)
    try:
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
    except ImportError as e:
        raise LibraryError(f"could not load {path}: {e}") from e
    _autograd = mod
    return mod


def strerror(code):
    return load().fa_strerror(code).decode()


def dtype_code(dtype):
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"fused kernels support float16 and bfloat16, got {dtype}") from None


def scale_log2(D):
    return LOG2E / math.sqrt(D)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


# The current stream's raw handle: torch's direct accessor when it has one (about 0.1 us
# against 2 us for current_stream(), which builds a Stream object; a small call is bound
# by host time), else the public route.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device):
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return ctypes.c_void_p(_raw_stream(index))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_device(*tensors):
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("fused kernels need GPU tensors; move Q, K, V to the GPU first")


def check(code, what):
    """Map a negative status to the reference's exception types."""
    if code == FA_OK:
        return
    msg = f"{what}: {strerror(code)} (status {code})"
    if code == FA_ERR_DTYPE:
        raise TypeError(msg)
    if code in (FA_ERR_DIMS, FA_ERR_HEADDIM, FA_ERR_TILE, FA_ERR_NULL, FA_ERR_UNSUPPORTED, FA_ERR_WORKSPACE,
                FA_ERR_SCRATCH):
        raise ValueError(msg)
    raise RuntimeError(msg)


def check_tiles(tile_m, tile_n):
    """The kernels' tile contract: tile_m, tile_n in {64, 128}; N needs no relation to them
    (a partial last tile is masked; the reference required N to be a multiple of both)."""
    if tile_m not in (64, 128) or tile_n not in (64, 128):
        raise ValueError(f"tile_m={tile_m} and tile_n={tile_n} must each be 64 or 128")


def fwd(q, k, v, o, lse, tile_m, tile_n):
    """Enqueue the forward on the current stream.  Shapes already checked by the caller."""
    lib = load()
    _require_device(q, k, v, o)
    B, H, S, D = q.shape
    H_kv = k.shape[1]
    code = lib.fa_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse),
                      B, H, H_kv, S, D, dtype_code(q.dtype), scale_log2(D),
                      int(tile_m), int(tile_n), _stream(q.device))
    check(code, "fa_fwd")


def bwd(q, k, v, o, do, lse, dq, dk, dv, tile_m, tile_n):
    """Enqueue the backward on the current stream (K/V may have fewer heads: GQA).

    Goes through fa_bwd_gqa with its workspace (H_kv = H included): the per-row -LSE/c and
    -Delta that let dQ run first and spare dK/dV forming Delta per key tile, plus fp32 partial
    dK/dV when the key tiles alone leave the GPU idle (MQA, few heads, small batch).  The
    caching allocator keeps the block for this stream's pending work.
    """
    lib = load()
    _require_device(q, k, v, o, do, lse, dq, dk, dv)
    B, H, S, D = q.shape
    H_kv = k.shape[1]
    # (the size depends on the device only through its CU count, the same on every MI355X;
    # the query costs about 0.4 us, so it is not cached)
    nbytes = lib.fa_bwd_gqa_workspace_size(B, H, H_kv, S, D)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    code = lib.fa_bwd_gqa(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(do), _ptr(lse),
                          _ptr(dq), _ptr(dk), _ptr(dv), B, H, H_kv, S, D, dtype_code(q.dtype),
                          scale_log2(D), 1.0 / math.sqrt(D), int(tile_m), int(tile_n),
                          _ptr(ws), nbytes, _stream(q.device))
    check(code, "fa_bwd_gqa")
