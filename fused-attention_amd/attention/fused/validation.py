"""Input checks shared by run_attention.py, the wrappers and the tests.

Restates the reference contract (attention/fused/validation.py:1-87) with three
widenings for this library:
  * dtypes: float16 and bfloat16 for the fused backend, and float32 as well for
    the fp32 reference backend (the reference accepts float16 only, :43-44);
  * sequence length up to MAX_SEQ_LEN = 65536 (the reference stops at 8192, :17);
  * any N: the kernels mask a partial last tile (the reference requires N to be a
    multiple of both tiles, :80-87, and lists partial edge tiles as future work);
    the tiles themselves must be 64 or 128 (the kernels' tile set).

Input requirements:
  Q: [B, H, N, D]   K: [B, H, N, D]   V: [B, H, N, D]   all contiguous, one dtype
  1 <= B <= 16, 1 <= H <= 32, 1 <= N <= 65536, D in {32, 64, 128}
  causal self-attention only, so Nq == Nk == N
  query tile block_m and key tile block_n each 64 or 128

Works on NumPy arrays and torch tensors (anything with .shape and .dtype).
Every failure raises ValidationError naming the offending input and the
allowed values, so the CLI can print it and exit with status 2.
"""

MAX_BATCH = 16
MAX_HEADS = 32
MAX_SEQ_LEN = 65536
SUPPORTED_HEAD_DIMS = (32, 64, 128)
SUPPORTED_DTYPES = ("float16", "bfloat16", "float32")
SUPPORTED_TILES = (64, 128)


class ValidationError(ValueError):
    """Raised for inputs outside the supported scope."""


def _dtype_name(x) -> str:
    # numpy: dtype('float16') -> 'float16'; torch: torch.bfloat16 -> 'bfloat16'
    return str(x.dtype).replace("torch.", "")


def _is_contiguous(x) -> bool:
    if hasattr(x, "is_contiguous"):  # torch
        return x.is_contiguous()
    flags = getattr(x, "flags", None)  # numpy
    return True if flags is None else bool(flags["C_CONTIGUOUS"])


def _check_tensors(tensors, dtypes):
    names = set()
    for name, t in tensors.items():
        dt = _dtype_name(t)
        if dt not in dtypes:
            raise ValidationError(f"{name} has dtype {dt}; supported: {', '.join(dtypes)}")
        names.add(dt)
        if len(t.shape) != 4:
            raise ValidationError(
                f"{name} must be 4-D [B, H, N, D], got {len(t.shape)}-D shape {tuple(t.shape)}")
        if not _is_contiguous(t):
            raise ValidationError(f"{name} must be contiguous")
    if len(names) != 1:
        raise ValidationError(f"Q, K and V must share one dtype, got {sorted(names)}")


def _check_bounds(B, H, N, D, block_m, block_n):
    if not 1 <= B <= MAX_BATCH:
        raise ValidationError(f"batch size B={B} out of range [1, {MAX_BATCH}]")
    if not 1 <= H <= MAX_HEADS:
        raise ValidationError(f"head count H={H} out of range [1, {MAX_HEADS}]")
    if not 1 <= N <= MAX_SEQ_LEN:
        raise ValidationError(f"sequence length N={N} out of range [1, {MAX_SEQ_LEN}]")
    if D not in SUPPORTED_HEAD_DIMS:
        raise ValidationError(f"head dim D={D} not supported; allowed {SUPPORTED_HEAD_DIMS}")
    for label, block in (("query tile block_m", block_m), ("key tile block_n", block_n)):
        if block not in SUPPORTED_TILES:
            raise ValidationError(f"{label}={block} not supported; allowed {SUPPORTED_TILES}")


def validate_qkv(q, k, v, block_m: int, block_n: int, dtypes=SUPPORTED_DTYPES) -> None:
    """Raise ValidationError if Q, K, V are not supported for the given tile sizes."""
    _check_tensors({"Q": q, "K": k, "V": v}, dtypes)
    B, H, Nq, D = q.shape
    Bk, Hk, Nk, Dk = k.shape
    Bv, Hv, Nv, Dv = v.shape
    if not (B == Bk == Bv):
        raise ValidationError(f"batch size mismatch: Q={B}, K={Bk}, V={Bv}")
    if not (H == Hk == Hv):
        raise ValidationError(f"head count mismatch: Q={H}, K={Hk}, V={Hv}")
    if not (Nq == Nk == Nv):
        raise ValidationError(
            f"sequence length mismatch: Q={Nq}, K={Nk}, V={Nv}; causal self-attention needs Nq == Nk")
    if not (D == Dk == Dv):
        raise ValidationError(
            f"head dim mismatch: Q={D}, K={Dk}, V={Dv}; Q, K and V must share the same head dim D")
    _check_bounds(B, H, Nq, D, block_m, block_n)
