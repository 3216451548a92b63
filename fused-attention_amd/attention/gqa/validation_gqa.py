"""GQA/MQA input checks shared by run_attention_gqa.py and the GQA tests.

Restates attention/gqa/validation_gqa.py:39-104 with the same widenings as
attention/fused/validation.py (float16 / bfloat16 / float32, N <= 65536, any N,
tiles 64 or 128).

Input requirements:
  Q: [B, H, N, D]   K: [B, H_kv, N, D]   V: [B, H_kv, N, D]   contiguous, one dtype
  1 <= B <= 16, 1 <= H <= 32, 1 <= N <= 65536, D in {32, 64, 128}
  1 <= H_kv <= H and H % H_kv == 0   (H_kv == H is MHA, H_kv == 1 is MQA)
  query head h reads K/V head h // (H // H_kv)
  query tile block_m and key tile block_n each 64 or 128
"""

from attention.fused.validation import (MAX_BATCH, MAX_HEADS, MAX_SEQ_LEN,  # noqa: F401
                                        SUPPORTED_DTYPES, SUPPORTED_HEAD_DIMS, ValidationError,
                                        _check_bounds, _check_tensors)


def validate_qkv(q, k, v, block_m: int, block_n: int, dtypes=SUPPORTED_DTYPES) -> int:
    """Raise ValidationError if Q, K, V are not supported; return the group size H // H_kv."""
    _check_tensors({"Q": q, "K": k, "V": v}, dtypes)
    B, H, Nq, D = q.shape
    Bk, Hk, Nk, Dk = k.shape
    Bv, Hv, Nv, Dv = v.shape
    if not (B == Bk == Bv):
        raise ValidationError(f"batch size mismatch: Q={B}, K={Bk}, V={Bv}")
    if Hk != Hv:
        raise ValidationError(f"K/V head count mismatch: K={Hk}, V={Hv}; K and V must have the same H_kv")
    if not (Nq == Nk == Nv):
        raise ValidationError(
            f"sequence length mismatch: Q={Nq}, K={Nk}, V={Nv}; causal self-attention needs Nq == Nk")
    if not (D == Dk == Dv):
        raise ValidationError(
            f"head dim mismatch: Q={D}, K={Dk}, V={Dv}; Q, K and V must share the same head dim D")
    if not 1 <= B <= MAX_BATCH:
        raise ValidationError(f"batch size B={B} out of range [1, {MAX_BATCH}]")
    if not 1 <= H <= MAX_HEADS:
        raise ValidationError(f"head count H={H} out of range [1, {MAX_HEADS}]")
    H_kv = Hk
    if not 1 <= H_kv <= H:
        raise ValidationError(f"KV head count H_kv={H_kv} out of range [1, H={H}]")
    if H % H_kv != 0:
        raise ValidationError(
            f"query heads H={H} not divisible by KV heads H_kv={H_kv}; "
            f"H_kv must divide H (each group of H // H_kv query heads shares one K/V head)")
    _check_bounds(B, H, Nq, D, block_m, block_n)
    return H // H_kv
