"""Command-line interface for causal GQA/MQA attention (drop-in for run_attention_gqa.py).

    python run_attention_gqa.py --input INPUT.npz --output OUTPUT.npy --backend hip

Input:  .npz with Q [B, H, N, D], K [B, H_kv, N, D], V [B, H_kv, N, D]; H_kv divides H
        (query head h reads K/V head h // (H // H_kv)); dtypes and limits as run_attention.py
Output: .npy, float16 (or --output-dtype float32), shape [B, H, N, D]

Backends:
  hip        fused gfx950 GQA kernel (attention/gqa/fused_gqa.py); `cutile` is an alias
  unfused    unfused three-step baseline (attention/gqa/unfused_gqa.py)
  reference  PyTorch reference, fp32 intermediates (attention/gqa/reference_gqa.py); runs on CPU too

Exit status: 0 success, 2 unsupported input or usage error, 1 runtime failure.
"""

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from attention import cli  # noqa: E402
from attention.gqa.validation_gqa import ValidationError, validate_qkv  # noqa: E402

BACKENDS = cli.BACKENDS


def _hip_backend():
    from attention.gqa.fused_gqa import fused_gqa_attention
    return fused_gqa_attention


def _unfused_backend():
    from attention.gqa.unfused_gqa import unfused_gqa_attention
    return lambda q, k, v, bm, bn: unfused_gqa_attention(q, k, v, bm, bn)


def _reference_backend():
    from attention.gqa.reference_gqa import causal_attention_reference_gqa
    return lambda q, k, v, bm, bn: causal_attention_reference_gqa(q, k, v)


# backend name -> factory (imports deferred to the pick; "cutile" names the fused HIP path)
_FACTORIES = {"hip": _hip_backend, "cutile": _hip_backend, "unfused": _unfused_backend,
              "reference": _reference_backend}


def get_backend(name):
    """The grouped-query attention callable of backend `name`, called as
    fn(q, k, v, block_m, block_n) with K/V of H_kv heads, returning O shaped like q
    (run_attention_gqa.py:64-75 in the reference)."""
    factory = _FACTORIES.get(name)
    if factory is None:
        raise NotImplementedError(f"backend '{name}' is not implemented")
    return factory()


def main(argv=None) -> int:
    return cli.main(argv, "Causal GQA/MQA scaled dot-product attention on Q, K, V from an .npz file.",
                    validate_qkv, ValidationError, get_backend)


if __name__ == "__main__":
    sys.exit(main())
