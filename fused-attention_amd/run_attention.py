"""Command-line interface for causal attention (drop-in for the reference's run_attention.py).

    python run_attention.py --input INPUT.npz --output OUTPUT.npy --backend hip

Input:  .npz with contiguous arrays Q [B, H, N, D], K [B, H, N, D], V [B, H, N, D]
        float16 (all backends) or float32 (reference backend, or GPU backends with
        --compute-dtype); limits 1<=B<=16, 1<=H<=32, 1<=N<=65536, D in {32, 64, 128},
        --block-m and --block-n each 64 or 128 (any N: a partial last tile is masked)
Output: .npy, float16 (or --output-dtype float32), shape [B, H, N, D]

Backends:
  hip        fused gfx950 kernel (attention/fused/fused.py); `cutile` is an alias
  unfused    unfused three-step baseline (attention/fused/unfused.py)
  reference  PyTorch reference, fp32 intermediates (attention/fused/reference.py); runs on CPU too

Exit status: 0 success, 2 unsupported input or usage error, 1 runtime failure.
"""

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from attention import cli  # noqa: E402
from attention.fused.validation import ValidationError, validate_qkv  # noqa: E402

BACKENDS = cli.BACKENDS


def _hip_backend():
    from attention.fused.fused import fused_attention
    return fused_attention


def _unfused_backend():
    from attention.fused.unfused import unfused_attention
    return lambda q, k, v, bm, bn: unfused_attention(q, k, v, bm, bn)


def _reference_backend():
    from attention.fused.reference import causal_attention_reference
    return lambda q, k, v, bm, bn: causal_attention_reference(q, k, v)


# backend name -> factory; modules are imported only when their backend is picked, so the
# reference backend runs where no GPU library can load ("cutile" names the fused HIP path,
# as the reference's command lines expect)
_FACTORIES = {"hip": _hip_backend, "cutile": _hip_backend, "unfused": _unfused_backend,
              "reference": _reference_backend}


def get_backend(name):
    """The attention callable of backend `name`, called as fn(q, k, v, block_m, block_n) and
    returning O with q's [B, H, N, D] shape (run_attention.py:62-73 in the reference)."""
    factory = _FACTORIES.get(name)
    if factory is None:
        raise NotImplementedError(f"backend '{name}' is not implemented")
    return factory()


def main(argv=None) -> int:
    return cli.main(argv, "Causal scaled dot-product attention on Q, K, V from an .npz file.",
                    validate_qkv, ValidationError, get_backend)


if __name__ == "__main__":
    sys.exit(main())
