"""Shared body of run_attention.py and run_attention_gqa.py.

Restates the reference CLIs (run_attention.py:1-134, run_attention_gqa.py:1-136):
.npz with Q, K, V -> validate -> backend fn(q, k, v, block_m, block_n) -> .npy.
Exit status: 0 success, 2 unsupported input or usage error, 1 runtime failure.
Messages go to stderr as `error: ...`.

Differences, all widenings:
  * backends: `hip` (the gfx950 kernels), `cutile` (accepted alias of `hip` so
    reference invocations keep working), `unfused`, `reference`;
  * the `reference` backend also runs without a GPU (on the CPU) and accepts
    float32 inputs; the GPU backends accept float16 inputs, or float32 inputs
    with --compute-dtype float16|bfloat16 (cast on the device);
  * --output-dtype float32 keeps the fp32 result (default float16, as the reference).
"""

import argparse
import os
import sys
import time

import numpy as np

EXIT_OK, EXIT_RUNTIME, EXIT_INVALID = 0, 1, 2
BACKENDS = ("hip", "cutile", "unfused", "reference")
GPU_BACKENDS = ("hip", "cutile", "unfused")


def parse_args(argv, description):
    p = argparse.ArgumentParser(description=description)
    p.add_argument("--input", required=True, help="input .npz containing Q, K, V")
    p.add_argument("--output", required=True, help="output .npy path")
    p.add_argument("--backend", choices=BACKENDS, default="hip",
                   help="implementation to run (default: hip; cutile is an alias of hip)")
    p.add_argument("--block-m", type=int, default=64, help="query tile size (default: 64)")
    p.add_argument("--block-n", type=int, default=64, help="key/value tile size (default: 64)")
    p.add_argument("--compute-dtype", choices=("input", "float16", "bfloat16"), default="input",
                   help="dtype the GPU backends compute in (default: the input dtype)")
    p.add_argument("--output-dtype", choices=("float16", "float32"), default="float16",
                   help="dtype of the written .npy (default: float16)")
    p.add_argument("--verbose", action="store_true", help="print shapes and timing to stderr")
    return p.parse_args(argv)


def load_qkv(path, ValidationError):
    """The Q, K and V arrays of an .npz archive.

    Every way the file can be unusable -- absent, not an archive, or lacking one of the
    three keys -- becomes the caller's ValidationError, whose text is the CLI's message
    (exit code 2); pickled members are refused."""
    if not os.path.exists(path):
        raise ValidationError(f"input file not found: {path}")
    try:
        archive = np.load(path, allow_pickle=False)
    except (OSError, ValueError) as e:
        raise ValidationError(f"could not read {path} as .npz: {e}")
    with archive:
        names = getattr(archive, "files", None)
        if names is None:  # a bare .npy array, not an archive of named arrays
            raise ValidationError(f"could not read {path} as .npz: not an archive of named arrays")
        absent = [name for name in ("Q", "K", "V") if name not in names]
        if absent:
            raise ValidationError(f"{path} is missing array(s) {', '.join(absent)}; found {sorted(names)}")
        try:
            return tuple(archive[name] for name in ("Q", "K", "V"))
        except (OSError, ValueError) as e:
            raise ValidationError(f"could not read {path} as .npz: {e}")


def input_dtypes(backend, compute_dtype):
    """The .npz dtypes a backend accepts."""
    if backend == "reference":
        return ("float16", "float32")
    if compute_dtype == "input":
        return ("float16",)
    return ("float16", "float32")


def run(q, k, v, fn, backend, block_m, block_n, compute_dtype):
    import torch

    if backend in GPU_BACKENDS:
        if not torch.cuda.is_available():
            raise RuntimeError("no GPU visible to PyTorch (the hip and unfused backends need one)")
        device = "cuda"
    else:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    tensors = [torch.from_numpy(x).to(device) for x in (q, k, v)]
    if backend in GPU_BACKENDS and compute_dtype != "input":
        cd = getattr(torch, compute_dtype)
        tensors = [t.to(cd) for t in tensors]
    out = fn(*tensors, block_m, block_n)
    if device == "cuda":
        torch.cuda.synchronize()
    return out.float().cpu().numpy()


def main(argv, description, validate_qkv, ValidationError, get_backend):
    args = parse_args(argv, description)
    try:
        q, k, v = load_qkv(args.input, ValidationError)
        validate_qkv(q, k, v, args.block_m, args.block_n,
                     dtypes=input_dtypes(args.backend, args.compute_dtype))
    except ValidationError as e:
        print(f"error: {e}", file=sys.stderr)
        return EXIT_INVALID

    if args.verbose:
        print(f"Q{q.shape} K{k.shape} V{v.shape} backend={args.backend} "
              f"block_m={args.block_m} block_n={args.block_n}", file=sys.stderr)

    try:
        fn = get_backend(args.backend)
        t0 = time.perf_counter()
        out = run(q, k, v, fn, args.backend, args.block_m, args.block_n, args.compute_dtype)
        elapsed = time.perf_counter() - t0
    except NotImplementedError as e:
        print(f"error: {str(e) or f'backend {args.backend!r} is not implemented yet'}", file=sys.stderr)
        return EXIT_RUNTIME
    except ModuleNotFoundError as e:
        print(f"error: missing module '{e.name}'", file=sys.stderr)
        return EXIT_RUNTIME
    except Exception as e:  # kernel, library or driver failures
        print(f"error: {args.backend} backend failed: {type(e).__name__}: {e}", file=sys.stderr)
        return EXIT_RUNTIME

    expected = tuple(q.shape[:3]) + (v.shape[3],)
    if out.shape != expected:
        print(f"error: backend returned shape {out.shape}, expected {expected}", file=sys.stderr)
        return EXIT_RUNTIME
    if not np.isfinite(out).all():
        print("error: output contains NaN or Inf", file=sys.stderr)
        return EXIT_RUNTIME

    out_dtype = np.dtype(args.output_dtype)
    np.save(args.output, out.astype(out_dtype, copy=False))
    if args.verbose:
        print(f"wrote {args.output} {out.shape} {out_dtype.name} in {elapsed:.3f}s "
              f"(includes transfers)", file=sys.stderr)
    return EXIT_OK
