"""Forward benchmark for grouped-query attention (GQA/MQA): fused vs unfused vs torch SDPA.

The reference's benchmarks/benchmark_forward_gqa.py command line and outputs: Q is [B, H, N, D],
K and V are [B, H_kv, N, D]; rows are the forward benchmark's columns with H_kv after
first_call_ms (plus pct_of_peak and gbps at the end).  FLOPs are those of MHA (they depend on H,
not H_kv); gbps counts Q and O of H heads and K and V of H_kv heads once.

    python -m benchmarks.benchmark_forward_gqa --H-kv 2 --tile-m 64 --tile-n 64
    python -m benchmarks.benchmark_forward_gqa --B 2 --H 32 --H-kv 8 --Ds 128 --Ns 8192 --dtype bf16
"""

import argparse
import os
import sys

import torch
import torch.nn.functional as F

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))  # package root
from attention.gqa.unfused_gqa import unfused_gqa_attention  # noqa: E402
from benchmarks import _timing as T  # noqa: E402
from benchmarks.benchmark_forward import emit, run  # noqa: E402

HEADER = ["D", "N", "B", "H", "impl", "tile_m", "tile_n", "median_ms", "tflops", "first_call_ms", "H_kv",
          "fused_speedup_vs_unfused", "fused_speedup_vs_sdpa", "gpu", "kernel", "pct_of_peak", "gbps"]


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--kernel", default="attention/gqa/fused_gqa.py",
                   help="Python file defining fused_gqa_attention(q, k, v, tile_m, tile_n)")
    p.add_argument("--tag", default=None, help="name used in output paths (default: kernel file name)")
    p.add_argument("--B", type=int, default=2)
    p.add_argument("--H", type=int, default=8)
    p.add_argument("--H-kv", type=int, default=8, help="K/V heads (must divide --H)")
    p.add_argument("--tile-m", type=int, default=64)
    p.add_argument("--tile-n", type=int, default=64)
    p.add_argument("--impls", default="fused,unfused,sdpa")
    p.add_argument("--Ds", default="32,64,128")
    p.add_argument("--Ns", default="128,512,2048,8192")
    p.add_argument("--dtype", choices=sorted(T.DTYPES), default="fp16")
    p.add_argument("--scale", type=float, default=1.0, help="inputs ~ N(0,1) x scale")
    p.add_argument("--out", default=None)
    p.add_argument("--summary-out", default=None)
    p.add_argument("--plot-out", default=None)
    args = p.parse_args(argv)
    if args.H_kv < 1 or args.H % args.H_kv:
        p.error(f"--H-kv={args.H_kv} must divide --H={args.H}")

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    kernel = args.kernel if os.path.isabs(args.kernel) else os.path.join(root, args.kernel)
    fused = T.load_function(kernel, "fused_gqa_attention")
    tag = args.tag or os.path.splitext(os.path.basename(args.kernel))[0]
    tile = f"{args.tile_m}x{args.tile_n}"
    base = f"results/benchmarks/fused_gqa/{tag}/{tile}/Hkv{args.H_kv}"
    out = args.out or f"{base}/bench_forward_gqa_sep_{tag}_{tile}_Hkv{args.H_kv}.csv"
    summary_out = args.summary_out or f"{base}/bench_forward_gqa_agg_{tag}_{tile}_Hkv{args.H_kv}.csv"
    plot_out = args.plot_out or f"{base}/bench_forward_gqa_plots_{tag}_{tile}_Hkv{args.H_kv}.png"
    print(f"kernel={args.kernel}  tag={tag}  tile={tile}  H={args.H}  H_kv={args.H_kv}  dtype={args.dtype}"
          f"  gpu={torch.cuda.get_device_name()}")

    impls = {
        "fused": lambda q, k, v, tm, tn: fused(q, k, v, tm, tn),
        "unfused": lambda q, k, v, tm, tn: unfused_gqa_attention(q, k, v, tm, tn),
        "sdpa": lambda q, k, v, tm, tn: F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True),
    }
    dt = T.DTYPES[args.dtype]
    gen = torch.Generator(device="cuda").manual_seed(0)

    def make_qkv(D, N):
        q = (torch.randn(args.B, args.H, N, D, device="cuda", generator=gen) * args.scale).to(dt)
        k, v = ((torch.randn(args.B, args.H_kv, N, D, device="cuda", generator=gen) * args.scale).to(dt)
                for _ in range(2))
        return q, k, v

    rows = run(args, impls, make_qkv, None,
               flops_of=lambda D, N: T.causal_flops(args.B, args.H, N, D),
               bytes_of=lambda D, N: T.forward_bytes(args.B, args.H, args.H_kv, N, D),
               extra_cols=(lambda D, N: args.H_kv,))
    emit(args, rows, args.kernel, HEADER, out, summary_out, plot_out,
         base_cols=lambda r: [r["D"], r["N"], args.B, args.H, r["impl"], args.tile_m, args.tile_n])
    return 0


if __name__ == "__main__":
    sys.exit(main())
