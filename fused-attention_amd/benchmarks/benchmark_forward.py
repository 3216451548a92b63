"""Forward benchmark (MHA): fused vs unfused vs torch SDPA, on MI355X.

The reference's benchmarks/benchmark_forward.py command line and outputs: --kernel loads
fused_attention from any kernel file (default attention/fused/fused.py), --tag names the
outputs, rows are [D, N, B, H, impl, tile_m, tile_n, median_ms, tflops, first_call_ms,
fused_speedup_vs_unfused, fused_speedup_vs_sdpa, gpu, kernel] (plus pct_of_peak and gbps at the
end), with a summary CSV of averages per N / per D and a plot.  Extensions: --Ds, --Ns, --dtype
(fp16 as the reference, or bf16), --scale (inputs ~ N(0,1) x scale).

    python -m benchmarks.benchmark_forward --tile-m 128 --tile-n 64
    python -m benchmarks.benchmark_forward --B 4 --H 32 --Ds 128 --Ns 4096 --dtype bf16
"""

import argparse
import os
import sys

import torch
import torch.nn.functional as F

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))  # package root
from attention.fused.unfused import unfused_attention  # noqa: E402
from benchmarks import _timing as T  # noqa: E402

HEADER = ["D", "N", "B", "H", "impl", "tile_m", "tile_n", "median_ms", "tflops", "first_call_ms",
          "fused_speedup_vs_unfused", "fused_speedup_vs_sdpa", "gpu", "kernel", "pct_of_peak", "gbps"]


def make_impls(fused):
    return {
        "fused": lambda q, k, v, tm, tn: fused(q, k, v, tm, tn),
        "unfused": lambda q, k, v, tm, tn: unfused_attention(q, k, v, tm, tn),
        "sdpa": lambda q, k, v, tm, tn: F.scaled_dot_product_attention(q, k, v, is_causal=True),
    }


def run(args, impls, make_qkv, h_kv_of, flops_of, bytes_of, extra_cols=()):
    """Time every (D, N, impl); returns rows without the speedup/gpu/kernel columns."""
    rows = []
    settled = False
    for D in map(int, args.Ds.split(",")):
        for N in map(int, args.Ns.split(",")):
            q, k, v = make_qkv(D, N)
            flops, nbytes = flops_of(D, N), bytes_of(D, N)
            for name in args.impls.split(","):
                fn = impls[name]
                call = lambda: fn(q, k, v, args.tile_m, args.tile_n)  # noqa: E731
                try:
                    if not settled:
                        T.settle_clocks(call)
                        settled = True
                    ms, first = T.time_call(call)
                    tflops = flops / (ms * 1e-3) / 1e12
                    print(f"D={D:<4} N={N:<6} {name:<8} {ms:9.4f} ms  {tflops:7.2f} TFLOP/s"
                          f"  (first call {first:.0f} ms)", flush=True)
                    rows.append(dict(D=D, N=N, impl=name, ms=ms, tflops=tflops, first=first,
                                     pct=100 * tflops / T.PEAK_TFLOPS[args.dtype],
                                     gbps=nbytes / (ms * 1e-3) / 1e9, extra=[c(D, N) for c in extra_cols]))
                except Exception as e:  # a failing implementation leaves an empty row, as the reference
                    print(f"D={D:<4} N={N:<6} {name:<8} FAILED: {type(e).__name__}: {e}", flush=True)
                    rows.append(dict(D=D, N=N, impl=name, ms=None, tflops=None, first=None, pct=None,
                                     gbps=None, extra=[c(D, N) for c in extra_cols]))
                torch.cuda.empty_cache()
            del q, k, v
    return rows


def emit(args, rows, kernel, header, out, summary_out, plot_out, base_cols):
    gpu = torch.cuda.get_device_name()
    sp = T.speedups(rows, key_of=lambda r: (r["D"], r["N"]), impl_of=lambda r: r["impl"],
                    ms_of=lambda r: r["ms"])
    fmt = lambda x, f: "" if x is None else format(x, f)  # noqa: E731
    table = []
    for r, s in zip(rows, sp):
        table.append(base_cols(r) + [fmt(r["ms"], ".4f"), fmt(r["tflops"], ".3f"), fmt(r["first"], ".1f")]
                     + r["extra"] + s + [gpu, kernel, fmt(r["pct"], ".2f"), fmt(r["gbps"], ".1f")])
    T.write_csv(out, header, table)
    ok = [(r["D"], r["N"], r["impl"], r["ms"], r["tflops"]) for r in rows if r["ms"] is not None]
    impls = list(dict.fromkeys(r[2] for r in ok))
    sh, srows = T.summary_rows(ok, impls)
    T.write_csv(summary_out, sh, srows)
    T.plot_panels(ok, plot_out)


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--kernel", default="attention/fused/fused.py",
                   help="Python file defining fused_attention(q, k, v, tile_m, tile_n)")
    p.add_argument("--tag", default=None, help="name used in output paths (default: kernel file name)")
    p.add_argument("--B", type=int, default=2)
    p.add_argument("--H", type=int, default=8)
    p.add_argument("--tile-m", type=int, default=64)
    p.add_argument("--tile-n", type=int, default=64)
    p.add_argument("--impls", default="fused,unfused,sdpa")
    p.add_argument("--Ds", default="64,128")
    p.add_argument("--Ns", default="128,512,2048,8192")
    p.add_argument("--dtype", choices=sorted(T.DTYPES), default="fp16")
    p.add_argument("--scale", type=float, default=1.0, help="inputs ~ N(0,1) x scale")
    p.add_argument("--out", default=None)
    p.add_argument("--summary-out", default=None)
    p.add_argument("--plot-out", default=None)
    args = p.parse_args(argv)

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    kernel = args.kernel if os.path.isabs(args.kernel) else os.path.join(root, args.kernel)
    fused = T.load_function(kernel, "fused_attention")
    tag = args.tag or os.path.splitext(os.path.basename(args.kernel))[0]
    tile = f"{args.tile_m}x{args.tile_n}"
    base = f"results/benchmarks/fused/{tag}/{tile}"
    out = args.out or f"{base}/bench_forward_sep_{tag}_{tile}.csv"
    summary_out = args.summary_out or f"{base}/bench_forward_agg_{tag}_{tile}.csv"
    plot_out = args.plot_out or f"{base}/bench_forward_plots_{tag}_{tile}.png"
    print(f"kernel={args.kernel}  tag={tag}  tile={tile}  dtype={args.dtype}  gpu={torch.cuda.get_device_name()}")

    dt = T.DTYPES[args.dtype]
    gen = torch.Generator(device="cuda").manual_seed(0)
    make_qkv = lambda D, N: tuple(  # noqa: E731
        (torch.randn(args.B, args.H, N, D, device="cuda", generator=gen) * args.scale).to(dt) for _ in range(3))
    rows = run(args, make_impls(fused), make_qkv, None,
               flops_of=lambda D, N: T.causal_flops(args.B, args.H, N, D),
               bytes_of=lambda D, N: T.forward_bytes(args.B, args.H, args.H, N, D))
    emit(args, rows, args.kernel, HEADER, out, summary_out, plot_out,
         base_cols=lambda r: [r["D"], r["N"], args.B, args.H, r["impl"], args.tile_m, args.tile_n])
    return 0


if __name__ == "__main__":
    sys.exit(main())
