"""Backward benchmark: fused forward + recompute backward vs eager PyTorch vs torch SDPA, on MI355X.

The reference's benchmarks/benchmark_backward.py command line and outputs.  Per configuration
(causal, autograd backward, median of --reps HIP-event timings after --warmup rounds):
  fwd_ms       forward only (no autograd graph)
  bwd_ms       backward only (its forward run untimed before each backward)
  fwd_bwd_ms   forward + backward
  tflops       fwd+bwd TFLOP/s with the FlashAttention convention: causal forward FLOPs
               2*B*H*N^2*D, backward 2.5x that, recomputation not counted
  peak_mem_mb  peak extra device memory of one forward + backward beyond the inputs and dO
Writes <out-dir>/bench_backward_<tile>.csv (the reference's columns, plus pct_of_peak) and .md.

Implementations:
  fused  attention.backward.fused_backward.fused_attention_autograd (GQA: fused_gqa_attention_autograd)
  naive  eager S = QK^T / sqrt(D), mask, softmax, P V with autograd, computed in float32 (the
         N x N probabilities are stored for the backward)
  sdpa   torch.nn.functional.scaled_dot_product_attention(is_causal=True), fp16 inputs only here
Extensions: --dtype bf16 (fused only: the eager and SDPA backward paths issue batched products on
transposed 16-bit operands, which this build keeps off bf16), --H-kv for the GQA/MQA backward.

    python -m benchmarks.benchmark_backward --tile-m 64 --tile-n 64
    python -m benchmarks.benchmark_backward --B 2 --H 16 --Ds 64 --Ns 4096 --tile-m 128 --tile-n 64
"""

import argparse
import csv
import math
import os
import statistics
import sys

import torch
import torch.nn.functional as F

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))  # package root
from attention.backward.fused_backward import fused_attention_autograd  # noqa: E402
from attention.gqa.fused_gqa import fused_gqa_attention_autograd  # noqa: E402
from benchmarks import _timing as T  # noqa: E402

FIELDS = ["D", "N", "B", "H", "impl", "tile_m", "tile_n", "fwd_ms", "bwd_ms", "fwd_bwd_ms", "tflops",
          "peak_mem_mb", "status", "gpu", "H_kv", "dtype", "pct_of_peak"]


def naive_attention(q, k, v):
    """Eager causal attention in float32 (K/V repeated to the query heads for GQA)."""
    g = q.shape[1] // k.shape[1]
    if g > 1:
        k, v = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
    N, D = q.shape[-2], q.shape[-1]
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) / math.sqrt(D)
    future = torch.ones(N, N, device=q.device, dtype=torch.bool).triu(1)
    p = torch.softmax(s.masked_fill(future, float("-inf")), dim=-1)
    return torch.matmul(p, v.float()).to(q.dtype)


def make_impls(tm, tn, gqa):
    fused = fused_gqa_attention_autograd if gqa else fused_attention_autograd
    return {
        "fused": lambda q, k, v: fused(q, k, v, tm, tn),
        "naive": naive_attention,
        "sdpa": lambda q, k, v: F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=gqa),
    }


def measure(fn, q, k, v, do, warmup, reps):
    """(fwd ms, bwd ms, fwd+bwd ms, peak extra MiB) of fn with autograd on q, k, v."""
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))

    def clear():
        q.grad = k.grad = v.grad = None

    def step():
        fn(q, k, v).backward(do)

    for _ in range(warmup):
        clear()
        step()
    torch.cuda.synchronize()
    fwd = []
    with torch.no_grad():
        for _ in range(reps):
            fwd.append(T.event_ms(lambda: fn(q, k, v)))
    bwd = []
    for _ in range(reps):
        clear()
        o = fn(q, k, v)
        torch.cuda.synchronize()
        bwd.append(T.event_ms(lambda: o.backward(do)))
        del o
    both = []
    for _ in range(reps):
        clear()
        both.append(T.event_ms(step))
    clear()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    step()
    torch.cuda.synchronize()
    peak = (torch.cuda.max_memory_allocated() - base) / 2**20
    return statistics.median(fwd), statistics.median(bwd), statistics.median(both), peak


def markdown(rows, tile, gpu, a):
    ok = {(r["D"], r["N"], r["impl"]): r for r in rows if r["status"] == "ok"}
    cfgs = sorted({(r["D"], r["N"]) for r in rows})
    f = lambda x, s: "" if x is None else format(x, s)  # noqa: E731
    get = lambda D, N, i, key: ok[(D, N, i)][key] if (D, N, i) in ok else None  # noqa: E731
    div = lambda x, y: x / y if x and y else None  # noqa: E731
    out = [f"# Backward benchmark (fused tile {tile})", "",
           f"GPU: {gpu}; B={a.B}, H={a.H}, H_kv={a.H_kv or a.H}; {a.dtype} inputs; causal; median of {a.reps}.",
           "Speedup = other ms / fused ms (>1: fused faster).  Memory = peak extra device memory of fwd+bwd.", "",
           "## Forward + backward", "",
           "| D | N | fused ms | naive ms | SDPA ms | vs naive | vs SDPA | fused TFLOP/s | fused % of peak |",
           "|---|---|---|---|---|---|---|---|---|"]
    for D, N in cfgs:
        fu, na, sd = (get(D, N, i, "fwd_bwd_ms") for i in ("fused", "naive", "sdpa"))
        out.append(f"| {D} | {N} | {f(fu, '.3f')} | {f(na, '.3f')} | {f(sd, '.3f')} | {f(div(na, fu), '.2f')} | "
                   f"{f(div(sd, fu), '.2f')} | {f(get(D, N, 'fused', 'tflops'), '.1f')} | "
                   f"{f(get(D, N, 'fused', 'pct_of_peak'), '.1f')} |")
    out += ["", "## Backward only", "", "| D | N | fused bwd ms | naive bwd ms | SDPA bwd ms | fused bwd / fused fwd |",
            "|---|---|---|---|---|---|"]
    for D, N in cfgs:
        fu, na, sd = (get(D, N, i, "bwd_ms") for i in ("fused", "naive", "sdpa"))
        out.append(f"| {D} | {N} | {f(fu, '.3f')} | {f(na, '.3f')} | {f(sd, '.3f')} | "
                   f"{f(div(fu, get(D, N, 'fused', 'fwd_ms')), '.2f')} |")
    out += ["", "## Peak extra memory (MiB)", "", "| D | N | fused | naive | SDPA |", "|---|---|---|---|---|"]
    for D, N in cfgs:
        out.append(f"| {D} | {N} | " + " | ".join(f(get(D, N, i, "peak_mem_mb"), ".1f") for i in ("fused", "naive", "sdpa")) + " |")
    return out


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--B", type=int, default=2)
    p.add_argument("--H", type=int, default=8)
    p.add_argument("--H-kv", type=int, default=None, help="K/V heads for the GQA/MQA backward (default: H)")
    p.add_argument("--tile-m", type=int, default=64)
    p.add_argument("--tile-n", type=int, default=64)
    p.add_argument("--Ds", default="64,128")
    p.add_argument("--Ns", default="128,512,2048,8192")
    p.add_argument("--impls", default="fused,naive,sdpa")
    p.add_argument("--dtype", choices=sorted(T.DTYPES), default="fp16")
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--reps", type=int, default=20)
    p.add_argument("--out-dir", default="results/benchmarks/backward")
    a = p.parse_args(argv)
    h_kv = a.H_kv or a.H
    if a.H % h_kv:
        p.error(f"--H-kv={h_kv} must divide --H={a.H}")
    tm, tn = a.tile_m, a.tile_n
    impls = make_impls(tm, tn, gqa=h_kv != a.H)
    names = a.impls.split(",")
    dt = T.DTYPES[a.dtype]
    gpu = torch.cuda.get_device_name()
    print(f"GPU: {gpu}  B={a.B} H={a.H} H_kv={h_kv} dtype={a.dtype}  fused tile {tm}x{tn}")

    rows, settled = [], False
    for D in map(int, a.Ds.split(",")):
        for N in map(int, a.Ns.split(",")):
            gen = torch.Generator(device="cuda").manual_seed(N + D)
            q, do = (torch.randn(a.B, a.H, N, D, device="cuda", generator=gen).to(dt) for _ in range(2))
            k, v = (torch.randn(a.B, h_kv, N, D, device="cuda", generator=gen).to(dt) for _ in range(2))
            total = 3.5 * T.causal_flops(a.B, a.H, N, D)
            for name in names:
                base = dict(D=D, N=N, impl=name, H_kv=h_kv, dtype=a.dtype)
                if name != "fused" and a.dtype == "bf16":
                    print(f"{D:>4} {N:>6} {name:<6} | skipped: bf16 eager/SDPA backward not run")
                    rows.append(dict(base, status="skipped (bf16)"))
                    continue
                try:
                    if not settled:  # clocks and the autograd path, forward and backward
                        qs, ks, vs = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
                        T.settle_clocks(lambda: impls["fused"](qs, ks, vs).backward(do))
                        del qs, ks, vs
                        settled = True
                    f_ms, b_ms, fb_ms, mem = measure(impls[name], q, k, v, do, a.warmup, a.reps)
                    tf = total / (fb_ms * 1e-3) / 1e12
                    print(f"{D:>4} {N:>6} {name:<6} | fwd {f_ms:8.3f}  bwd {b_ms:8.3f}  fwd+bwd {fb_ms:8.3f} ms"
                          f" | {tf:7.1f} TFLOP/s | {mem:9.1f} MiB", flush=True)
                    rows.append(dict(base, fwd_ms=f_ms, bwd_ms=b_ms, fwd_bwd_ms=fb_ms, tflops=tf, peak_mem_mb=mem,
                                     pct_of_peak=100 * tf / T.PEAK_TFLOPS[a.dtype], status="ok"))
                except torch.cuda.OutOfMemoryError:
                    print(f"{D:>4} {N:>6} {name:<6} | out of memory")
                    rows.append(dict(base, status="OOM"))
                except Exception as e:
                    print(f"{D:>4} {N:>6} {name:<6} | FAILED: {type(e).__name__}: {e}")
                    rows.append(dict(base, status=f"FAILED: {type(e).__name__}"))
                torch.cuda.empty_cache()
            del q, k, v, do

    tile = f"{tm}x{tn}"
    os.makedirs(a.out_dir, exist_ok=True)
    csv_path = os.path.join(a.out_dir, f"bench_backward_{tile}.csv")
    with open(csv_path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow({**{k: (f"{v:.4f}" if isinstance(v, float) else v) for k, v in r.items()},
                        "B": a.B, "H": a.H, "tile_m": tm, "tile_n": tn, "gpu": gpu})
    md = markdown(rows, tile, gpu, a)
    md_path = os.path.join(a.out_dir, f"bench_backward_{tile}.md")
    with open(md_path, "w") as f:
        f.write("\n".join(md) + "\n")
    print("\n" + "\n".join(md))
    print(f"\nwrote {csv_path}\nwrote {md_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
