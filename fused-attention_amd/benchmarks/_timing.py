"""Shared pieces of the benchmark scripts: the timing protocol, FLOP and byte counts, loading
a kernel file by path, and the CSV summaries.

Timing follows the reference protocol (benchmarks/benchmark_forward.py:34-57 there): one untimed
first call, 10 warm-up calls, then the median of 30 per-call HIP-event timings with a
synchronize after each.  Before the first size, about a second of untimed calls settles the
GPU clocks (a cold MI355X runs ~12 % slow for its first second).
"""

import csv
import importlib.util
import os
import re
import statistics
import time

import torch

PEAK_TFLOPS = {"fp16": 2516.6, "bf16": 2516.6}  # dense MFMA peak of MI355X
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def causal_flops(B, H, N, D):
    """Useful causal FLOPs of the forward: 2 matmuls x 2*N*N*D, halved by the mask."""
    return 2.0 * B * H * N * N * D


def forward_bytes(B, H, H_kv, N, D, elem=2):
    """Algorithmic HBM bytes of the forward: Q and O of H heads, K and V of H_kv heads, once."""
    return (2 * B * H * N * D + 2 * B * H_kv * N * D) * elem


def load_function(path, name):
    """Import `name` from a Python file by path (the reference's kernel-file plugin mechanism)."""
    mod_name = "kernel_" + re.sub(r"\W", "_", os.path.splitext(os.path.basename(path))[0])
    spec = importlib.util.spec_from_file_location(mod_name, path)
    if spec is None or spec.loader is None:
        raise FileNotFoundError(path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return getattr(mod, name)


def settle_clocks(fn, seconds=1.0):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        torch.cuda.synchronize()


def event_ms(fn):
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b)


def time_call(fn, warmup=10, reps=30):
    """(median ms of `reps` event-timed calls, ms of the first call)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    return statistics.median(event_ms(fn) for _ in range(reps)), first_ms


def write_csv(path, header, rows):
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)
    print(f"wrote {path}")


def speedups(rows, key_of, impl_of, ms_of, others=("unfused", "sdpa")):
    """Per row: ms(other) / ms(fused) for the same configuration, '' where either is missing or
    the row is not the fused one (>1 means fused is faster)."""
    lat = {(key_of(r), impl_of(r)): ms_of(r) for r in rows if ms_of(r) is not None}
    out = []
    for r in rows:
        f_ms = lat.get((key_of(r), "fused")) if impl_of(r) == "fused" else None
        out.append([f"{lat[(key_of(r), o)] / f_ms:.3f}" if f_ms and (key_of(r), o) in lat else ""
                    for o in others])
    return out


def summary_rows(ok, impls, others=("unfused", "sdpa")):
    """Averages per N, per D and overall of (median ms, TFLOP/s) per implementation, and the
    geometric mean over configurations of ms(other) / ms(fused).  `ok` holds tuples
    (D, N, impl, ms, tflops) of the runs that completed."""
    def one(scope, value, sub):
        row = [scope, value]
        for name in impls:
            ms = [r[3] for r in sub if r[2] == name]
            tf = [r[4] for r in sub if r[2] == name]
            row += [f"{statistics.mean(ms):.4f}" if ms else "", f"{statistics.mean(tf):.3f}" if tf else ""]
        lat = {(r[0], r[1], r[2]): r[3] for r in sub}
        for other in others:
            ratios = [lat[(d, n, other)] / ms for (d, n, name), ms in lat.items()
                      if name == "fused" and (d, n, other) in lat]
            row.append(f"{statistics.geometric_mean(ratios):.2f}" if ratios else "")
        return row

    out = [one("N", n, [r for r in ok if r[1] == n]) for n in sorted({r[1] for r in ok})]
    out += [one("D", d, [r for r in ok if r[0] == d]) for d in sorted({r[0] for r in ok})]
    out.append(one("all", "all", ok))
    header = (["scope", "value"] + [f"{name}_{m}" for name in impls for m in ("avg_median_ms", "avg_tflops")]
              + [f"fused_speedup_vs_{o}" for o in others])
    return header, out


def plot_panels(ok, path, others=("unfused", "sdpa")):
    """One row of panels per head dim: median latency, throughput and the fused speedup over
    the other implementations, each against N.  `ok` holds (D, N, impl, ms, tflops)."""
    try:
        import matplotlib
        matplotlib.use("Agg")
        import matplotlib.pyplot as plt
    except ImportError:
        print("matplotlib not installed; skipping plots")
        return
    Ds = sorted({r[0] for r in ok})
    Ns = sorted({r[1] for r in ok})
    impls = list(dict.fromkeys(r[2] for r in ok))
    ms = {(r[0], r[1], r[2]): r[3] for r in ok}
    tf = {(r[0], r[1], r[2]): r[4] for r in ok}
    fig, axes = plt.subplots(len(Ds), 3, figsize=(15, 4 * len(Ds)), squeeze=False)
    for row, D in zip(axes, Ds):
        for ax, table, label, logy in ((row[0], ms, "median latency (ms)", True),
                                       (row[1], tf, "TFLOP/s", False)):
            for name in impls:
                pts = [(n, table[(D, n, name)]) for n in Ns if (D, n, name) in table]
                if pts:
                    ax.plot(*zip(*pts), marker="o", label=name)
            ax.set_ylabel(label)
            if logy:
                ax.set_yscale("log")
        for other in others:
            pts = [(n, ms[(D, n, other)] / ms[(D, n, "fused")]) for n in Ns
                   if (D, n, "fused") in ms and (D, n, other) in ms]
            if pts:
                row[2].plot(*zip(*pts), marker="s", label=f"vs {other}")
        row[2].axhline(1.0, linestyle="--", linewidth=1, color="gray")
        row[2].set_ylabel("fused speedup (x)")
        for ax, title in zip(row, ("latency", "throughput", "speedup")):
            ax.set_title(f"{title}, D={D}")
            ax.set_xscale("log", base=2)
            ax.set_xlabel("N")
            ax.legend(frameon=False)
    fig.tight_layout()
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    fig.savefig(path, dpi=120)
    plt.close(fig)
    print(f"wrote {path}")
