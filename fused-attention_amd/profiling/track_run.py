"""Record one numbered performance run of the fused kernel on MI355X, with its environment.

The MI355X counterpart of the reference's Nsight-based tracker (profiling/track_run.py there):
same command line, same records, rocprofv3 in place of Nsight Compute.

Each run
  1. checks the kernel against the fp32 PyTorch reference (D 64/128, N 512/2048, normal and
     large scores, the reference tracker's gate at profiling/track_run.py:155-183 there);
     a failing kernel is not recorded;
  2. times fused (and torch SDPA, optionally the unfused baseline) on a grid of sizes:
     first call, 10 warm-up calls, median of 30 HIP-event timings (benchmarks/benchmark_forward.py:34-57
     there), after the GPU clocks have been settled by ~1 s of untimed calls;
  3. optionally (--profile) runs one size under rocprofv3 in child processes: a kernel trace
     (duration) and two counter passes (MFMA busy, VALU mix, LDS activity and bank conflicts,
     wave waits), summarised as percentages;
  4. appends every measurement to runs.csv, one section to RUNS.md (environment, results with
     the change against the previous and the first run on the same GPU, the profile, the code
     diff of the measured kernel file against the previous run's), and writes run_NNN/ with
     env.json, summary.md, change.diff and the profiler's CSVs.

Usage (from fused-attention_amd/, the package root):

    python -m profiling.track_run --note "baseline"
    python -m profiling.track_run --tiles 64x64,128x64 --dtype bf16 --profile --note "tile sweep"
    python -m profiling.track_run --kernel path/to/variant.py --reason "..." --change "..."
    python -m profiling.track_run --import-csv bench.csv --gpu "AMD Instinct MI355X" --note "imported"

--kernel names a Python file defining fused_attention(q, k, v, tile_m, tile_n) (default
attention/fused/fused.py).  --records-dir moves runs.csv / RUNS.md / run_NNN/ (default: this folder).
"""

import argparse
import csv
import datetime as dt
import difflib
import json
import os
import platform
import re
import shlex
import socket
import statistics
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
DEFAULT_KERNEL = "attention/fused/fused.py"
# what a forward run measures besides the kernel file: the library sources behind
# fused_attention, snapshotted into run_NNN/src/ so the next run can diff against them
# even where git is absent (the GPU machine); the snapshots are working files, kept out
# of version control (change.diff records what changed)
DEFAULT_SOURCES = "csrc/fa_fwd.hip,csrc/fa_api.hip,csrc/fa_device.h,csrc/fa_launch.h"
CSV_FIELDS = ["run", "timestamp", "gpu", "commit", "kernel", "note", "D", "N", "B", "H",
              "impl", "tile_m", "tile_n", "median_ms", "tflops", "dtype", "pct_peak"]
PEAK_TFLOPS = 2516.6  # MI355X dense bf16/fp16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk

# rocprofv3 counter passes (each within one pass's hardware limits: <= 8 SQ, <= 2 GRBM)
COUNTER_PASSES = [
    ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU",
     "SQ_INSTS_VALU_TRANS_F32", "GRBM_GUI_ACTIVE"],
    ["SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_LDS_LOAD_BANDWIDTH", "SQ_WAIT_ANY",
     "SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE"],
]
NUM_XCD, NUM_SIMD, NUM_CU = 8, 1024, 256


# --------------------------------------------------------------------------- small helpers
def sh(cmd, timeout=60):
    try:
        return subprocess.run(cmd, shell=True, capture_output=True, text=True, timeout=timeout).stdout.strip()
    except Exception:
        return ""


def now_utc():
    return dt.datetime.now(dt.timezone.utc).strftime("%Y-%m-%d %H:%M")


def git_commit():
    """Abbreviated HEAD, marked when tracked files differ from it; 'unknown' without git."""
    desc = sh(f"git -C {shlex.quote(PKG_ROOT)} describe --always --abbrev=10 --dirty=+dirty")
    if not desc:
        return "unknown"
    head, dirty = desc.split("+")[0], desc.endswith("+dirty")
    return head + (" (+ uncommitted changes)" if dirty else "")


def parse_list(s, cast=int):
    return [cast(x) for x in s.split(",") if x.strip()]


def parse_tiles(s):
    return [tuple(int(v) for v in t.lower().split("x")) for t in s.split(",") if t.strip()]


class Records:
    """runs.csv, RUNS.md and run_NNN/ under one folder."""

    def __init__(self, root):
        self.root = root
        self.csv = os.path.join(root, "runs.csv")
        self.md = os.path.join(root, "RUNS.md")

    def history(self):
        if not os.path.exists(self.csv):
            return []
        with open(self.csv) as f:
            return list(csv.DictReader(f))

    def next_run(self, history):
        return max((int(r["run"]) for r in history), default=0) + 1

    def run_dir(self, run, out_dir=None):
        return os.path.join(out_dir or os.path.join(self.root, "runs"), f"run_{run:03d}")

    def append(self, run, ts, env, note, rows, markdown, run_dir, extra_files=None):
        os.makedirs(self.root, exist_ok=True)
        os.makedirs(run_dir, exist_ok=True)
        new = not os.path.exists(self.csv)
        with open(self.csv, "a", newline="") as f:
            w = csv.DictWriter(f, fieldnames=CSV_FIELDS)
            if new:
                w.writeheader()
            for r in rows:
                w.writerow({**{k: "" for k in CSV_FIELDS},
                            **dict(run=run, timestamp=ts, gpu=env.get("gpu", ""), commit=env.get("commit", ""),
                                   kernel=env.get("kernel", ""), note=note), **r})
        if not os.path.exists(self.md):
            with open(self.md, "w") as f:
                f.write("# Performance runs\n\nOne section per run, newest at the bottom.  Times are UTC.  "
                        "Changes compare the same size, tile and dtype on the same GPU.\n\n")
        with open(self.md, "a") as f:
            f.write(markdown + "\n")
        with open(os.path.join(run_dir, "summary.md"), "w") as f:
            f.write(markdown + "\n")
        with open(os.path.join(run_dir, "env.json"), "w") as f:
            json.dump({"run": run, "timestamp": ts, "note": note, "env": env}, f, indent=2)
        for name, text in (extra_files or {}).items():
            path = os.path.join(run_dir, name)
            os.makedirs(os.path.dirname(path), exist_ok=True)
            with open(path, "w") as f:
                f.write(text)


# --------------------------------------------------------------------------- environment
def collect_env(args):
    import torch
    props = torch.cuda.get_device_properties(0)
    # rocminfo lists the host CPU agents first: read the fields of the first GPU agent only
    gpu_agents = [a for a in re.split(r"\n\*+\s*\nAgent \d+", sh("rocminfo"))
                  if re.search(r"Name:\s+gfx", a)]
    agent = gpu_agents[0] if gpu_agents else ""
    arch = re.findall(r"Name:\s+(gfx\d+\w*)", agent)
    cus = re.findall(r"Compute Unit:\s+(\d+)", agent)
    env = {
        "gpu": torch.cuda.get_device_name(0) or "AMD GPU",
        "gfx_arch": arch[0] if arch else getattr(props, "gcnArchName", "unknown"),
        "compute_units": int(cus[0]) if cus else props.multi_processor_count,
        "gpu_memory_gb": round(props.total_memory / 2**30, 1),
        "rocm_smi_clocks": sh("rocm-smi --showclocks --csv").splitlines()[1:2] or "unavailable",
        "torch": torch.__version__,
        "torch_hip": getattr(torch.version, "hip", None),
        "python": platform.python_version(),
        "host": socket.gethostname(),
        "host_cpus": os.cpu_count(),
        "rocprofv3": sh("rocprofv3 --version 2>&1 | head -1") or "not found",
        "commit": git_commit(),
        "B": args.B, "H": args.H, "dtype": args.dtype,
    }
    return env


# --------------------------------------------------------------------------- kernel under test
def load_fused(kernel_path):
    """fused_attention(q, k, v, tile_m, tile_n) from a kernel file (default: the package's)."""
    if kernel_path in (None, "", DEFAULT_KERNEL):
        from attention.fused.fused import fused_attention
        return fused_attention
    import runpy
    path = os.path.abspath(kernel_path if os.path.exists(kernel_path) else os.path.join(PKG_ROOT, kernel_path))
    # the file's top level runs once, as a script would; its fused_attention is the entry
    namespace = runpy.run_path(path, run_name="tracked_" + re.sub(r"\W", "_", os.path.basename(path)))
    if "fused_attention" not in namespace:
        raise AttributeError(f"{kernel_path} defines no fused_attention")
    return namespace["fused_attention"]


def torch_dtype(name):
    import torch
    return {"fp16": torch.float16, "bf16": torch.bfloat16}[name]


def check_correctness(fused_attention, tiles, dtype, B=2, H=8):
    """Gate before timing: every element within 2e-2 + 2e-2 |ref| of the fp32 reference, finite."""
    import torch
    from attention.fused.reference import causal_attention_reference
    ok = True
    g = torch.Generator(device="cuda").manual_seed(1)
    for D in (64, 128):
        for N in (512, 2048):
            for sigma in (1.0, 7.0):
                q, k, v = (torch.randn(B, H, N, D, device="cuda", generator=g).mul(s).to(dtype)
                           for s in (sigma, sigma, 1.0))
                ref = causal_attention_reference(q.float(), k.float(), v.float())
                for tm, tn in tiles:
                    if N % tm or N % tn:
                        continue
                    try:
                        out = fused_attention(q, k, v, tm, tn).float()
                        err = (out - ref).abs()
                        bad = bool((err > 2e-2 + 2e-2 * ref.abs()).any()) or not bool(torch.isfinite(out).all())
                    except Exception as e:  # a kernel that raises fails the gate
                        print(f"[check] D={D} N={N} sigma={sigma} tile {tm}x{tn}: ERROR {type(e).__name__}: {e}")
                        ok = False
                        continue
                    ok &= not bad
                    print(f"[check] D={D:<4} N={N:<5} sigma={sigma:<4} tile {tm}x{tn}: "
                          f"{'FAIL' if bad else 'ok'} (max abs err {float(err.max()):.2e})")
    return ok


# --------------------------------------------------------------------------- timing
def settle_clocks(fn, seconds):
    import torch
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        torch.cuda.synchronize()


def time_fn(fn, warmup=10, reps=30):
    """First call, `warmup` calls, then the median of `reps` HIP-event timings."""
    import torch
    fn()
    torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def causal_flops(B, H, N, D):
    return 2.0 * B * H * N * N * D


def measure(args, impls, tiles):
    import torch
    import torch.nn.functional as F
    fused_attention = load_fused(args.kernel)
    unfused_attention = None
    if "unfused" in impls:
        from attention.fused.unfused import unfused_attention
    dtype = torch_dtype(args.dtype)
    out = []
    g = torch.Generator(device="cuda").manual_seed(0)
    settled = False
    for D in parse_list(args.Ds):
        for N in parse_list(args.Ns):
            q, k, v = (torch.randn(args.B, args.H, N, D, device="cuda", generator=g).to(dtype) for _ in range(3))
            flops = causal_flops(args.B, args.H, N, D)
            for impl in impls:
                for tm, tn in (tiles if impl in ("fused", "unfused") else [("-", "-")]):
                    if impl == "fused":
                        fn = lambda: fused_attention(q, k, v, tm, tn)  # noqa: E731
                    elif impl == "unfused":
                        fn = lambda: unfused_attention(q, k, v, tm, tn)  # noqa: E731
                    else:
                        fn = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True)  # noqa: E731
                    label = f"{impl} {tm}x{tn}" if tm != "-" else impl
                    try:
                        if not settled:
                            settle_clocks(fn, args.settle_s)
                            settled = True
                        ms = time_fn(fn)
                    except Exception as e:
                        print(f"D={D:<4} N={N:<5} {label:<16} FAILED: {type(e).__name__}: {e}")
                        continue
                    tf = flops / (ms * 1e-3) / 1e12
                    print(f"D={D:<4} N={N:<5} {label:<16} {ms:8.3f} ms  {tf:7.2f} TFLOP/s")
                    out.append(dict(D=D, N=N, B=args.B, H=args.H, impl=impl, tile_m=tm, tile_n=tn,
                                    median_ms=f"{ms:.4f}", tflops=f"{tf:.3f}", dtype=args.dtype,
                                    pct_peak=f"{100.0 * tf / PEAK_TFLOPS:.2f}"))
            del q, k, v
            torch.cuda.empty_cache()
    return out


# timing columns of a results CSV and how each is read back; SDPA rows carry no tiles
_ROW_FIELDS = (("D", int), ("N", int), ("B", int), ("H", int), ("impl", str), ("tile_m", str),
               ("tile_n", str), ("median_ms", str), ("tflops", str), ("dtype", str), ("pct_peak", str))


def import_rows(path):
    """Timing rows of a results CSV written by this tracker (rows without a time are skipped)."""
    with open(path) as f:
        found = [r for r in csv.DictReader(f) if r.get("median_ms")]
    rows = []
    for r in found:
        row = {name: conv(r.get(name) or ("-" if name.startswith("tile_") else "")) for name, conv in _ROW_FIELDS}
        if row["impl"] == "sdpa":
            row["tile_m"] = row["tile_n"] = "-"
        rows.append(row)
    return rows


# --------------------------------------------------------------------------- rocprofv3
def profile_target(args):
    """Child-process mode: a few calls of one size for rocprofv3 to record."""
    import torch
    fused_attention = load_fused(args.kernel)
    D, N = parse_list(args.profile_size)
    tm, tn = parse_tiles(args.profile_tile)[0]
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v = (torch.randn(args.B, args.H, N, D, device="cuda", generator=g).to(torch_dtype(args.dtype))
               for _ in range(3))
    for _ in range(3):
        fused_attention(q, k, v, tm, tn)
    torch.cuda.synchronize()


def summarize_counters(values):
    """Percentages from one dispatch's summed counters (names as in COUNTER_PASSES)."""
    out = {}
    cyc = values.get("GRBM_GUI_ACTIVE")
    if cyc:
        per_xcd = cyc / NUM_XCD
        if "SQ_VALU_MFMA_BUSY_CYCLES" in values:
            out["MFMA busy %"] = 100.0 * values["SQ_VALU_MFMA_BUSY_CYCLES"] / (per_xcd * NUM_SIMD)
        if "SQ_VALU_MFMA_COEXEC_CYCLES" in values:
            out["VALU+MFMA co-exec %"] = 100.0 * values["SQ_VALU_MFMA_COEXEC_CYCLES"] / (per_xcd * NUM_SIMD)
        if "SQ_LDS_IDX_ACTIVE" in values:
            out["LDS active %"] = 100.0 * values["SQ_LDS_IDX_ACTIVE"] / (per_xcd * NUM_CU)
        if "SQ_LDS_BANK_CONFLICT" in values:
            out["LDS conflict cycles %"] = 100.0 * values["SQ_LDS_BANK_CONFLICT"] / (per_xcd * NUM_CU)
    mfma = values.get("SQ_INSTS_MFMA")
    if mfma:
        if "SQ_INSTS_VALU" in values:
            out["VALU instr / MFMA"] = (values["SQ_INSTS_VALU"] - mfma) / mfma
        if "SQ_INSTS_VALU_TRANS_F32" in values:
            out["exp-class instr / MFMA"] = values["SQ_INSTS_VALU_TRANS_F32"] / mfma
        if "SQ_INSTS_LDS_LOAD_BANDWIDTH" in values:
            out["LDS bytes read / MFMA"] = 64.0 * values["SQ_INSTS_LDS_LOAD_BANDWIDTH"] / mfma
    if values.get("SQ_WAVE_CYCLES") and "SQ_WAIT_ANY" in values:
        out["wave-wait %"] = 100.0 * values["SQ_WAIT_ANY"] / values["SQ_WAVE_CYCLES"]
    return out


def last_dispatch_counters(csv_path, kernel_regex):
    """Summed counter values of the last dispatch whose kernel name matches kernel_regex."""
    sums, names = {}, {}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            if not re.search(kernel_regex, r["Kernel_Name"]):
                continue
            d = int(r["Dispatch_Id"])
            names[d] = r["Kernel_Name"]
            sums.setdefault(d, {})
            sums[d][r["Counter_Name"]] = sums[d].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    if not sums:
        return None, {}
    d = max(sums)
    return names[d], sums[d]


def run_profile(args, run_dir):
    prof_dir = os.path.join(run_dir, "rocprof")
    os.makedirs(prof_dir, exist_ok=True)
    target = [sys.executable, "-m", "profiling.track_run", "--_profile-target", "--profile-size", args.profile_size,
              "--profile-tile", args.profile_tile, "--B", str(args.B), "--H", str(args.H), "--dtype", args.dtype,
              "--kernel", args.kernel]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    result = {"size": f"D,N = {args.profile_size}, tile {args.profile_tile}, {args.dtype}", "status": "ok"}
    logs = []

    def rocprof(extra, name):
        cmd = ["timeout", "-s", "KILL", str(args.profile_timeout), "rocprofv3", *extra, "--output-format", "csv",
               "-d", os.path.join(prof_dir, name), "-o", name, "--", *target]
        logs.append(" ".join(cmd))
        r = subprocess.run(cmd, cwd=PKG_ROOT, env=env, capture_output=True, text=True)
        with open(os.path.join(prof_dir, f"{name}.log"), "w") as f:
            f.write(r.stdout + "\n" + r.stderr)
        return r.returncode

    if rocprof(["--kernel-trace", "--stats"], "trace") != 0:
        result["status"] = "failed: kernel trace (see rocprof/trace.log)"
        return result, logs
    stats = os.path.join(prof_dir, "trace", "trace_kernel_stats.csv")
    if os.path.exists(stats):
        with open(stats) as f:
            for r in csv.DictReader(f):
                if re.search(args.profile_kernel, r["Name"]):
                    result["kernel"] = r["Name"].split("(")[0]
                    result["avg duration (us)"] = float(r["AverageNs"]) / 1e3
                    break
    counters = {}
    for i, names in enumerate(COUNTER_PASSES, 1):
        if rocprof(["--pmc", *names], f"pmc{i}") != 0:
            result["status"] = f"failed: counter pass {i} (see rocprof/pmc{i}.log)"
            return result, logs
        _, vals = last_dispatch_counters(os.path.join(prof_dir, f"pmc{i}", f"pmc{i}_counter_collection.csv"),
                                         args.profile_kernel)
        counters.update(vals)
    result.update(summarize_counters(counters))
    return result, logs


# --------------------------------------------------------------------------- code diff
def snap_name(path):
    """Where a measured source is kept inside run_NNN/src/: its path below the package root
    (a file outside the package keeps only its name)."""
    rel = os.path.relpath(os.path.join(PKG_ROOT, path), PKG_ROOT)
    return os.path.basename(path) if rel.startswith("..") else rel


def source_at(commit, path):
    """path (relative to the package root) at a git commit, or '' where that is unknown."""
    if not commit or commit == "unknown":
        return ""
    return sh(f"git -C {shlex.quote(PKG_ROOT)} show {shlex.quote(commit)}:./{shlex.quote(path)}")


def previous_sources(records_dir, out_dir, prev, row, paths):
    """{path: text} of the previous run: its src/ snapshot, else git at its commit."""
    snap = os.path.join(out_dir or os.path.join(records_dir, "runs"), f"run_{prev:03d}", "src")
    commit = ((row or {}).get("commit") or "").split(" ")[0]
    out = {}
    for pth in paths:
        f = os.path.join(snap, snap_name(pth))
        out[pth] = open(f).read() if os.path.exists(f) else source_at(commit, pth)
    return out


def code_diff(history, gpu, run, paths, records_dir, out_dir=None):
    """(previous run, unified diff of every measured source) or None when the previous
    run's sources are not known (no snapshot and no usable commit)."""
    prev = find_ref(history, gpu, run, "prev")
    if prev is None:
        return None
    row = next((r for r in history if int(r["run"]) == prev), None)
    old = previous_sources(records_dir, out_dir, prev, row, paths)
    if not any(old.values()):
        return None
    parts = []
    for pth in paths:
        cur = open(os.path.join(PKG_ROOT, pth)).read() if os.path.exists(os.path.join(PKG_ROOT, pth)) else ""
        parts.append("".join(difflib.unified_diff(old[pth].splitlines(True), cur.splitlines(True),
                                                  fromfile=f"Run {prev}: {pth}", tofile=f"Run {run}: {pth}", n=2)))
    d = "".join(parts).rstrip("\n")
    return prev, (d or "(no code changes)")


# --------------------------------------------------------------------------- report
def key_of(r):
    return (int(r["D"]), int(r["N"]), r["impl"], str(r["tile_m"]), str(r["tile_n"]), r.get("dtype", ""))


def find_ref(history, gpu, run, which):
    """Run number to compare `run` with on the same GPU: the latest earlier one ("prev") or the
    earliest ("first"); None for the first run on that GPU."""
    earlier = {int(r["run"]) for r in history if r["gpu"] == gpu and int(r["run"]) < run}
    if not earlier:
        return None
    return max(earlier) if which == "prev" else min(earlier)


def change(new_ms, old_ms):
    """Relative time change of a row against an earlier run's same row, in words."""
    if not old_ms or old_ms <= 0:
        return "-"
    ratio = new_ms / old_ms
    return f"{100.0 * abs(1.0 - ratio):.1f}% {'faster' if ratio <= 1.0 else 'slower'}"


def build_markdown(run, ts, env, note, rows, history, profile=None, reason="", change_txt="", diff=None):
    gpu = env.get("gpu", "")
    prev, base = find_ref(history, gpu, run, "prev"), find_ref(history, gpu, run, "first")
    hist = {(int(r["run"]),) + key_of(r): float(r["median_ms"]) for r in history}
    # heading, then the optional narrative sections (the reference's RUNS.md layout)
    sections = [(None, [f"**Note:** {note}"] if note else []),
                ("Why (from profiling)", [reason] if reason else []),
                ("Change", ([change_txt] if change_txt else [])
                 + ([f"Code diff vs Run {diff[0]}:", "", "```diff", diff[1], "```"] if diff else []))]
    L = [f"## Run {run} — {ts} UTC", ""]
    for title, body in sections:
        if not body:
            continue
        if title:
            L += [f"### {title}", ""]
        L += body + [""]
    labels = [("kernel", "Kernel file"), ("gpu", "GPU"), ("gfx_arch", "Architecture"),
              ("compute_units", "Compute units"), ("gpu_memory_gb", "GPU memory (GB)"),
              ("rocm_smi_clocks", "rocm-smi clocks"), ("torch", "PyTorch"), ("torch_hip", "HIP"),
              ("python", "Python"), ("rocprofv3", "rocprofv3"), ("host", "Host"), ("host_cpus", "Host CPUs"),
              ("commit", "Git commit"), ("B", "Batch B"), ("H", "Heads H"), ("dtype", "dtype"), ("source", "Imported from")]
    L += ["### Environment", "", "| Environment | |", "|---|---|"]
    L += [f"| {name} | {env[k]} |" for k, name in labels if k in env]
    L.append("")
    sdpa = {(r["D"], r["N"]): float(r["median_ms"]) for r in rows if r["impl"] == "sdpa"}
    unf = {(r["D"], r["N"], r["tile_m"], r["tile_n"]): float(r["median_ms"]) for r in rows if r["impl"] == "unfused"}
    head = "| D | N | Tile | Fused ms | Fused TFLOP/s | % of peak | SDPA ms | Fused vs SDPA |"
    sep = "|---|---|---|---|---|---|---|---|"
    if unf:
        head += " Fused vs unfused |"
        sep += "---|"
    head += (f" vs previous run{f' (Run {prev})' if prev else ''} |"
             f" vs first run{f' (Run {base})' if base else ''} |")
    sep += "---|---|"
    L += ["### Result (fused kernel, median of 30 runs)", "", head, sep]
    for r in sorted((r for r in rows if r["impl"] == "fused"), key=lambda r: (r["D"], r["N"], str(r["tile_m"]))):
        ms = float(r["median_ms"])
        s = sdpa.get((r["D"], r["N"]))
        vs = "-" if s is None else (f"{ms / s:.2f}x slower" if ms > s else f"{s / ms:.2f}x faster")
        line = (f"| {r['D']} | {r['N']} | {r['tile_m']}x{r['tile_n']} | {ms:.3f} | {float(r['tflops']):.1f} | "
                f"{r.get('pct_peak') or '-'} | {'-' if s is None else f'{s:.3f}'} | {vs} |")
        if unf:
            u = unf.get((r["D"], r["N"], r["tile_m"], r["tile_n"]))
            line += f" {'-' if u is None else f'{u / ms:.2f}x faster'} |"
        k = key_of(r)
        line += f" {change(ms, hist.get((prev,) + k) if prev else None)} | {change(ms, hist.get((base,) + k) if base else None)} |"
        L.append(line)
    L.append("")
    if prev is None:
        L += ["_First run on this GPU: the baseline for later runs._", ""]
    if profile:
        L += ["### rocprofv3", ""]
        if profile.get("status") != "ok":
            L += [f"Profiling {profile['status']}.", ""]
        else:
            L += [f"{profile.get('kernel', 'kernel')}, {profile['size']}.", "", "| Metric | Value |", "|---|---|"]
            for k, v in profile.items():
                if k in ("status", "size", "kernel"):
                    continue
                L.append(f"| {k} | {v:.2f} |" if isinstance(v, float) else f"| {k} | {v} |")
            L.append("")
    L += ["---", ""]
    return "\n".join(L)


# --------------------------------------------------------------------------- main
def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0],
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--note", default="", help="short title of this run")
    p.add_argument("--reason", default="", help="why the change was made (cite the profile)")
    p.add_argument("--change", default="", help="what was changed, in words (the code diff is added)")
    p.add_argument("--kernel", default=DEFAULT_KERNEL, help="Python file defining fused_attention(q, k, v, tile_m, tile_n)")
    p.add_argument("--records-dir", default=HERE, help="where runs.csv, RUNS.md and runs/ live")
    p.add_argument("--sources", default=DEFAULT_SOURCES,
                   help="comma-separated library sources (relative to the package root) snapshotted with "
                        "the kernel file and diffed against the previous run")
    p.add_argument("--out-dir", default="", help="folder for run_NNN/ (default: <records-dir>/runs)")
    p.add_argument("--no-check", action="store_true", help="skip the correctness gate")
    p.add_argument("--B", type=int, default=2)
    p.add_argument("--H", type=int, default=8)
    p.add_argument("--Ds", default="64,128")
    p.add_argument("--Ns", default="512,2048,8192")
    p.add_argument("--tiles", default="64x64")
    p.add_argument("--dtype", default="fp16", choices=["fp16", "bf16"])
    p.add_argument("--settle-s", type=float, default=1.0, help="untimed seconds before the first timing")
    p.add_argument("--with-unfused", action="store_true")
    p.add_argument("--with-sdpa", action=argparse.BooleanOptionalAction, default=True)
    p.add_argument("--profile", "--ncu", dest="profile", action="store_true",
                   help="also record one size under rocprofv3 (trace + counters)")
    p.add_argument("--profile-size", "--ncu-size", dest="profile_size", default="64,8192", help="D,N")
    p.add_argument("--profile-tile", "--ncu-tile", dest="profile_tile", default="64x64")
    p.add_argument("--profile-kernel", "--ncu-kernel", dest="profile_kernel", default="fwd_kernel",
                   help="regex selecting the kernel in the profiler output")
    p.add_argument("--profile-timeout", type=int, default=120)
    p.add_argument("--import-csv", help="record an existing benchmark CSV as a run instead of measuring")
    p.add_argument("--timestamp", help="for --import-csv: 'YYYY-MM-DD HH:MM' (UTC)")
    p.add_argument("--gpu", help="for --import-csv: GPU name")
    p.add_argument("--commit", help="git commit of the measured code (for --import-csv, or where git is absent)")
    p.add_argument("--_profile-target", dest="profile_target", action="store_true", help=argparse.SUPPRESS)
    return p.parse_args(argv)


def main(argv=None):
    args = parse_args(argv)
    for path in (PKG_ROOT,):
        if path not in sys.path:
            sys.path.insert(0, path)
    if args.profile_target:
        profile_target(args)
        return 0
    rec = Records(args.records_dir)
    history = rec.history()
    run = rec.next_run(history)
    if args.import_csv:
        rows = import_rows(args.import_csv)
        ts = args.timestamp or now_utc()
        env = {"gpu": args.gpu or "unknown", "commit": args.commit or "unknown", "kernel": "",
               "B": rows[0]["B"] if rows else "", "H": rows[0]["H"] if rows else "", "source": args.import_csv}
        md = build_markdown(run, ts, env, args.note, rows, history, None, args.reason, args.change)
        rec.append(run, ts, env, args.note, rows, md, rec.run_dir(run, args.out_dir))
        print(md)
        return 0
    # a relative kernel path names a file below the working directory or the package root
    if not os.path.exists(args.kernel) and not os.path.exists(os.path.join(PKG_ROOT, args.kernel)):
        sys.exit(f"kernel file not found: {args.kernel}")
    ts = now_utc()
    env = collect_env(args)
    env["kernel"] = args.kernel
    if args.commit:
        env["commit"] = args.commit
    if not args.no_check:
        print(f"Checking {args.kernel} against the fp32 reference ...")
        if not check_correctness(load_fused(args.kernel), parse_tiles(args.tiles), torch_dtype(args.dtype), args.B, args.H):
            sys.exit("correctness check FAILED: run not recorded (fix the kernel, or use --no-check)")
    print(f"Run {run} — {ts} UTC — {env['gpu']} ({env['gfx_arch']}) — commit {env['commit']}")
    impls = ["fused"] + (["sdpa"] if args.with_sdpa else []) + (["unfused"] if args.with_unfused else [])
    rows = measure(args, impls, parse_tiles(args.tiles))
    run_dir = rec.run_dir(run, args.out_dir)
    profile, logs = (run_profile(args, run_dir) if args.profile else (None, []))
    paths = [args.kernel] + [x for x in args.sources.split(",") if x]
    diff = code_diff(history, env["gpu"], run, paths, args.records_dir, args.out_dir)
    md = build_markdown(run, ts, env, args.note, rows, history, profile, args.reason, args.change, diff)
    extra = {os.path.join("src", snap_name(pth)): open(os.path.join(PKG_ROOT, pth)).read()
             for pth in paths if os.path.exists(os.path.join(PKG_ROOT, pth))}
    if diff:
        extra["change.diff"] = diff[1] + "\n"
    if logs:
        extra["rocprof_commands.txt"] = "\n".join(logs) + "\n"
    rec.append(run, ts, env, args.note, rows, md, run_dir, extra)
    print("\n" + md)
    print(f"saved run {run}: {rec.md}, {rec.csv}, {run_dir}/")
    return 0


if __name__ == "__main__":
    sys.exit(main())
