"""Tile and occupancy study: rocprofv3 counters behind every workgroup-shape rule.

    python -m benchmarks.tile_study --out-dir DIR [--groups fwd,gqa,dq,dkdv] [--calls 3]

The library picks its workgroup shapes by rules (fa_api.hip): rows per forward and dQ
workgroup (`fwd_block_m`, `dq_block_m`), query heads per forward workgroup
(`heads_per_wg`, `fwd_heads_per_wg`) and the dK/dV split (`dkdv_nsplit`).  This script
runs each rule's chosen shape beside its rejected ones -- literally, through
fa_fwd_exact / fa_bwd_gqa_exact -- under rocprofv3 (one kernel-trace pass and two
counter passes, each in a child process of its own) and writes, per variant: kernel
time, achieved TFLOP/s against the dense MFMA peak, algorithmic HBM GB/s, MFMA busy,
VALU/MFMA co-execution, LDS activity and bank-conflict cycles, instructions per MFMA
and the wave-wait fraction.  Registers, LDS and the waves per SIMD they allow are
compile-time facts: `python -m benchmarks.kernel_resources` prints the compiler's own figures.  The
reference backs its tile choice the same way, with one profiler run per tile
(profiling/3_tile_study/README.md:8-19).

Run it from fused-attention_amd/ with rocprofv3 on PATH; TMPDIR should be writable.
"""

import argparse
import csv
import json
import math
import os
import re
import statistics
import subprocess
import sys

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if PKG_ROOT not in sys.path:
    sys.path.insert(0, PKG_ROOT)

PEAK_TFLOPS = 2516.6          # MI355X dense bf16/fp16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
NUM_XCD, NUM_SIMD, NUM_CU = 8, 1024, 256

PASSES = [
    ("trace", ["--kernel-trace"]),
    ("pmc1", ["--pmc", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU",
              "SQ_INSTS_VALU_TRANS_F32", "SQ_BUSY_CYCLES", "SQ_WAVES", "GRBM_GUI_ACTIVE"]),
    ("pmc2", ["--pmc", "SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_LDS_LOAD_BANDWIDTH", "SQ_WAIT_ANY",
              "SQ_WAVE_CYCLES", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_VALU", "GRBM_GUI_ACTIVE"]),
]

# ---------------------------------------------------------------------------- variants
# Workloads: (B, H, H_kv, S, D, dtype)
CFG2 = (4, 32, 32, 4096, 128, "bf16")          # the headline MHA shape
CFG3 = (2, 32, 8, 8192, 128, "bf16")           # GQA, group 4
SMALL_GQA = (2, 8, 1, 8192, 128, "fp16")       # few workgroups: the 4 -> 2 heads rule
MQA_BWD = (1, 32, 1, 4096, 64, "fp16")         # few key tiles: the dK/dV split
MHA_FEW = (2, 8, 8, 2048, 128, "bf16")         # heaviest key tile < 64 pairs: no split


def variants(groups):
    """(group, name, workload, kind, params, rule note) in run order."""
    out = []
    if "fwd" in groups:
        for D in (128, 64, 32):
            wl = (4, 32, 32, 4096, D, "bf16")
            for bm, bn in ((64, 64), (128, 64), (64, 128), (128, 128)):
                out.append(("fwd", f"fwd D={D} rows {bm} keys {bn}", wl, "fwd", dict(bm=bm, bn=bn, gh=1), ""))
    if "gqa" in groups:
        for bm, bn, gh in ((64, 64, 1), (64, 64, 2), (64, 64, 4), (128, 64, 1), (128, 64, 2), (64, 128, 2)):
            out.append(("gqa", f"gqa rows {bm} keys {bn} heads/wg {gh}", CFG3, "fwd", dict(bm=bm, bn=bn, gh=gh), ""))
        for gh in (2, 4):
            out.append(("gqa", f"gqa-few rows 64 keys 64 heads/wg {gh}", SMALL_GQA, "fwd", dict(bm=64, bn=64, gh=gh), ""))
    if "dq" in groups:
        for D in (128, 64):
            wl = (4, 32, 32, 4096, D, "bf16")
            for bm, bn in ((64, 64), (128, 64), (64, 128), (128, 128)):
                out.append(("dq", f"bwd D={D} dQ rows {bm} keys {bn}", wl, "bwd", dict(bm=bm, bn=bn, nsplit=1), ""))
    if "dkdv" in groups:
        for ns in (1, 4, 16, 64):
            out.append(("dkdv", f"mqa-bwd split {ns}", MQA_BWD, "bwd", dict(bm=64, bn=64, nsplit=ns), ""))
        for ns in (1, 2):
            out.append(("dkdv", f"cfg2-bwd split {ns}", CFG2, "bwd", dict(bm=128, bn=64, nsplit=ns), ""))
        for ns in (1, 16):
            out.append(("dkdv", f"mha-few-bwd split {ns}", MHA_FEW, "bwd", dict(bm=128, bn=64, nsplit=ns), ""))
    if "rules" in groups:  # the shapes behind the dispatch rules' thresholds
        for D in (128, 64, 32):
            for gh in (2, 4):
                out.append(("rules", f"gqa-few D={D} heads/wg {gh}", (2, 8, 1, 8192, D, "fp16"), "fwd",
                            dict(bm=64, bn=64, gh=gh), ""))
        for gh in (2, 4):
            out.append(("rules", f"gqa-small heads/wg {gh}", (1, 16, 4, 4096, 128, "bf16"), "fwd",
                        dict(bm=64, bn=64, gh=gh), ""))
        for D in (32,):
            for bm in (64, 128):
                out.append(("rules", f"bwd D={D} dQ rows {bm} keys 64", (4, 32, 32, 4096, D, "bf16"), "bwd",
                            dict(bm=bm, bn=64, nsplit=1), ""))
        for wl, splits in (((1, 32, 1, 16384, 64, "fp16"), (4, 8, 16, 32)),
                           ((1, 8, 1, 16384, 128, "bf16"), (4, 8, 16, 32)),
                           ((1, 32, 4, 8192, 128, "bf16"), (1, 2, 4, 8)),
                           ((1, 8, 8, 4096, 128, "bf16"), (1, 2, 4)),
                           ((1, 16, 16, 8192, 128, "bf16"), (1, 2, 4)),
                           ((2, 32, 32, 8192, 128, "bf16"), (1, 2))):
            for ns in splits:
                out.append(("rules", "split {} B{} H{} Hkv{} S{} D{}".format(ns, *wl[:5]), wl, "bwd",
                            dict(bm=64, bn=64, nsplit=ns), ""))
    if "splits" in groups:  # the dK/dV split rule: both dK/dV kernels, several grid sizes
        for wl, splits in (((1, 32, 1, 4096, 128, "bf16"), (4, 8, 16, 32)),
                           ((1, 4, 4, 8192, 128, "bf16"), (1, 2, 4, 8)),
                           ((1, 8, 8, 4096, 128, "bf16"), (1, 2, 4)),
                           ((1, 32, 4, 8192, 128, "bf16"), (1, 2, 4)),
                           ((1, 8, 1, 16384, 128, "bf16"), (4, 8, 16)),
                           ((1, 32, 1, 4096, 64, "fp16"), (8, 16, 32, 64)),
                           ((1, 16, 16, 4096, 64, "fp16"), (1, 2, 4)),
                           ((2, 16, 16, 4096, 64, "fp16"), (1, 2, 4)),
                           ((1, 32, 1, 16384, 64, "fp16"), (8, 16, 32))):
            for ns in splits:
                out.append(("splits", "split {} B{} H{} Hkv{} S{} D{}".format(ns, *wl[:5]), wl, "bwd",
                            dict(bm=64, bn=64, nsplit=ns), ""))
    return out


def causal_matmul_flops(B, H, S, D):
    """One causal S x S x D product over B*H heads (2 FLOP per multiply-add, half the square)."""
    return float(B) * H * S * S * D


# ---------------------------------------------------------------------------- child: run the variants
def _inputs(torch, wl, cache):
    """Device inputs of workload wl (made once per workload: the forward that writes O and LSE
    for the backward variants is one extra library dispatch, counted as the variant's `pre`)."""
    if wl in cache:
        return cache[wl], 0
    from attention import _lib
    cache.clear()
    torch.cuda.empty_cache()
    B, H, Hkv, S, D, dt = wl
    dtype = torch.bfloat16 if dt == "bf16" else torch.float16
    g = torch.Generator(device="cuda").manual_seed(0)
    q, do = (torch.randn(B, H, S, D, device="cuda", generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(B, Hkv, S, D, device="cuda", generator=g).to(dtype) for _ in range(2))
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device="cuda", dtype=torch.float32)
    _lib.fwd(q, k, v, o, lse, 64, 64)
    outs = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v))
    cache[wl] = (q, k, v, o, do, lse, outs)
    return cache[wl], 1


def run_target(args):
    import ctypes

    import torch

    from attention import _lib
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)  # noqa: E731
    cache = {}
    stream = torch.cuda.current_stream()
    if args.warm_s > 0:  # settle the clocks with torch work (not this library's kernels)
        import time
        a = torch.randn(4096, 4096, device="cuda", dtype=torch.bfloat16)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < args.warm_s:
            for _ in range(8):
                a = (a @ a).clamp_(-1, 1)
            torch.cuda.synchronize()
        del a
    todo = variants(args.groups.split(",")) * args.rounds
    for group, name, wl, kind, prm, _ in todo:
        (q, k, v, o, do, lse, (dq, dk, dv)), pre = _inputs(torch, wl, cache)
        B, H, Hkv, S, D, dt = wl
        code_dt = _lib.dtype_code(q.dtype)
        st = ctypes.c_void_p(stream.cuda_stream)
        if kind == "fwd":
            def call():
                return lib.fa_fwd_exact(P(q), P(k), P(v), P(o), P(None), B, H, Hkv, S, D, code_dt,
                                        _lib.scale_log2(D), prm["bm"], prm["bn"], prm["gh"], st)
            per_call = 1
        else:
            ns = prm["nsplit"]
            nbytes = (8 * B * H * S + 255) // 256 * 256 + (8 * B * Hkv * ns * S * D if ns > 1 else 0)
            ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")

            def call(ws=ws, nbytes=nbytes, ns=ns):
                return lib.fa_bwd_gqa_exact(P(q), P(k), P(v), P(o), P(do), P(lse), P(dq), P(dk), P(dv),
                                            B, H, Hkv, S, D, code_dt, _lib.scale_log2(D), 1.0 / math.sqrt(D),
                                            prm["bm"], prm["bn"], ns, P(ws), nbytes, st)
            per_call = 2 + (1 if ns > 1 else 0)
        for _ in range(args.calls):
            rc = call()
            if rc != 0:
                raise RuntimeError(f"{name}: {_lib.strerror(rc)}")
        torch.cuda.synchronize()
        print("VARIANT " + json.dumps({"name": name, "pre": pre, "per_call": per_call, "calls": args.calls}),
              flush=True)


# ---------------------------------------------------------------------------- parent: profile and report
def fa_dispatches(path):
    """[(dispatch id, {name, row, counters})] of this library's kernels, in dispatch order."""
    rows = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if "fa::" not in name:
                continue
            d = int(r["Dispatch_Id"])
            e = rows.setdefault(d, {"name": name, "row": r, "counters": {}})
            if "Counter_Name" in r:
                e["counters"][r["Counter_Name"]] = e["counters"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [(d, rows[d]) for d in sorted(rows)]


def split_by_variant(disp, manifest):
    """Dispatch records per variant: the last call's dispatches, plus every call's (for timing)."""
    out, i = [], 0
    for m in manifest:
        i += m["pre"]
        n = m["per_call"] * m["calls"]
        block = disp[i:i + n]
        if len(block) != n:
            raise RuntimeError(f"dispatch count mismatch at {m['name']}: {len(block)} of {n}")
        calls = [block[c * m["per_call"]:(c + 1) * m["per_call"]] for c in range(m["calls"])]
        out.append(calls)
        i += n
    if i != len(disp):
        raise RuntimeError(f"{len(disp) - i} dispatches left over")
    return out


def short_kernel(name):
    m = re.search(r"fa::(\w+)<([^>]*)>", name)
    return f"{m.group(1)}<{m.group(2)}>" if m else name.split("(")[0]


def derive(c):
    out = {}
    cyc = c.get("GRBM_GUI_ACTIVE")
    if cyc:
        per_xcd = cyc / NUM_XCD
        if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            out["mfma_busy"] = 100.0 * c["SQ_VALU_MFMA_BUSY_CYCLES"] / (per_xcd * NUM_SIMD)
        if "SQ_VALU_MFMA_COEXEC_CYCLES" in c:
            out["coexec"] = 100.0 * c["SQ_VALU_MFMA_COEXEC_CYCLES"] / (per_xcd * NUM_SIMD)
        if "SQ_LDS_IDX_ACTIVE" in c:
            out["lds_active"] = 100.0 * c["SQ_LDS_IDX_ACTIVE"] / (per_xcd * NUM_CU)
        if "SQ_LDS_BANK_CONFLICT" in c:
            out["lds_conflict"] = 100.0 * c["SQ_LDS_BANK_CONFLICT"] / (per_xcd * NUM_CU)
    mf = c.get("SQ_INSTS_MFMA")
    if mf:
        if "SQ_INSTS_VALU" in c:
            out["valu_per_mfma"] = (c["SQ_INSTS_VALU"] - mf) / mf
        if "SQ_INSTS_VALU_TRANS_F32" in c:
            out["trans_per_mfma"] = c["SQ_INSTS_VALU_TRANS_F32"] / mf
        if "SQ_INSTS_LDS_LOAD_BANDWIDTH" in c:
            out["lds_bytes_per_mfma"] = 64.0 * c["SQ_INSTS_LDS_LOAD_BANDWIDTH"] / mf
    if c.get("SQ_WAVE_CYCLES") and "SQ_WAIT_ANY" in c:
        out["wave_wait"] = 100.0 * c["SQ_WAIT_ANY"] / c["SQ_WAVE_CYCLES"]
    if c.get("SQ_WAVE_CYCLES") and "SQ_WAIT_INST_LDS" in c:
        out["lds_wait"] = 100.0 * c["SQ_WAIT_INST_LDS"] / c["SQ_WAVE_CYCLES"]
    return out


def kernel_flops_bytes(kernel, wl):
    """Executed FLOPs and algorithmic HBM bytes of one dispatch of `kernel` on workload wl."""
    B, H, Hkv, S, D, _ = wl
    mm = causal_matmul_flops(B, H, S, D)
    e = 2
    if kernel.startswith("fwd_kernel"):
        return 2 * mm, e * S * D * (2 * B * H + 2 * B * Hkv)
    if kernel.startswith("dq_kernel"):
        return 3 * mm, e * S * D * (4 * B * H + 2 * B * Hkv) + 4 * B * H * S
    if kernel.startswith("dkdv_kernel") or kernel.startswith("dkdv_pair_kernel"):
        return 4 * mm, e * S * D * (2 * B * H + 4 * B * Hkv) + 8 * B * H * S
    return 0.0, 4 * 2 * B * Hkv * S * D  # the split's reduction: fp32 partial sums read (per chunk, at least)


def profile(args):
    os.makedirs(args.out_dir, exist_ok=True)
    env = dict(os.environ)
    env.setdefault("TMPDIR", "/tmp")
    def child(calls, warm, rounds):
        return [sys.executable, "-m", "benchmarks.tile_study", "--_target", "--groups", args.groups,
                "--calls", str(calls), "--warm-s", str(warm), "--rounds", str(rounds)]
    results = {}
    manifest = None
    commands = []
    for name, extra in PASSES:
        d = os.path.join(args.out_dir, name)
        timed = name == "trace"   # the timing pass warms the clocks first and takes more calls
        cmd = ["timeout", "-s", "KILL", str(args.pass_timeout), "rocprofv3", *extra, "--output-format", "csv",
               "-d", d, "-o", name, "--",
               *child(args.calls if timed else 2, args.warm_s if timed else 0, args.rounds if timed else 1)]
        commands.append(" ".join(cmd))
        print(f"[tile_study] pass {name}: {' '.join(extra)}", flush=True)
        log = os.path.join(args.out_dir, f"{name}.log")
        with open(log, "w") as f:   # streamed: the log grows as the variants finish
            r = subprocess.run(cmd, cwd=PKG_ROOT, env=env, stdout=f, stderr=subprocess.STDOUT, text=True)
        with open(log) as f:
            man = [json.loads(ln[8:]) for ln in f.read().splitlines() if ln.startswith("VARIANT ")]
        if r.returncode != 0 and len(man) != len(variants(args.groups.split(","))) * (args.rounds if timed else 1):
            sys.exit(f"pass {name} failed (rc {r.returncode}); see {args.out_dir}/{name}.log")
        manifest = man
        csv_name = "kernel_trace" if name == "trace" else "counter_collection"
        path = os.path.join(d, f"{name}_{csv_name}.csv")
        if not os.path.exists(path):
            found = [os.path.join(dp, fn) for dp, _, fns in os.walk(d) for fn in fns if fn.endswith(csv_name + ".csv")]
            if not found:
                sys.exit(f"pass {name}: no {csv_name}.csv under {d}")
            path = found[0]
        # per variant name: every call of every round, in order
        per_name = {}
        for m, calls in zip(manifest, split_by_variant(fa_dispatches(path), manifest)):
            per_name.setdefault(m["name"], []).append(calls)
        results[name] = per_name
    rows = []
    for group, vname, wl, kind, prm, _ in variants(args.groups.split(",")):
        rounds = results["trace"][vname]           # [round][call][dispatch]
        last = {k: results[k][vname][-1][-1] for k in ("pmc1", "pmc2")}
        for pos in range(len(rounds[-1][-1])):
            _, rec = rounds[-1][-1][pos]
            kern = short_kernel(rec["name"])
            # every call but the first of each round
            durs = [(int(c[pos][1]["row"]["End_Timestamp"]) - int(c[pos][1]["row"]["Start_Timestamp"])) / 1e3
                    for calls in rounds for c in (calls[1:] or calls)]
            us = statistics.median(durs)
            flops, nbytes = kernel_flops_bytes(kern, wl)
            counters = {}
            for k in ("pmc1", "pmc2"):
                counters.update(last[k][pos][1]["counters"])
            rows.append(dict(group=group, variant=vname, workload="B{} H{} Hkv{} S{} D{} {}".format(*wl),
                             kernel=kern, us=us, tflops=flops / (us * 1e-6) / 1e12 if flops else 0.0,
                             gbs=nbytes / (us * 1e-6) / 1e9, **derive(counters)))
    with open(os.path.join(args.out_dir, "tile_study.json"), "w") as f:
        json.dump({"rows": rows, "commands": commands}, f, indent=1)
    md = report(rows, commands)
    with open(os.path.join(args.out_dir, "tile_study.md"), "w") as f:
        f.write(md)
    print(md)


def report(rows, commands):
    cols = [("kernel", "kernel", "{}"), ("us", "µs", "{:.1f}"), ("tflops", "TFLOP/s (executed)", "{:.0f}"),
            ("pct", "% of peak", "{:.1f}"), ("gbs", "GB/s (algorithmic)", "{:.0f}"),
            ("mfma_busy", "MFMA busy %", "{:.1f}"), ("coexec", "VALU+MFMA co-exec %", "{:.1f}"),
            ("lds_active", "LDS active %", "{:.1f}"), ("lds_conflict", "LDS conflict %", "{:.1f}"),
            ("valu_per_mfma", "VALU/MFMA", "{:.2f}"), ("trans_per_mfma", "exp/MFMA", "{:.2f}"),
            ("lds_bytes_per_mfma", "LDS B/MFMA", "{:.0f}"), ("wave_wait", "wave-wait %", "{:.1f}"),
            ("lds_wait", "LDS-wait %", "{:.1f}")]
    L = ["| variant | workload | " + " | ".join(c[1] for c in cols) + " |",
         "|---|---|" + "---|" * len(cols)]
    for r in rows:
        r = dict(r, pct=100.0 * r["tflops"] / PEAK_TFLOPS)
        cells = []
        for key, _, fmt in cols:
            v = r.get(key)
            cells.append("-" if v is None or (key == "tflops" and not v) or (key == "pct" and not r["tflops"])
                         else fmt.format(v))
        L.append(f"| {r['variant']} | {r['workload']} | " + " | ".join(cells) + " |")
    L += ["", "Commands (from fused-attention_amd/):", ""] + [f"    {c}" for c in commands] + [""]
    return "\n".join(L)


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--out-dir", default=os.path.join(os.path.dirname(PKG_ROOT), "out", "tile_study"))
    p.add_argument("--groups", default="fwd,gqa,dq,dkdv")
    p.add_argument("--rounds", type=int, default=3,
                   help="passes over all variants in the timing pass (interleaves them in time)")
    p.add_argument("--calls", type=int, default=8,
                   help="calls per variant and round in the timing pass (median over all calls but the "
                        "first of each round); the counter passes make 2 and keep the last one's counters")
    p.add_argument("--warm-s", type=float, default=2.0, help="seconds of untimed GPU work before the timing pass")
    p.add_argument("--pass-timeout", type=int, default=240)
    p.add_argument("--_target", dest="target", action="store_true", help=argparse.SUPPRESS)
    return p.parse_args(argv)


def main(argv=None):
    args = parse_args(argv)
    if args.target:
        run_target(args)
    else:
        profile(args)


if __name__ == "__main__":
    main()
