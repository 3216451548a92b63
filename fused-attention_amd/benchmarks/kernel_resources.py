"""Registers, LDS, scratch and waves per SIMD of every kernel instance, from the compiler.

    python -m benchmarks.kernel_resources [--hipcc /opt/rocm/bin/hipcc] [--out FILE.md]

Compiles each (kernel family, element type, head dim) slice of csrc/ the way the
Makefile does, adding `-Rpass-analysis=kernel-resource-usage`, and tabulates the
compiler's own report per kernel: VGPRs, AGPRs, SGPRs, spills, scratch bytes per lane,
LDS bytes per workgroup and the occupancy in waves per SIMD those allow.  These are the
static half of the tile study (benchmarks/tile_study.py measures the run-time half with
rocprofv3 counters).  Needs no GPU.
"""

import argparse
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "csrc")
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-fvisibility=hidden", "-Wno-unused-command-line-argument",
         "-Rpass-analysis=kernel-resource-usage", "-c", "-o", os.devnull]
SLICES = [(e, d) for e in ("bf16", "f16") for d in (128, 64, 32)]
FIELDS = ["VGPRs", "AGPRs", "TotalSGPRs", "ScratchSize [bytes/lane]", "Occupancy [waves/SIMD]",
          "SGPRs Spill", "VGPRs Spill", "LDS Size [bytes/block]"]


def makefile_sched():
    """The Makefile's machine-scheduler options per object group ({variable: [flags]})."""
    text = open(os.path.join(CSRC, "Makefile")).read()
    raw = dict(re.findall(r"^(ILP|SCHED_\w+)\s*[:?]?=[ \t]*(.*)$", text, re.M))
    return {k: v.replace("$(ILP)", raw.get("ILP", "")).split() for k, v in raw.items()}


def objects():
    """(family, etype, D, forward part, scheduler flags) of every object the Makefile builds:
    the D = 128 forward as its one-head part and its grouped part, the other forward slices
    whole, the backward per slice, each under its group's scheduler options."""
    sch = makefile_sched()
    out = []
    for e, d in SLICES:
        if d == 128:
            out += [("fwd", e, d, 1, sch["SCHED_FWD1"]), ("fwd", e, d, 2, sch["SCHED_FWDG"]),
                    ("bwd", e, d, 0, sch["SCHED_BWD128"])]
        else:
            out += [("fwd", e, d, 0, sch["SCHED_FWD"]), ("bwd", e, d, 0, sch["SCHED_BWD"])]
    return out


def sched_name(flags):
    """Short name of a scheduler option list: 'max-ilp, topdown', 'bottomup', 'default'."""
    names = [f.split("=", 1)[1] for f in flags if "=" in f]
    return ", ".join(names) if names else "default"


def compile_slice(hipcc, family, etype, D, part, sched):
    et = "fa::BF16" if etype == "bf16" else "fa::F16"
    if family == "fwd":
        defs = [f"-DFA_FWD_PART={part}", f"-DFA_FWD_TABLE=fa_fwd_table_{etype}_{D}",
                f"-DFA_FWD_TABLE_GROUPED=fa_fwd_table_{etype}_{D}_grouped"]
    else:
        defs = [f"-DFA_BWD_TABLE=fa_bwd_table_{etype}_{D}"]
    src = os.path.join(CSRC, f"fa_{family}.hip")
    r = subprocess.run([hipcc, *FLAGS, *sched, f"-DFA_ETYPE={et}", f"-DFA_D={D}", *defs, src],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{src} ({etype}, D={D}, part {part}) failed:\n{r.stderr[-2000:]}")
    kernels = parse(r.stderr)
    for k in kernels.values():
        k["Scheduler"] = sched_name(sched)
    return kernels


def demangle(name):
    try:
        out = subprocess.run(["c++filt", name], capture_output=True, text=True).stdout.strip()
    except OSError:
        return name
    m = re.match(r"void (fa::\w+<[^>]*>)", out)
    return m.group(1) if m else out


def parse(text):
    """{mangled kernel name: {field: value}} from the remarks."""
    kernels, cur = {}, None
    for line in text.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = kernels.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([^:]+(?:\[[^\]]*\])?): (\S+) \[-Rpass-analysis", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = m.group(2)
    return kernels


HEADER = [
    "# Registers, LDS, scratch and occupancy of every kernel instance (compiler report, gfx950)",
    "",
    "    cd fused-attention_amd && python3 -m benchmarks.kernel_resources --out ../profiles/kernel_resources.md",
    "",
    "Each object of `csrc/` compiled as the Makefile does with `-Rpass-analysis=kernel-resource-usage`;",
    "\"Occupancy\" is the compiler's waves per SIMD for the registers and LDS; \"Scheduler\" the machine",
    "scheduler options its object is built under (the Makefile's `SCHED_*`: strategy, pre-RA direction).",
    "Template arguments:",
    "`fwd_kernel<E, D, rows per head, keys per tile, heads per workgroup, LSE>`,",
    "`dq_kernel<E, D, rows, keys>`, `dkdv_kernel<E, D, query rows per tile, keys per workgroup, per-row terms>`,",
    "`dkdv_pair_kernel<E, D, query rows per tile, keys per workgroup>` (D = 128 only).",
    "",
]


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--hipcc", default="/opt/rocm/bin/hipcc")
    p.add_argument("--out", default="")
    args = p.parse_args(argv)
    jobs = sorted(objects(), key=lambda j: (j[0] != "fwd", j[1], -j[2], j[3]))
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        results = list(ex.map(lambda j: compile_slice(args.hipcc, *j), jobs))
    cols = FIELDS + ["Scheduler"]
    L = HEADER + ["| kernel | " + " | ".join(cols) + " |", "|---|" + "---|" * len(cols)]
    for kernels in results:
        for name in sorted(kernels, key=demangle):
            k = kernels[name]
            L.append(f"| `{demangle(name)}` | " + " | ".join(k.get(f, "-") for f in cols) + " |")
    text = "\n".join(L) + "\n"
    if args.out:
        with open(args.out, "w") as f:
            f.write(text)
    sys.stdout.write(text)


if __name__ == "__main__":
    main()
