"""Set this build's per-case correctness records beside the reference's committed ones.

    python tests/records/compare_with_reference.py [--ours results/correctness]
        [--reference /root/reference/results/correctness] [--out results/correctness/README.md]

Both sides are CSVs in the reference's layout (one row per case): the forward suite
(84 MHA cases x 4 tiles: max_abs_err, max_rel_err, tol_ratio), the GQA suite (96 cases)
and the backward suite (7 shapes: relative Frobenius error of O, dQ, dK, dV).  The GPU
suites under tests/ write this build's rows (tests/gpu_util.py, conftest.py); the
reference's rows are its committed results (results/correctness/...).  This script only
reads CSV files.
"""

import argparse
import csv
import glob
import math
import os

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def load(path):
    with open(path) as f:
        return list(csv.DictReader(f))


def fnum(x):
    try:
        return float(x)
    except (TypeError, ValueError):
        return math.nan


def suite_section(title, ours_glob, ref_glob, key="case"):
    L = [f"## {title}", ""]
    ours = {os.path.basename(os.path.dirname(p)): load(p) for p in sorted(glob.glob(ours_glob))}
    refs = {os.path.basename(os.path.dirname(p)): load(p) for p in sorted(glob.glob(ref_glob))}
    if not ours:
        return L + ["(no records of this build)", ""]
    L += ["| tile | cases (this build) | passed | worst max_abs_err | worst tol_ratio | reference cases | "
          "reference worst max_abs_err | reference worst tol_ratio | cases where this build's max_abs_err "
          "is lower |", "|---|---|---|---|---|---|---|---|---|"]
    for tile in sorted(set(ours) | set(refs)):
        o, r = ours.get(tile, []), refs.get(tile, [])
        ro = {row[key]: row for row in r}
        lower = sum(1 for row in o if row[key] in ro and fnum(row["max_abs_err"]) < fnum(ro[row[key]]["max_abs_err"]))
        common = sum(1 for row in o if row[key] in ro)
        w = lambda rows, c: max((fnum(x[c]) for x in rows), default=math.nan)  # noqa: E731
        L.append(f"| {tile} | {len(o)} | {sum(x['result'] == 'PASS' for x in o)} | {w(o, 'max_abs_err'):.3e} | "
                 f"{w(o, 'tol_ratio'):.3f} | {len(r)} | {w(r, 'max_abs_err'):.3e} | {w(r, 'tol_ratio'):.3f} | "
                 f"{lower} of {common} |")
    # per case at the reference's default tile
    tile = "64x64" if "64x64" in ours else sorted(ours)[0]
    o, r = ours.get(tile, []), {row[key]: row for row in refs.get(tile, [])}
    L += ["", f"Per case, tile {tile} (this build / reference):", "",
          "| case | max_abs_err | reference max_abs_err | tol_ratio | reference tol_ratio | result |",
          "|---|---|---|---|---|---|"]
    for row in o:
        rr = r.get(row[key], {})
        L.append(f"| {row[key]} | {fnum(row['max_abs_err']):.3e} | {fnum(rr.get('max_abs_err')):.3e} | "
                 f"{fnum(row['tol_ratio']):.4f} | {fnum(rr.get('tol_ratio')):.4f} | {row['result']} |")
    return L + [""]


def backward_section(ours_glob, ref_path):
    L = ["## Backward suite (relative Frobenius error vs fp32 autograd)", ""]
    ours = sorted(glob.glob(ours_glob))
    ref = [r for r in load(ref_path) if r["test"] == "correctness"] if os.path.exists(ref_path) else []
    if not ours:
        return L + ["(no records of this build)", ""]
    rkey = {(r["B"], r["H"], r["N"], r["D"], str(fnum(r["sigma"]))): r for r in ref}
    L += ["| file | B | H | N | D | sigma | O | dQ | dK | dV | reference O | reference dQ | reference dK | "
          "reference dV | result |", "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for p in ours:
        for row in load(p):
            rr = rkey.get((row["B"], row["H"], row["N"], row["D"], str(fnum(row["sigma"]))), {})
            L.append(f"| {os.path.basename(p)} | {row['B']} | {row['H']} | {row['N']} | {row['D']} | {row['sigma']} | "
                     + " | ".join(row[f"relerr_{n}"] for n in ("O", "dQ", "dK", "dV")) + " | "
                     + " | ".join(rr.get(f"relerr_{n}", "-") for n in ("O", "dQ", "dK", "dV"))
                     + f" | {row['result']} |")
    return L + [""]


def margins_section(path):
    """The full-size workloads' error margins (written by the GPU suites; no reference counterpart:
    the reference records its suites' cases only)."""
    L = ["## Full-size workloads: error margins", ""]
    if not os.path.exists(path):
        return L + ["(no records of this build)", ""]
    rows = load(path)
    L += ["Max-abs error of each output against the fp32 reference on every element (the north-star bar "
          "is 2e-2), its ratio to that bar, and the other measures the test applies: the mixed ratio "
          "max |x-r| / (2e-2 + 2e-2 |r|) (forward suites, and dK / dV of a K/V group), the relative "
          "Frobenius error (backward), the float64 oracle's max-abs on sampled heads or rows.", "",
          "| workload | dtype | tiles | output | max_abs_err | / 2e-2 | mixed ratio | rel. Frobenius | oracle max_abs |",
          "|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        bar = fnum(r["bar"])
        L.append(f"| {r['test']} | {r['dtype']} | {r['tiles']} | {r['output']} | {r['max_abs_err']} | "
                 f"{fnum(r['max_abs_err']) / bar:.3f} | {r['mixed_tol_ratio']} | {r['rel_frobenius']} | "
                 f"{r['oracle_max_abs']} |" if bar == 2e-2 else
                 f"| {r['test']} | {r['dtype']} | {r['tiles']} | {r['output']} (bar {r['bar']}) | {r['max_abs_err']} | "
                 f"{r['max_abs_over_bar']} | | | |")
    return L + [""]


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--ours", default=os.path.join(REPO, "results", "correctness"))
    p.add_argument("--reference", default="/root/reference/results/correctness")
    p.add_argument("--out", default="")
    p.add_argument("--commit", default="", help="the commit whose GPU run wrote this build's CSVs")
    a = p.parse_args(argv)
    L = ["# Per-case correctness: this build (MI355X, libfa.so) beside the reference's committed records",
         "", "Reference: its committed CSVs (`results/correctness/fused/v3_occupancy2/*`, "
         "`results/correctness/fused_gqa/v0_baseline/*`, `results/correctness/backward/backward_64x64.csv`, "
         "NVIDIA RTX PRO 6000, cuTile).  This build: the CSVs beside this file, written by the `-m gpu` "
         "suites (`tests/test_fwd_gpu.py`, `tests/test_gqa_gpu.py`, `tests/test_bwd_gpu.py`) with the "
         "reference's metrics (`tests/fused/run_correctness.py:33-36,70-80`: max-abs, relative error "
         "floored at 1e-3, tol_ratio = max |o-r| / (2e-2 + 2e-2 |r|); backward: ||x-r|| / ||r||).  "
         "Cases whose N is not a multiple of a tile, which the reference skips, run here with a partial "
         "last tile." + (f"  This build's CSVs were written by the GPU run of commit {a.commit}." if a.commit else ""),
         ""]
    L += suite_section("MHA forward suite (84 cases, fp16)", os.path.join(a.ours, "fused", "hip", "*", "*.csv"),
                       os.path.join(a.reference, "fused", "v3_occupancy2", "*", "*.csv"))
    L += suite_section("GQA forward suite (96 cases, fp16)", os.path.join(a.ours, "fused_gqa", "hip", "*", "*.csv"),
                       os.path.join(a.reference, "fused_gqa", "v0_baseline", "*", "*.csv"))
    L += backward_section(os.path.join(a.ours, "backward", "*.csv"),
                          os.path.join(a.reference, "backward", "backward_64x64.csv"))
    L += margins_section(os.path.join(a.ours, "margins", "full_size_margins.csv"))
    text = "\n".join(L) + "\n"
    if a.out:
        with open(a.out, "w") as f:
            f.write(text)
    print(text)


if __name__ == "__main__":
    main()
