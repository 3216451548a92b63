"""Helpers for the GPU parity tests: device inputs, the two checks, reporting.

Every fused output is checked twice:
  * against the float64 oracle on sampled (batch, head) slices and sampled query rows
    (rows are independent, so the oracle can evaluate any subset exactly);
  * element by element against the reference's fp32 PyTorch formula on the GPU,
    head-chunked under 2 GiB as the reference harness does, with the reference's
    mixed tolerance |out - ref| <= 2e-2 + 2e-2 |ref| and max-abs <= 2e-2.
"""

import sys

import numpy as np
import torch

from oracle import attention_oracle as orc
from oracle import cpu_reference

ATOL = 2e-2
RTOL = 2e-2
MAX_ABS = 2e-2
REL_FLOOR = 1e-3  # relative error divides by max(|ref|, 1e-3) (tests/fused/run_correctness.py:35)

# Per-case records of the reference's correctness suites, in the reference's CSV layout
# (tests/fused/run_correctness.py:187-197, tests/gqa/run_correctness_gqa.py,
# tests/backward/run_correctness_backward.py:110-113): {(file path, columns): [rows]},
# written by conftest.py at the end of the session.
RECORDS = {}

FUSED_COLS = ["case", "B", "H", "N", "D", "magnitude", "seed", "max_abs_err", "max_rel_err", "tol_ratio",
              "time_s", "result", "note"]
GQA_COLS = ["case", "B", "H", "H_kv", "group", "N", "D", "magnitude", "seed", "max_abs_err", "max_rel_err",
            "tol_ratio", "time_s", "result", "note"]
BWD_COLS = ["test", "B", "H", "N", "D", "sigma", "relerr_O", "relerr_dQ", "relerr_dK", "relerr_dV", "result",
            "fused_ms", "sdpa_ms", "fused_speedup_vs_sdpa"]


MARGIN_COLS = ["test", "B", "H", "H_kv", "N", "D", "dtype", "tiles", "output", "max_abs_err", "bar",
               "max_abs_over_bar", "mixed_tol_ratio", "rel_frobenius", "oracle_max_abs"]


def margin(test, q, k, tiles, output, max_abs, bar, mixed=None, rel=None, oracle=None):
    """One row of the full-size workloads' error margins (margins/full_size_margins.csv): the
    output's max-abs error against the fp32 reference, the bar it is held to, and the other
    measures its test applies (mixed 2e-2 + 2e-2|ref| ratio, relative Frobenius, oracle)."""
    B, H, N, D = q.shape
    fmt = lambda x: "" if x is None else f"{x:.4e}"
    record("margins/full_size_margins.csv", MARGIN_COLS,
           dict(test=test, B=B, H=H, H_kv=k.shape[1], N=N, D=D, dtype=str(q.dtype).replace("torch.", ""),
                tiles=f"{tiles[0]}x{tiles[1]}", output=output, max_abs_err=fmt(max_abs), bar=f"{bar:g}",
                max_abs_over_bar=f"{max_abs / bar:.3f}", mixed_tol_ratio=fmt(mixed), rel_frobenius=fmt(rel),
                oracle_max_abs=fmt(oracle)))


def record(path, columns, row):
    RECORDS.setdefault((path, tuple(columns)), []).append([row.get(c, "") for c in columns])


def write_records(root):
    import csv
    import os
    written = []
    for (path, columns), rows in RECORDS.items():
        full = os.path.join(root, path)
        os.makedirs(os.path.dirname(full), exist_ok=True)
        with open(full, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(columns)
            w.writerows(rows)
        written.append(full)
    return written


def compare_ref(out, ref):
    """(max_abs, max_rel, tol_ratio, nonfinite) of out vs ref, as the reference's compare()
    (tests/fused/run_correctness.py:70-80): a case passes iff tol_ratio <= 1."""
    out = out.float()
    nonfinite = int((~torch.isfinite(out)).sum())
    if nonfinite:
        return float("inf"), float("inf"), float("inf"), nonfinite
    err = (out - ref).abs()
    return (float(err.max()), float((err / ref.abs().clamp_min(REL_FLOOR)).max()),
            float((err / (ATOL + RTOL * ref.abs())).max()), 0)


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype).contiguous()


def compare_full(out, ref):
    """(max_abs, tol_ratio) of out vs ref; both must pass."""
    out = out.float()
    assert torch.isfinite(out).all(), "non-finite values in the fused output"
    err = (out - ref).abs()
    return float(err.max()), float((err / (ATOL + RTOL * ref.abs())).max())


def head_samples(B, H):
    picks = {(0, 0), (B - 1, H - 1), (B // 2, H // 2)}
    return sorted(picks)


def check_forward(out, q, k, v, rows_count=40, label="", case=None, tiles=None, seconds=None, margin_test=None):
    """Assert out (GPU) matches the oracle on sampled rows and the fp32 reference everywhere.
    With `case` (one of the reference's suite cases) the comparison is also recorded; with
    `margin_test` (a full-size workload) its margin is."""
    B, H, N, D = q.shape
    g = H // k.shape[1]
    ref = cpu_reference.reference_chunked(q, k, v)
    if case is not None:
        a, rel, rat, nonfinite = compare_ref(out, ref)
        tile = f"{tiles[0]}x{tiles[1]}"
        row = dict(case=case.id, B=B, H=H, N=N, D=D, magnitude=case.magnitude, seed=case.seed,
                   max_abs_err=a, max_rel_err=rel, tol_ratio=rat, time_s=seconds,
                   result="PASS" if (nonfinite == 0 and rat <= 1.0) else "FAIL",
                   note=f"{nonfinite} NaN/Inf values" if nonfinite else "")
        if k.shape[1] == H and not hasattr(case, "H_kv"):
            record(f"fused/hip/{tile}/correctness_fused_hip_{tile}.csv", FUSED_COLS, row)
        else:
            record(f"fused_gqa/hip/{tile}/correctness_fused_gqa_hip_{tile}.csv", GQA_COLS,
                   dict(row, H_kv=k.shape[1], group=g))
    max_abs, ratio = compare_full(out, ref)
    del ref
    rows = orc.sample_rows(N, count=rows_count)
    worst = 0.0
    for b, h in head_samples(B, H):
        hk = h // g
        qs = q[b:b + 1, h:h + 1].double().cpu().numpy()
        ks = k[b:b + 1, hk:hk + 1].double().cpu().numpy()
        vs = v[b:b + 1, hk:hk + 1].double().cpu().numpy()
        want = orc.forward(qs, ks, vs, rows)
        got = out[b:b + 1, h:h + 1, rows].double().cpu().numpy()
        worst = max(worst, float(np.abs(got - want).max()))
    log(f"{label} max_abs={max_abs:.3e} tol_ratio={ratio:.3f} oracle_rows_max_abs={worst:.3e}")
    if margin_test is not None:
        margin(margin_test, q, k, tiles, "O", max_abs, MAX_ABS, mixed=ratio, oracle=worst)
    assert max_abs <= MAX_ABS and ratio <= 1.0, (label, max_abs, ratio)
    assert worst <= MAX_ABS, (label, worst)
    return max_abs, ratio, worst
