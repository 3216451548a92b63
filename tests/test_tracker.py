"""Host logic of profiling/track_run.py (the rocprofv3 run tracker), without a GPU."""

import csv
import os

import pytest

from profiling import track_run as tr


def rows_for(ms_fused, ms_sdpa=None, dtype="bf16"):
    rows = [dict(D=128, N=4096, B=4, H=32, impl="fused", tile_m=128, tile_n=64, median_ms=f"{ms_fused:.4f}",
                 tflops="100.000", dtype=dtype, pct_peak="3.97")]
    if ms_sdpa is not None:
        rows.append(dict(D=128, N=4096, B=4, H=32, impl="sdpa", tile_m="-", tile_n="-", median_ms=f"{ms_sdpa:.4f}",
                         tflops="50.000", dtype=dtype, pct_peak="1.99"))
    return rows


def test_records_append_number_and_compare(tmp_path):
    rec = tr.Records(str(tmp_path))
    assert rec.history() == [] and rec.next_run([]) == 1
    env = {"gpu": "AMD Instinct MI355X", "commit": "abc", "kernel": tr.DEFAULT_KERNEL}
    md1 = tr.build_markdown(1, "2026-12-01 10:00", env, "first", rows_for(1.0, 2.0), [])
    assert "First run on this GPU" in md1 and "2.00x faster" in md1
    rec.append(1, "2026-12-01 10:00", env, "first", rows_for(1.0, 2.0), md1, rec.run_dir(1))
    hist = rec.history()
    assert rec.next_run(hist) == 2 and len(hist) == 2 and set(tr.CSV_FIELDS) == set(hist[0])
    md2 = tr.build_markdown(2, "2026-12-01 11:00", env, "faster", rows_for(0.8), hist)
    # 1.0 ms -> 0.8 ms is 20% faster than both the previous and the first run
    assert md2.count("20.0% faster") == 2 and "(Run 1)" in md2
    rec.append(2, "2026-12-01 11:00", env, "faster", rows_for(0.8), md2, rec.run_dir(2), {"change.diff": "x\n"})
    assert os.path.exists(os.path.join(rec.run_dir(2), "change.diff"))
    assert open(rec.md).read().count("## Run") == 2
    # another GPU does not compare against these runs
    md3 = tr.build_markdown(3, "t", {"gpu": "other"}, "", rows_for(0.5), rec.history())
    assert "First run on this GPU" in md3


def test_dtype_is_part_of_the_comparison_key(tmp_path):
    env = {"gpu": "G"}
    hist = [dict(run="1", timestamp="t", gpu="G", commit="", kernel="", note="", **r) for r in rows_for(1.0, dtype="fp16")]
    md = tr.build_markdown(2, "t", env, "", rows_for(0.5, dtype="bf16"), hist)
    row = [ln for ln in md.splitlines() if ln.startswith("| 128 | 4096 |")]
    assert len(row) == 1 and row[0].endswith("| - | - |")  # no bf16 row in run 1 to compare with
    md_same = tr.build_markdown(2, "t", env, "", rows_for(0.5, dtype="fp16"), hist)
    assert "50.0% faster" in md_same


def test_import_rows(tmp_path):
    p = tmp_path / "bench.csv"
    with open(p, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["D", "N", "B", "H", "impl", "tile_m", "tile_n", "median_ms", "tflops"])
        w.writeheader()
        w.writerow(dict(D=64, N=512, B=2, H=8, impl="fused", tile_m=64, tile_n=64, median_ms="0.02", tflops="27"))
        w.writerow(dict(D=64, N=512, B=2, H=8, impl="sdpa", tile_m=64, tile_n=64, median_ms="0.03", tflops="20"))
        w.writerow(dict(D=64, N=512, B=2, H=8, impl="fused", tile_m=64, tile_n=64, median_ms="", tflops=""))
    rows = tr.import_rows(str(p))
    assert len(rows) == 2 and rows[1]["tile_m"] == "-" and rows[0]["N"] == 512


def test_counter_parsing_and_percentages(tmp_path):
    p = tmp_path / "c.csv"
    with open(p, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for d, kern in ((1, "void fa::fwd_kernel<...>"), (2, "void other"), (3, "void fa::fwd_kernel<...>")):
            for _ in range(2):  # counters arrive split across dimensions: summed per dispatch
                w.writerow(dict(Dispatch_Id=d, Kernel_Name=kern, Counter_Name="SQ_INSTS_MFMA", Counter_Value=50 * d))
                w.writerow(dict(Dispatch_Id=d, Kernel_Name=kern, Counter_Name="GRBM_GUI_ACTIVE", Counter_Value=4000))
    name, vals = tr.last_dispatch_counters(str(p), "fwd_kernel")
    assert "fwd_kernel" in name and vals == {"SQ_INSTS_MFMA": 300.0, "GRBM_GUI_ACTIVE": 8000.0}
    assert tr.last_dispatch_counters(str(p), "nomatch") == (None, {})
    # 1000 cycles per XCD; MFMA busy = busy / (cycles x 1024 SIMDs)
    out = tr.summarize_counters({"GRBM_GUI_ACTIVE": 8000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 512000.0,
                                 "SQ_INSTS_MFMA": 100.0, "SQ_INSTS_VALU": 500.0, "SQ_INSTS_VALU_TRANS_F32": 100.0,
                                 "SQ_LDS_IDX_ACTIVE": 64000.0, "SQ_INSTS_LDS_LOAD_BANDWIDTH": 1600.0,
                                 "SQ_WAIT_ANY": 25.0, "SQ_WAVE_CYCLES": 100.0})
    assert out["MFMA busy %"] == pytest.approx(50.0)
    assert out["VALU instr / MFMA"] == pytest.approx(4.0)
    assert out["exp-class instr / MFMA"] == pytest.approx(1.0)
    assert out["LDS active %"] == pytest.approx(25.0)
    assert out["LDS bytes read / MFMA"] == pytest.approx(1024.0)
    assert out["wave-wait %"] == pytest.approx(25.0)


def test_counter_passes_fit_one_rocprof_pass():
    for names in tr.COUNTER_PASSES:
        assert sum(n.startswith("SQ_") for n in names) <= 8
        assert sum(n.startswith("GRBM_") for n in names) <= 2
        assert not any(n.startswith(("TCC_", "TCP_", "TA_", "TD_")) for n in names)


def test_cli_parsing_keeps_reference_flags():
    a = tr.parse_args(["--ncu", "--ncu-size", "128,4096", "--ncu-tile", "128x64", "--tiles", "64x64,128x64"])
    assert a.profile and a.profile_size == "128,4096" and a.profile_tile == "128x64"
    assert tr.parse_tiles(a.tiles) == [(64, 64), (128, 64)] and tr.parse_list("64,128") == [64, 128]
    assert tr.change(0.8, 1.0) == "20.0% faster" and tr.change(1.25, 1.0) == "25.0% slower" and tr.change(1, None) == "-"


def test_code_diff_uses_the_previous_runs_source_snapshot(tmp_path, monkeypatch):
    """Where git is absent (the GPU machine) the diff comes from run_NNN/src/ of the previous
    run; without a snapshot or a usable commit no diff is claimed."""
    pkg = tmp_path / "pkg"
    (pkg / "csrc").mkdir(parents=True)
    (pkg / "csrc" / "k.hip").write_text("a\nb\nc\n")
    monkeypatch.setattr(tr, "PKG_ROOT", str(pkg))
    rec_dir = tmp_path / "records"
    history = [{"run": "1", "gpu": "G", "commit": "unknown"}]
    assert tr.code_diff(history, "G", 2, ["csrc/k.hip"], str(rec_dir)) is None
    snap = rec_dir / "runs" / "run_001" / "src" / "csrc"
    snap.mkdir(parents=True)
    (snap / "k.hip").write_text("a\nb\nc\n")
    assert tr.code_diff(history, "G", 2, ["csrc/k.hip"], str(rec_dir)) == (1, "(no code changes)")
    (pkg / "csrc" / "k.hip").write_text("a\nB\nc\n")
    prev, d = tr.code_diff(history, "G", 2, ["csrc/k.hip"], str(rec_dir))
    assert prev == 1 and "-b" in d and "+B" in d and "Run 1: csrc/k.hip" in d
    assert tr.snap_name("/elsewhere/x.py") == "x.py"


def test_records_create_their_folder(tmp_path):
    """A records folder that does not exist yet (runs kept elsewhere) is created on the first run."""
    rec = tr.Records(str(tmp_path / "new" / "records"))
    env = {"gpu": "g", "commit": "c", "kernel": tr.DEFAULT_KERNEL}
    md = tr.build_markdown(1, "t", env, "n", rows_for(1.0), [])
    rec.append(1, "t", env, "n", rows_for(1.0), md, str(tmp_path / "elsewhere" / "run_001"))
    assert len(rec.history()) == 1 and os.path.exists(rec.md)
