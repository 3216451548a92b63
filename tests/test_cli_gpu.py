"""The user-facing paths on the GPU: both CLIs' GPU backends, the unfused baseline and the
run tracker, each end to end on the device and checked against the float64 oracle.

The reference's CLI path is .npz -> validate -> backend fn(q, k, v, block_m, block_n) on the
device -> fp16 .npy with exit codes 0 / 1 / 2 (run_attention.py:62-130,
run_attention_gqa.py:64-132); its unfused baseline is attention/fused/unfused.py:92-116 and
attention/gqa/unfused_gqa.py; its run tracker gates a run on correctness before timing it
(profiling/track_run.py:155-183).
"""

import csv
import os

import numpy as np
import pytest
import torch

import run_attention
import run_attention_gqa
from gpu_util import log
from oracle import attention_oracle as orc
from oracle import cases

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
GPU_BACKENDS = ("hip", "cutile", "unfused")


def plumbing_inputs():
    """The CPU plumbing workload's inputs: B=1 H=4 S=256 D=64, N(0,1) fp32 from default_rng(0)."""
    return cases.normal_inputs([(1, 4, 256, 64)] * 3, seed=0)


def run_cli(main, tmp_path, q, k, v, *extra):
    inp, out = tmp_path / "qkv.npz", tmp_path / "o.npy"
    np.savez(inp, Q=q, K=k, V=v)
    rc = main(["--input", str(inp), "--output", str(out), *extra])
    return rc, (np.load(out) if rc == 0 else None)


def oracle_error(o, q, k, v):
    """Max-abs error of the CLI's output against the float64 oracle on the values the
    backend actually received (inputs rounded to the compute dtype)."""
    assert np.isfinite(o).all()
    return float(np.abs(o.astype(np.float64) - orc.forward(q, k, v)).max())


@pytest.mark.parametrize("backend", GPU_BACKENDS)
@pytest.mark.parametrize("tiles", [(64, 64), (128, 64)])
def test_mha_cli_gpu_backends_fp16(tmp_path, backend, tiles):
    q, k, v = (x.astype(np.float16) for x in plumbing_inputs())
    rc, o = run_cli(run_attention.main, tmp_path, q, k, v, "--backend", backend,
                    "--block-m", str(tiles[0]), "--block-n", str(tiles[1]))
    assert rc == 0
    assert o.dtype == np.float16 and o.shape == q.shape  # the reference CLI writes fp16
    err = oracle_error(o, q, k, v)
    log(f"run_attention --backend {backend} tiles={tiles} fp16: max_abs={err:.3e}")
    assert err <= MAX_ABS


@pytest.mark.parametrize("backend", GPU_BACKENDS)
@pytest.mark.parametrize("compute", ["bfloat16", "float16"])
def test_mha_cli_cpu_plumbing_workload_on_gpu(tmp_path, backend, compute):
    """The CPU plumbing workload's fp32 inputs through a GPU backend with --compute-dtype."""
    q, k, v = plumbing_inputs()
    rc, o = run_cli(run_attention.main, tmp_path, q, k, v, "--backend", backend, "--compute-dtype", compute,
                    "--output-dtype", "float32")
    assert rc == 0 and o.dtype == np.float32
    tdt = torch.bfloat16 if compute == "bfloat16" else torch.float16
    qr, kr, vr = (torch.from_numpy(x).to(tdt).double().numpy() for x in (q, k, v))
    err = oracle_error(o, qr, kr, vr)
    log(f"run_attention --backend {backend} --compute-dtype {compute}: max_abs={err:.3e}")
    assert err <= MAX_ABS
    # and against the fp32 inputs themselves (what the user asked for): rounding of the
    # inputs to the compute dtype adds at most a few 1e-3 here
    assert oracle_error(o, q, k, v) <= MAX_ABS


@pytest.mark.parametrize("backend", GPU_BACKENDS)
@pytest.mark.parametrize("hkv", [1, 2, 8])
def test_gqa_cli_gpu_backends(tmp_path, backend, hkv):
    q, k, v = (x.astype(np.float16) for x in cases.normal_inputs(
        [(2, 8, 200, 64), (2, hkv, 200, 64), (2, hkv, 200, 64)], seed=3))
    rc, o = run_cli(run_attention_gqa.main, tmp_path, q, k, v, "--backend", backend)
    assert rc == 0 and o.dtype == np.float16 and o.shape == q.shape
    err = oracle_error(o, q, k, v)
    log(f"run_attention_gqa --backend {backend} H_kv={hkv}: max_abs={err:.3e}")
    assert err <= MAX_ABS


def test_gqa_cli_bf16_compute(tmp_path):
    q, k, v = cases.normal_inputs([(1, 8, 128, 128), (1, 2, 128, 128), (1, 2, 128, 128)], seed=4)
    rc, o = run_cli(run_attention_gqa.main, tmp_path, q, k, v, "--backend", "hip", "--compute-dtype", "bfloat16")
    assert rc == 0
    qr, kr, vr = (torch.from_numpy(x).bfloat16().double().numpy() for x in (q, k, v))
    assert oracle_error(o, qr, kr, vr) <= MAX_ABS


def test_cli_exit_codes_on_gpu(tmp_path, capsys):
    q, k, v = (x.astype(np.float16) for x in plumbing_inputs())
    # 2: fp32 input to a GPU backend without --compute-dtype
    rc, _ = run_cli(run_attention.main, tmp_path, *(x.astype(np.float32) for x in (q, k, v)), "--backend", "hip")
    assert rc == 2 and "supported: float16" in capsys.readouterr().err
    # 2: a tile outside {64, 128}
    rc, _ = run_cli(run_attention.main, tmp_path, q, k, v, "--backend", "hip", "--block-n", "32")
    assert rc == 2
    # 2: K/V head count that does not divide H (GQA CLI)
    rc, _ = run_cli(run_attention_gqa.main, tmp_path, q, k[:, :3], v[:, :3], "--backend", "hip")
    assert rc == 2
    # 1: a NaN input makes the device output non-finite, reported as a runtime failure
    qn = q.copy()
    qn[0, 1, 7, 3] = np.nan
    for backend in GPU_BACKENDS:
        rc, _ = run_cli(run_attention.main, tmp_path, qn, k, v, "--backend", backend)
        assert rc == 1, backend
        assert "NaN or Inf" in capsys.readouterr().err


# --------------------------------------------------------------------------- unfused baseline
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_unfused_baselines_match_oracle(dtype):
    from attention.fused.unfused import unfused_attention
    from attention.gqa.unfused_gqa import unfused_gqa_attention

    q, k, v = cases.normal_inputs([(2, 4, 192, 64)] * 3, seed=5)
    qd, kd, vd = (torch.from_numpy(x).cuda().to(dtype) for x in (q, k, v))
    o, S, P = unfused_attention(qd, kd, vd, 64, 64, return_intermediates=True)
    torch.cuda.synchronize()
    qr, kr, vr = (t.double().cpu().numpy() for t in (qd, kd, vd))
    assert o.dtype == dtype and P.dtype == dtype and S.dtype == torch.float32
    err = float(np.abs(o.double().cpu().numpy() - orc.forward(qr, kr, vr)).max())
    perr = float(np.abs(P.double().cpu().numpy() - orc.probs(qr, kr)).max())
    log(f"unfused {dtype}: O max_abs={err:.3e} P max_abs={perr:.3e}")
    assert err <= MAX_ABS and perr <= MAX_ABS
    # GQA: H = 8 query heads over H_kv = 2
    q, k, v = cases.normal_inputs([(1, 8, 160, 32), (1, 2, 160, 32), (1, 2, 160, 32)], seed=6)
    qd, kd, vd = (torch.from_numpy(x).cuda().to(dtype) for x in (q, k, v))
    o = unfused_gqa_attention(qd, kd, vd, 64, 64)
    torch.cuda.synchronize()
    qr, kr, vr = (t.double().cpu().numpy() for t in (qd, kd, vd))
    err = float(np.abs(o.double().cpu().numpy() - orc.forward(qr, kr, vr)).max())
    log(f"unfused_gqa {dtype}: O max_abs={err:.3e}")
    assert err <= MAX_ABS


# --------------------------------------------------------------------------- run tracker
def test_tracker_end_to_end_records_a_gated_run(tmp_path, capsys):
    from profiling import track_run as tr

    rec_dir = tmp_path / "records"
    argv = ["--records-dir", str(rec_dir), "--out-dir", str(tmp_path / "runs"), "--note", "gpu test",
            "--B", "1", "--H", "2", "--Ds", "64", "--Ns", "256", "--tiles", "64x64", "--dtype", "bf16",
            "--settle-s", "0.2", "--with-unfused"]
    assert tr.main(argv) == 0
    out = capsys.readouterr().out
    # the correctness gate ran on the device and passed for every checked shape
    checks = [ln for ln in out.splitlines() if ln.startswith("[check]")]
    assert checks and all(ln.split(": ", 1)[1].startswith("ok") for ln in checks), checks
    with open(rec_dir / "runs.csv") as f:
        rows = list(csv.DictReader(f))
    impls = {r["impl"] for r in rows}
    assert {"fused", "sdpa", "unfused"} <= impls and all(r["run"] == "1" for r in rows)
    fused = next(r for r in rows if r["impl"] == "fused")
    assert float(fused["median_ms"]) > 0 and fused["dtype"] == "bf16" and fused["tile_m"] == "64"
    md = (rec_dir / "RUNS.md").read_text()
    assert "## Run 1" in md and "gpu test" in md and "First run on this GPU" in md
    assert os.path.exists(tmp_path / "runs" / "run_001" / "summary.md")
    # a second run compares against the first and records the (empty) code diff
    assert tr.main(argv[:-1] + ["--note", "second"]) == 0
    md = (rec_dir / "RUNS.md").read_text()
    assert "## Run 2" in md and "vs previous run (Run 1)" in md and "(no code changes)" in md


def test_tracker_gate_rejects_a_wrong_kernel(tmp_path):
    """A kernel file whose output is off fails the gate and no run is recorded."""
    from profiling import track_run as tr

    bad = tmp_path / "bad_kernel.py"
    bad.write_text("import torch\n"
                   "from attention.fused.fused import fused_attention as _f\n"
                   "def fused_attention(q, k, v, tile_m=64, tile_n=64):\n"
                   "    return _f(q, k, v, tile_m, tile_n) * 1.1\n")
    rec_dir = tmp_path / "records"
    with pytest.raises(SystemExit) as e:
        tr.main(["--kernel", str(bad), "--records-dir", str(rec_dir), "--B", "1", "--H", "2",
                 "--Ds", "64", "--Ns", "256", "--tiles", "64x64"])
    assert "correctness check FAILED" in str(e.value)
    assert not (rec_dir / "runs.csv").exists()
