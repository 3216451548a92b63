"""CLI plumbing on the CPU (the fp32 reference path of run_attention.py, and exit codes).

The CPU plumbing workload: causal MHA forward B=1, H=4, S=256, D=64 with Q, K, V ~ N(0,1)
float32 from default_rng(0) drawn in the order Q, K, V; O written to .npy through the
reference backend and checked against the float64 oracle and the committed fixture.
"""

import hashlib
import os
import subprocess
import sys

import numpy as np
import pytest

import run_attention
import run_attention_gqa
from oracle import attention_oracle as orc
from oracle import cases

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "fused-attention_amd")
GOLDEN = os.path.join(REPO, "tests", "golden", "cpu_plumbing_B1_H4_S256_D64.npz")


def plumbing_inputs():
    return cases.normal_inputs([(1, 4, 256, 64)] * 3, seed=0)


def test_cpu_plumbing_reference_backend(tmp_path):
    q, k, v = plumbing_inputs()
    inp, out = tmp_path / "qkv.npz", tmp_path / "o.npy"
    np.savez(inp, Q=q, K=k, V=v)
    rc = run_attention.main(["--input", str(inp), "--output", str(out), "--backend", "reference",
                             "--output-dtype", "float32"])
    assert rc == 0
    o = np.load(out)
    assert o.shape == (1, 4, 256, 64) and o.dtype == np.float32
    want = orc.forward(q, k, v)
    np.testing.assert_allclose(o, want, rtol=0, atol=1e-5)
    gold = np.load(GOLDEN)
    digest = hashlib.sha256(q.tobytes() + k.tobytes() + v.tobytes()).digest()
    assert bytes(gold["QKV_SHA256"]) == digest, "input generator drifted from the fixture"
    np.testing.assert_allclose(o, gold["O"], rtol=0, atol=1e-5)
    # default output dtype is float16, as the reference CLI writes
    rc = run_attention.main(["--input", str(inp), "--output", str(out), "--backend", "reference"])
    assert rc == 0 and np.load(out).dtype == np.float16
    np.testing.assert_allclose(np.load(out).astype(np.float64), want, atol=2e-3)


def test_cli_as_a_subprocess(tmp_path):
    q, k, v = (x.astype(np.float16) for x in plumbing_inputs())
    inp, out = tmp_path / "qkv.npz", tmp_path / "o.npy"
    np.savez(inp, Q=q, K=k, V=v)
    r = subprocess.run([sys.executable, os.path.join(PKG, "run_attention.py"), "--input", str(inp),
                        "--output", str(out), "--backend", "reference", "--verbose"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert "wrote" in r.stderr and np.load(out).shape == (1, 4, 256, 64)


def test_exit_codes(tmp_path, capsys):
    q, k, v = plumbing_inputs()
    out = tmp_path / "o.npy"
    missing = tmp_path / "missing.npz"
    assert run_attention.main(["--input", str(missing), "--output", str(out), "--backend", "reference"]) == 2
    assert "input file not found" in capsys.readouterr().err
    bad = tmp_path / "bad.npz"
    np.savez(bad, Q=q, K=k)
    assert run_attention.main(["--input", str(bad), "--output", str(out), "--backend", "reference"]) == 2
    assert "missing array(s) V" in capsys.readouterr().err
    garbled = tmp_path / "garbled.npz"
    garbled.write_bytes(b"not a zip file")
    assert run_attention.main(["--input", str(garbled), "--output", str(out), "--backend", "reference"]) == 2
    # fp32 inputs are rejected by the GPU backends unless a compute dtype is given
    inp = tmp_path / "qkv.npz"
    np.savez(inp, Q=q, K=k, V=v)
    assert run_attention.main(["--input", str(inp), "--output", str(out), "--backend", "hip"]) == 2
    assert "supported: float16" in capsys.readouterr().err
    # a tile outside the kernels' set {64, 128}
    assert run_attention.main(["--input", str(inp), "--output", str(out), "--backend", "reference",
                               "--block-m", "96"]) == 2
    # NaN in the input gives a non-finite output -> runtime failure (1)
    qn = q.copy()
    qn[0, 0, 5, 0] = np.nan
    np.savez(inp, Q=qn, K=k, V=v)
    assert run_attention.main(["--input", str(inp), "--output", str(out), "--backend", "reference"]) == 1
    assert "NaN or Inf" in capsys.readouterr().err
    with pytest.raises(SystemExit):
        run_attention.main(["--input", str(inp), "--output", str(out), "--backend", "nope"])


def test_gpu_backend_without_gpu_is_a_runtime_error(tmp_path, capsys):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    q, k, v = (x.astype(np.float16) for x in plumbing_inputs())
    inp, out = tmp_path / "qkv.npz", tmp_path / "o.npy"
    np.savez(inp, Q=q, K=k, V=v)
    assert run_attention.main(["--input", str(inp), "--output", str(out), "--backend", "cutile"]) == 1
    assert "no GPU" in capsys.readouterr().err


def test_gqa_cli_reference_backend(tmp_path):
    q, k, v = cases.normal_inputs([(1, 8, 128, 32), (1, 2, 128, 32), (1, 2, 128, 32)], seed=1)
    inp, out = tmp_path / "qkv.npz", tmp_path / "o.npy"
    np.savez(inp, Q=q, K=k, V=v)
    assert run_attention_gqa.main(["--input", str(inp), "--output", str(out), "--backend", "reference",
                                   "--output-dtype", "float32"]) == 0
    np.testing.assert_allclose(np.load(out), orc.forward(q, k, v), atol=1e-5)
    np.savez(inp, Q=q, K=k[:, :1], V=v)
    assert run_attention_gqa.main(["--input", str(inp), "--output", str(out), "--backend", "reference"]) == 2
