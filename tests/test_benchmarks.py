"""The benchmark scripts (the reference's benchmarks/ CLIs): host-side pieces on the CPU, one tiny
end-to-end run of each on the GPU."""

import csv
import math
import os
import sys

import pytest

PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fused-attention_amd")
sys.path.insert(0, PKG)

from benchmarks import _timing as T  # noqa: E402
from benchmarks import benchmark_backward, benchmark_forward, benchmark_forward_gqa  # noqa: E402


def test_flop_and_byte_counts():
    # the reference's count: 4*B*H*N*N*D/2 (benchmarks/benchmark_forward.py:206 there)
    assert T.causal_flops(4, 32, 4096, 128) == 4 * 4 * 32 * 4096 * 4096 * 128 / 2 == 5.4975581388800e11
    # GQA: Q, O of 32 heads and K, V of 8 heads, bf16
    assert T.forward_bytes(2, 32, 8, 8192, 128) == 335_544_320


def test_speedups_and_summary():
    rows = [dict(D=64, N=128, impl="fused", ms=1.0), dict(D=64, N=128, impl="unfused", ms=4.0),
            dict(D=64, N=128, impl="sdpa", ms=2.0), dict(D=64, N=512, impl="fused", ms=2.0),
            dict(D=64, N=512, impl="sdpa", ms=None)]
    sp = T.speedups(rows, key_of=lambda r: (r["D"], r["N"]), impl_of=lambda r: r["impl"], ms_of=lambda r: r["ms"])
    assert sp[0] == ["4.000", "2.000"] and sp[1] == ["", ""] and sp[3] == ["", ""]
    ok = [(64, 128, "fused", 1.0, 10.0), (64, 128, "unfused", 4.0, 2.5), (64, 512, "fused", 2.0, 20.0),
          (64, 512, "unfused", 2.0, 20.0)]
    header, out = T.summary_rows(ok, ["fused", "unfused"])
    assert header[:4] == ["scope", "value", "fused_avg_median_ms", "fused_avg_tflops"]
    overall = out[-1]
    assert overall[:2] == ["all", "all"]
    # geometric mean of 4.0 and 1.0
    assert overall[header.index("fused_speedup_vs_unfused")] == f"{math.sqrt(4.0):.2f}"
    assert overall[header.index("fused_speedup_vs_sdpa")] == ""


def test_csv_and_plot(tmp_path):
    path = tmp_path / "x" / "a.csv"
    T.write_csv(str(path), ["a", "b"], [[1, 2]])
    assert list(csv.reader(open(path))) == [["a", "b"], ["1", "2"]]
    ok = [(64, 128, "fused", 1.0, 10.0), (64, 128, "sdpa", 2.0, 5.0), (64, 512, "fused", 2.0, 20.0)]
    T.plot_panels(ok, str(tmp_path / "p.png"))


def test_load_function_by_path():
    fn = T.load_function(os.path.join(PKG, "attention", "fused", "fused.py"), "fused_attention")
    assert callable(fn) and fn.__name__ == "fused_attention"
    with pytest.raises(FileNotFoundError):
        T.load_function(os.path.join(PKG, "no_such_kernel.py"), "fused_attention")


def test_gqa_benchmark_rejects_bad_group():
    with pytest.raises(SystemExit):
        benchmark_forward_gqa.main(["--H", "8", "--H-kv", "3"])
    with pytest.raises(SystemExit):
        benchmark_backward.main(["--H", "8", "--H-kv", "3"])


def test_naive_backward_baseline_matches_oracle():
    """The eager baseline of the backward benchmark is the causal formula (MHA and GQA)."""
    import numpy as np
    import torch
    from oracle import attention_oracle as orc
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 4, 40, 16), dtype=np.float32)
    kv = [rng.standard_normal((1, 2, 40, 16), dtype=np.float32) for _ in range(2)]
    got = benchmark_backward.naive_attention(torch.from_numpy(q), *map(torch.from_numpy, kv))
    np.testing.assert_allclose(got.numpy(), orc.forward(q, *kv), atol=2e-5)


@pytest.mark.gpu
def test_benchmarks_run_end_to_end(tmp_path):
    d = str(tmp_path)
    assert benchmark_forward.main(["--Ds", "64", "--Ns", "200", "--B", "1", "--H", "2", "--tile-m", "128",
                                   "--out", f"{d}/f.csv", "--summary-out", f"{d}/fs.csv",
                                   "--plot-out", f"{d}/f.png"]) == 0
    rows = list(csv.DictReader(open(f"{d}/f.csv")))
    assert [r["impl"] for r in rows] == ["fused", "unfused", "sdpa"] and all(r["median_ms"] for r in rows)
    assert benchmark_forward_gqa.main(["--Ds", "64", "--Ns", "256", "--B", "1", "--H", "4", "--H-kv", "1",
                                       "--impls", "fused,unfused", "--out", f"{d}/g.csv",
                                       "--summary-out", f"{d}/gs.csv", "--plot-out", f"{d}/g.png"]) == 0
    assert [r["H_kv"] for r in csv.DictReader(open(f"{d}/g.csv"))] == ["1", "1"]
    assert benchmark_backward.main(["--Ds", "64", "--Ns", "256", "--B", "1", "--H", "2", "--impls", "fused,naive",
                                    "--warmup", "1", "--reps", "3", "--out-dir", d]) == 0
    rows = list(csv.DictReader(open(f"{d}/bench_backward_64x64.csv")))
    assert [r["status"] for r in rows] == ["ok", "ok"]
