"""Throughput of the fused causal attention path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--device-warmup-s T] [--tile-m 128 --tile-n 64] [--no-cpu-baseline]

One step = one fused causal forward over the full workload B=4, H=32, S=4096,
D=128 in bfloat16 (inputs resident in HBM).  K steps are timed between two
device synchronisations, after T seconds (default 1.5) of untimed steps that let
the GPU clocks settle and W untimed warm-up steps; the forward+backward of the
same shape (through the autograd Function) is timed the same way.
FLOPs follow the reference's causal convention: 2*B*H*S^2*D for the forward,
2.5x that for the backward (benchmarks/benchmark_forward.py:206,
benchmarks/benchmark_backward.py:126-127).

Prints one JSON line.  `roofline` is the forward kernel's achieved TFLOP/s
(algorithmic FLOPs / mean kernel duration from HIP events around each launch
on the launch stream) against the dense bf16 MFMA peak; `cpu_baseline` is the
reference's fp32 PyTorch path (oracle/cpu_reference.py) timed on the host cores
on a bounded slice of the same workload, and `fwd_bwd.cpu_baseline` fp32 autograd of
the same formula (forward + backward) on a bounded slice.
"""

import argparse
import json
import os
import platform
import re
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(REPO, "fused-attention_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16/fp16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_PEAK_GBS = 8000.0
WORKLOAD = dict(B=4, H=32, S=4096, D=128)
TRAFFIC_FILE = os.path.join(REPO, "profiles", "fwd_mha_B4_H32_S4096_D128_bf16_traffic.md")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--tile-m", type=int, default=128)
    p.add_argument("--tile-n", type=int, default=64)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-bwd", action="store_true", help="skip the forward+backward timing")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline wall time")
    p.add_argument("--device-warmup-s", type=float, default=1.5,
                   help="untimed seconds of the step before the warm-up steps (GPU clock ramp)")
    p.add_argument("--traffic-run", action="store_true",
                   help="only run one 1 GiB device copy and --steps forward launches (for rocprofv3 "
                        "--pmc FETCH_SIZE / WRITE_SIZE: the copy calibrates the counters)")
    return p.parse_args()


def causal_fwd_flops(B, H, S, D):
    return 2.0 * B * H * S * S * D


def traffic_from_profile():
    """HBM bytes per forward launch, from the committed rocprofv3 PMC summary (or None)."""
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def device_warmup(fn, seconds, torch):
    """Run the step untimed until `seconds` have passed, so the GPU clocks have
    settled before the warm-up steps (a cold MI355X ramps for about a second)."""
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
    return n


def time_steps(fn, steps, warmup, torch, warm_seconds):
    """Wall time of `steps` back-to-back steps between two device synchronisations (nothing
    else on the stream in between), then the same number of steps again with an event pair
    around each on the current (launch) stream, for the mean and median step duration on
    the device.  The events go in a pass of their own: each one is a packet of its own in
    the queue, and the device time they add between kernels is not part of the work."""
    device_warmup(fn, warm_seconds, torch)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) for a, b in evs]
    return wall_ms / steps, statistics.mean(per), statistics.median(per)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_cpu(fn, make_inputs, seconds, max_heads, torch):
    """Median of 3 timed passes of fn over a head slice sized so the three take about
    `seconds` (one warm-up pass on one head sets the size).  Returns (heads, seconds per pass)."""
    fn(*make_inputs(1))  # warm-up
    t0 = time.perf_counter()
    fn(*make_inputs(1))
    one = time.perf_counter() - t0
    heads = int(max(1, min(max_heads, seconds / 3 / max(one, 1e-3))))
    inputs = make_inputs(heads)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        fn(*inputs)
        times.append(time.perf_counter() - t0)
    return heads, statistics.median(times)


def cpu_baseline(args, torch):
    """The reference's fp32 PyTorch formula on the host cores, over a bounded head slice:
    forward (oracle.cpu_reference.reference_attention_explicit, the path of
    attention/fused/reference.py:16-23) and forward+backward by fp32 autograd of the same
    formula (oracle.cpu_reference.reference_grads, as tests/backward/run_correctness_backward.py:25-44)."""
    from oracle.cpu_reference import reference_attention_explicit, reference_grads

    S, D = WORKLOAD["S"], WORKLOAD["D"]
    g = torch.Generator().manual_seed(0)

    def make(heads, n=3):
        return [torch.randn(1, heads, S, D, generator=g).bfloat16().float() for _ in range(n)]

    host = f"host {_cpu_model()}, os.cpu_count()={os.cpu_count()}"
    heads, t = _time_cpu(reference_attention_explicit, make, args.cpu_seconds, WORKLOAD["B"] * WORKLOAD["H"], torch)
    fwd = {"value": round(causal_fwd_flops(1, heads, S, D) / t / 1e12, 4), "unit": "TFLOP/s",
           "cores": torch.get_num_threads(), "kind": "port",
           "sample": f"reference fp32 explicit formula, B=1 H={heads} S={S} D={D} of the bf16 workload "
                     f"(values rounded to bf16), median of 3 after 1 warm-up; {t:.2f} s per pass; {host}"}
    if args.no_bwd:
        return fwd, None
    # autograd holds a few N x N fp32 tensors per head: at most 16 heads (about 6 GB) per pass
    heads, t = _time_cpu(lambda q, k, v, do: reference_grads(q, k, v, do), lambda h: make(h, 4),
                         args.cpu_seconds, 16, torch)
    fb = {"value": round(3.5 * causal_fwd_flops(1, heads, S, D) / t / 1e12, 4), "unit": "TFLOP/s",
          "cores": torch.get_num_threads(), "kind": "port",
          "sample": f"fp32 autograd of the reference's explicit formula (forward + backward), B=1 H={heads} "
                    f"S={S} D={D} of the bf16 workload, 3.5x causal FLOP convention, median of 3 after "
                    f"1 warm-up; {t:.2f} s per pass; {host}"}
    return fwd, fb


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the kernels run on one "
              f"MI355X and nothing here shards across GPUs", file=sys.stderr)
        sys.exit(2)
    import torch

    from attention import _lib
    from attention.backward.fused_backward import fused_attention_autograd
    from attention.fused.fused import fused_attention

    B, H, S, D = WORKLOAD["B"], WORKLOAD["H"], WORKLOAD["S"], WORKLOAD["D"]
    tm, tn = args.tile_m, args.tile_n
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v, do = (torch.randn(B, H, S, D, device="cuda", generator=g, dtype=torch.float32).bfloat16()
                   for _ in range(4))
    flops = causal_fwd_flops(B, H, S, D)

    if args.traffic_run:
        src = torch.empty(1 << 29, device="cuda", dtype=torch.int16).fill_(1)  # 1 GiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # calibration: reads 1 GiB, writes 1 GiB
        torch.cuda.synchronize()
        del src, dst
        for _ in range(args.steps):
            fused_attention(q, k, v, tm, tn)
        torch.cuda.synchronize()
        print(json.dumps({"traffic_run": True, "copy_bytes": 1 << 30, "fwd_launches": args.steps}), flush=True)
        return

    fused_attention(q, k, v, tm, tn)  # first call
    torch.cuda.synchronize()
    ms_step, kern_ms_mean, kern_ms_med = time_steps(lambda: fused_attention(q, k, v, tm, tn),
                                                   args.steps, args.warmup, torch, args.device_warmup_s)
    fwd_tflops = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (kern_ms_mean * 1e-3) / 1e12

    result = {
        "metric": "causal attn fwd & fwd+bwd TFLOP/s and % of MFMA peak, bf16 S=4096 D=128",
        "value": round(fwd_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: Q, K, V, dO ~ N(0,1) from torch.Generator(cuda).manual_seed(0), cast to bf16",
        "config": {"workload": "causal MHA forward B=4 H=32 S=4096 D=128 bf16", "B": B, "H": H, "S": S,
                   "D": D, "tile_m": tm, "tile_n": tn, "flops_per_step": flops,
                   "flop_convention": "causal 2*B*H*S^2*D (fwd), 3.5x for fwd+bwd",
                   "device_warmup_s": args.device_warmup_s},
        "pct_of_peak": round(100.0 * fwd_tflops / PEAK_BF16_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profile(),
                     "traffic_source": "profiles/" + os.path.basename(TRAFFIC_FILE) + " (rocprofv3 --pmc "
                                       "FETCH_SIZE and WRITE_SIZE runs of bench.py --traffic-run; not "
                                       "measured in this run)",
                     "kernel": "fa::fwd_kernel", "kernel_ms_mean": round(kern_ms_mean, 4),
                     "kernel_ms_median": round(kern_ms_med, 4),
                     "algorithmic_bytes": 4 * B * H * S * D * 2},
    }

    if not args.no_bwd and _lib.load().fa_supported(_lib.FA_BF16, D, tm, tn, 1, 1, 1):
        qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))

        def step():
            qg.grad = kg.grad = vg.grad = None
            fused_attention_autograd(qg, kg, vg, tm, tn).backward(do)

        step()
        torch.cuda.synchronize()
        fb_ms, _, fb_med = time_steps(step, args.steps, args.warmup, torch, args.device_warmup_s)
        fb_tflops = 3.5 * flops / (fb_ms * 1e-3) / 1e12
        result["fwd_bwd"] = {"value": round(fb_tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(fb_ms, 4),
                             "pct_of_peak": round(100.0 * fb_tflops / PEAK_BF16_TFLOPS, 2),
                             "flops_per_step": 3.5 * flops}
    else:
        result["fwd_bwd"] = None

    if not args.no_cpu_baseline:
        result["cpu_baseline"], fb_cpu = cpu_baseline(args, torch)
        if result["fwd_bwd"] is not None:
            result["fwd_bwd"]["cpu_baseline"] = fb_cpu
    else:
        result["cpu_baseline"] = None
    result["host"] = {"python": platform.python_version(), "torch": torch.__version__,
                      "hip": getattr(torch.version, "hip", None), "device": torch.cuda.get_device_name(0)}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
