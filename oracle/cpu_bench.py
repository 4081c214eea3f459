"""TEST INFRASTRUCTURE — CPU baseline leg of bench.py.

Times the oracle CPU device (the reference's clang backend restated:
clang -shared -O3 -march=native, one call per kernel on the calling thread,
cpu.rs:151-208, 328-380) on a bounded sample of a benchmark config, pinned to
one core like the reference. Prints one JSON object.

Usage: python -m oracle.cpu_bench <c1|c2|c3|c4|c5> [--core N]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def _time(fn, runs: int, warmup: int = 1) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def host_cpu(core: int, nproc: int) -> dict:
    """The host CPU the baseline ran on: lscpu's model, CPU count and clock
    fields, nproc (CPUs this process could use before pinning itself to one
    core) and the pinned core's current clock from /proc/cpuinfo."""
    info = {"nproc": nproc, "cpu_count": os.cpu_count(), "pinned_core": core}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        fields = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        for key, name in (("Model name", "model"), ("CPU(s)", "lscpu_cpus"), ("Socket(s)", "sockets"),
                          ("Thread(s) per core", "threads_per_core"), ("CPU max MHz", "max_mhz"),
                          ("CPU min MHz", "min_mhz"), ("Hypervisor vendor", "hypervisor")):
            if key in fields:
                info[name] = fields[key].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            blocks = f.read().split("\n\n")
        for b in blocks:
            kv = dict((k.strip(), v.strip()) for k, v in (ln.split(":", 1) for ln in b.splitlines() if ":" in ln))
            if kv.get("processor") == str(core):
                info["core_mhz"] = float(kv.get("cpu MHz", "nan"))
                info.setdefault("model", kv.get("model name"))
    except OSError:
        pass
    return info


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("config")
    ap.add_argument("--core", type=int, default=None)
    args = ap.parse_args()
    cores = sorted(os.sched_getaffinity(0))
    core = args.core if args.core is not None else cores[0]
    os.sched_setaffinity(0, {core})

    import numpy as np

    import oracle
    import ferrograd_amd as fg
    from ferrograd_amd import Tensor

    oracle.load()
    dev = "cpu"
    out = {"cores": 1, "kind": "port", "core": core, "host": host_cpu(core, len(cores))}
    if args.config == "c2":
        n = 1 << 26
        r = np.random.default_rng(2)
        a, b, c = (Tensor.new(r.uniform(-1, 1, n).astype(np.float32), [n], dev) for _ in range(3))
        step = lambda: a.mul(b).add(c).relu().realize()  # noqa: E731
        t = _time(step, runs=5)
        out.update(value=4 * n * 4 / t / 1e9, unit="GB/s", seconds=t,
                   sample="full C2 (2^26 elements, 2 reference kernels), median of 5 after 1 warmup")
    elif args.config == "c1":
        x = Tensor.new(np.random.default_rng(1).standard_normal((4096, 4096)).astype(np.float32), [4096, 4096], dev)
        s0, s1 = Tensor.scalar(0.5, dev), Tensor.scalar(1.0, dev)
        step = lambda: x.mul(s0).add(s1).relu().sum([1]).realize()  # noqa: E731
        t = _time(step, runs=5)
        out.update(value=(4096 * 4096 * 4 + 4096 * 4) / t / 1e9, unit="GB/s", seconds=t,
                   sample="full C1 ([4096,4096], 2 reference kernels), median of 5 after 1 warmup")
    elif args.config == "c3":
        # The full config: about 9 s per product on one core, once after one
        # warm-up product (which also compiles the kernels).
        rows = 4096
        r = np.random.default_rng(5)
        x = Tensor.new(r.standard_normal((rows, 4096)).astype(np.float32), [rows, 4096], dev)
        w = Tensor.new(r.uniform(-1 / 64, 1 / 64, (4096, 4096)).astype(np.float32), [4096, 4096], dev)
        b = Tensor.zeros([4096], dev)
        step = lambda: x.matmul(w.permute([1, 0])).add(b).realize()  # noqa: E731
        t = _time(step, runs=1)
        flops = 2 * rows * 4096 * 4096
        out.update(value=flops / t / 1e12, unit="TFLOP/s", seconds=t,
                   sample="full C3 (x[4096,4096] @ W[4096,4096]^T + b, 2 reference kernels), once after 1 warmup")
    elif args.config == "c4":
        from ferrograd_amd.mlp import mlp_setup

        step, _ = mlp_setup(fg, dev, batch=256, dims=(784, 128, 10))
        t = _time(step, runs=10, warmup=2)
        out.update(value=1.0 / t, unit="steps/s", seconds=t, sample="C4 train step, median of 10 after 2 warmup")
    elif args.config == "c5":
        # A C5 step on one core takes about 25 minutes. Every GEMM of the step
        # scales with the batch and the SGD update does not, so time steps at
        # the full layer widths for two batches and extrapolate t(B) = a + b*B.
        # Measured on one core: 1.1, 2.2, 8.7 and 20 s at B = 16, 32, 64, 128.
        # Up to B = 32 the activations stay in cache; from B = 64 on the time
        # grows linearly, so the fit uses 64 and 128.
        from ferrograd_amd.mlp import mlp_setup

        ts = {}
        for batch in (64, 128):
            step, _ = mlp_setup(fg, dev, batch=batch, dims=(784, 4096, 4096, 10))
            ts[batch] = _time(step, runs=1, warmup=1)
        b = (ts[128] - ts[64]) / 64.0
        a = ts[64] - 64.0 * b
        t = a + 8192.0 * b
        out.update(value=1.0 / t, unit="steps/s", seconds=t, sample_seconds={str(k): v for k, v in ts.items()},
                   sample="C5 widths (784->4096->4096->10) at B=64 and B=128, one step each after 1 warmup; "
                          "step time extrapolated linearly in B to B=8192")
    else:
        raise SystemExit(f"unknown config {args.config}")
    print(json.dumps(out))


if __name__ == "__main__":
    main()
