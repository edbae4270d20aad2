"""Benchmark of the Pairformer triangle hot path on one MI355X.

One step = one pass of the pair-track triangle sublayers of a Pairformer
block (tri-mul outgoing, incoming, tri-attn starting, ending; residuals
fused) at N=1024, c_z=128, 4 heads x 32, bf16, on a synthetic z ~ N(0,1) with
a 5% padded tail (973 real tokens) and random-init weights.

Prints one JSON line. Per-kernel durations come from HIP events that the
library records on its launch stream around every kernel during the timed
steps (``fjx_prof_*``); the roofline object is for the kernel with the largest
total time. The CPU baseline times the float64 numpy oracle (``oracle/``) on a
bounded sample and scales it to the metric's unit.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--n N] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "ms/Pairformer block @N=1024 c_z=128 bf16; tri-mul+tri-attn MFMA % of peak"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--n", type=int, default=1024)
    p.add_argument("--pad-frac", type=float, default=0.05)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--cpu-n", type=int, default=256, help="size of the CPU oracle sample")
    return p.parse_args()


def cpu_baseline(n_target: int, n_sample: int, budget_s: float = 25.0) -> dict:
    """Time the float64 oracle on one triangle block at ``n_sample`` and scale
    to ``n_target`` by the ratio of algorithmic flops."""
    import numpy as np

    from foldjax_amd import synthetic as syn
    from foldjax_amd.pairformer import flops_triangle
    from oracle import triangle as O

    try:
        from threadpoolctl import threadpool_info

        threads = max([int(i.get("num_threads", 1)) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover - informational only
        threads = len(os.sched_getaffinity(0))
    n = n_sample
    n_real = n - int(round(0.05 * n))
    z = syn.bf16_round(syn.pair_input(n, 128, seed=0)).astype(np.float64)
    m = syn.pair_mask(n, n_real).astype(np.float64)
    ws = [syn.trimul_weights(seed=2), syn.trimul_weights(seed=3)]
    wa = [syn.triattn_weights(seed=4), syn.triattn_weights(seed=5)]

    def block(z):
        z = z + O.protenix_triangle_multiplication(z, m, ws[0], "outgoing")
        z = z + O.protenix_triangle_multiplication(z, m, ws[1], "incoming")
        z = z + O.protenix_triangle_attention(z, m, wa[0], num_heads=4, starting=True)
        z = z + O.protenix_triangle_attention(z, m, wa[1], num_heads=4, starting=False)
        return z

    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        block(z)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s / 2 or len(times) >= 5:
            break
    t = float(np.median(times))
    f = lambda nn: sum(2 * v for k, v in flops_triangle(nn).items() if k in ("trimul", "triattn"))  # noqa: E731
    scale = f(n_target) / f(n)
    return {
        "value": t * scale * 1e3,
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"float64 numpy oracle, one triangle block (tri-mul out+in, tri-attn start+end) at N={n} "
            f"({n_real} real tokens), median of {len(times)} run(s) = {t * 1e3:.1f} ms, scaled to N={n_target} "
            f"by the algorithmic-flop ratio {scale:.1f}"
        ),
    }


def main() -> int:
    a = _args()
    if a.gpus != 1:
        print(
            "bench.py measures one MI355X: this build has no multi-GPU path "
            f"(asked for --gpus {a.gpus}); run with --gpus 1",
            file=sys.stderr,
        )
        return 2

    import torch

    from foldjax_amd import _lib
    from foldjax_amd import synthetic as syn
    from foldjax_amd.pairformer import TriangleSublayers, flops_triangle

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    n = a.n
    n_real = n - int(round(a.pad_frac * n))
    z0 = torch.from_numpy(syn.pair_input(n, 128, seed=0)).to(dev, dtype)
    mask = torch.from_numpy(syn.pair_mask(n, n_real)).to(dev, dtype)
    block = TriangleSublayers.random(dtype, dev, seed=2)

    for _ in range(a.warmup):
        block.forward(z0, mask)
    torch.cuda.synchronize(dev)

    _lib.prof_reset()
    _lib.prof_enable(True)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    z = z0
    for _ in range(a.steps):
        z = block.forward(z0, mask)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    _lib.prof_enable(False)
    stats = _lib.prof_read()
    if not torch.isfinite(z.float()).all():
        print("non-finite output", file=sys.stderr)
        return 1

    ms_step = elapsed * 1e3 / a.steps
    fl = flops_triangle(n)
    per_launch = {
        "trimul_contract": fl["contraction"],
        "triattn_flash": fl["attn_core"],
    }
    kern = {}
    for name, (tot_ms, cnt) in stats.items():
        if cnt == 0:
            continue
        avg = tot_ms / cnt
        entry = {"avg_ms": round(avg, 4), "launches": cnt, "share": round(tot_ms / (elapsed * 1e3), 4)}
        if name in per_launch:
            tf = per_launch[name] / (avg * 1e-3) / 1e12
            entry.update(tflops=round(tf, 1), mfma_frac=round(tf / PEAK_BF16_TFLOPS, 4))
        kern[name] = entry
    dominant = max(kern, key=lambda k: kern[k]["avg_ms"] * kern[k]["launches"])
    t_contract = kern["trimul_contract"]["avg_ms"] * 2
    t_flash = kern["triattn_flash"]["avg_ms"] * 2
    primary = (2 * fl["contraction"] + 2 * fl["attn_core"]) / ((t_contract + t_flash) * 1e-3) / 1e12 / PEAK_BF16_TFLOPS
    sub_t = sum(v["avg_ms"] * v["launches"] for v in kern.values()) / a.steps
    secondary = (2 * fl["trimul"] + 2 * fl["triattn"]) / (sub_t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS
    dom_flops = per_launch.get(dominant)
    if dom_flops is not None:
        ach = dom_flops / (kern[dominant]["avg_ms"] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": None, "kernel": dominant}
    else:
        roof = {"bound": "hbm", "achieved": None, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": None,
                "traffic": None, "kernel": dominant}

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(n, a.cpu_n)

    out = {
        "metric": METRIC,
        "value": round(ms_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: z~N(0,1) (PCG64 seed 0), Glorot-uniform random-init weights, 5% padded tail mask",
        "config": {
            "workload": "pairformer block triangle sublayers (tri-mul out+in, tri-attn start+end, fused residuals)",
            "n": n, "n_real": n_real, "c_z": 128, "c_hidden": 128, "heads": 4, "head_dim": 32,
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "mfma_frac": {"primary": round(primary, 4), "secondary": round(secondary, 4)},
        "kernels": kern,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
