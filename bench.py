"""Benchmark of one Pairformer block on one MI355X.

One step = one Boltz-2-form Pairformer layer at N=1024, c_z=128, c_s=384,
bf16: tri-mul outgoing and incoming, tri-attn starting and ending node
(4 heads x 32), the pair transition (4x SwiGLU), the single attention with
pair bias (16 heads) and the single transition, every residual fused. Inputs
are synthetic (z, s ~ N(0,1), PCG64 seeds 0/1) with a 5% padded tail (973 real
tokens) and random-init weights (seed 2).

Prints one JSON line. ``value`` times the K steps with no instrumentation;
the same K steps then run again while the library records HIP events on its
launch stream around every kernel (``fjx_prof_*``), which gives the
per-kernel durations, ``ms_per_step_profiled`` and the roofline object (for
the kernel with the largest total time). The CPU baseline times the float64
numpy oracle (``oracle/``) on a bounded sample and scales it to the metric's
unit.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--n N] [--no-cpu]
    python bench.py --config trunk|long      (the N=2048 trunk / the N=3072 block)
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
    p.add_argument("--op", default="block", choices=["block", "trimul", "triattn", "transition", "copy"],
                   help="profiling aid: run only one sublayer kind per step instead of the whole block")
    p.add_argument("--config", default="block", choices=["block", "trunk", "long"],
                   help="block: one layer at N=1024 (the headline line); trunk: the 48-layer trunk at N=2048 "
                        "with an all-ones mask; long: one unchunked layer at N=3072 with 3012 real tokens")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_pairformer_block_n1024_bf16.json")


def measured_traffic(kernel: str, n: int):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (already scaled by the copy-kernel
    calibration), or None when that summary does not cover this kernel/N."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    k = rec.get("kernels", {}).get(kernel)
    if rec.get("n") != n or not k:
        return None
    return int(k["hbm_bytes"])


def cpu_baseline(n_target: int, n_sample: int, budget_s: float = 25.0) -> dict:
    """Time the float64 oracle on one Pairformer layer at ``n_sample`` and
    scale to ``n_target`` by the ratio of algorithmic flops."""
    import numpy as np

    from foldjax_amd import synthetic as syn
    from foldjax_amd.pairformer import flops_block
    from oracle import triangle as O

    try:
        from threadpoolctl import threadpool_info

        threads = max([int(i.get("num_threads", 1)) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover - informational only
        threads = len(os.sched_getaffinity(0))
    n = n_sample
    n_real = n - int(round(0.05 * n))
    r = lambda a: syn.bf16_round(a).astype(np.float64)  # noqa: E731
    z = r(syn.pair_input(n, 128, seed=0, batch=1))
    s = r(syn.single_input(n, 384, seed=1, batch=1))
    tm = syn.token_mask(n, n_real)[None].astype(np.float64)
    pm = syn.pair_mask(n, n_real)[None].astype(np.float64)
    w = syn.pairformer_layer_weights(seed=2)

    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        O.boltz2_pairformer_layer(w, s, z, tm, pm)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s / 2 or len(times) >= 5:
            break
    t = float(np.median(times))
    scale = sum(flops_block(n_target).values()) / sum(flops_block(n).values())
    return {
        "value": t * scale * 1e3,
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"float64 numpy oracle, one Pairformer layer (tri-mul out+in, tri-attn start+end, pair transition, "
            f"single attention with pair bias, single transition) at N={n} ({n_real} real tokens), median of "
            f"{len(times)} run(s) = {t * 1e3:.1f} ms, scaled to N={n_target} by the algorithmic-flop ratio {scale:.1f}"
        ),
    }


def run_config(a) -> int:
    """The other two BASELINE configurations, reported as their own JSON
    lines: the 48-layer trunk at N=2048 (all-ones mask, each layer with its
    own random weights) and one unchunked layer at N=3072 (3012 real tokens)."""
    import torch

    from foldjax_amd import _lib
    from foldjax_amd import synthetic as syn
    from foldjax_amd.pairformer import PairformerLayerWeights, flops_block

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    if a.config == "trunk":
        n, n_real, layers = 2048, 2048, 48
    else:
        n, n_real, layers = 3072, 3012, 1
    z0 = torch.from_numpy(syn.pair_input(n, 128, seed=0, batch=1)).to(dev, dtype)
    s0 = torch.from_numpy(syn.single_input(n, 384, seed=1, batch=1)).to(dev, dtype)
    tmask = torch.from_numpy(syn.token_mask(n, n_real)[None]).to(dev, dtype)
    pmask = torch.from_numpy(syn.pair_mask(n, n_real)[None]).to(dev, dtype)
    stack = [PairformerLayerWeights.random(dtype, dev, seed=2 + l) for l in range(layers)]

    def step():
        s, z = s0, z0
        for layer in stack:
            s, z = layer.forward(s, z, tmask, pmask)
        return s, z

    steps = max(1, min(a.steps, 3 if layers > 1 else a.steps))
    for _ in range(max(1, min(a.warmup, 1))):
        step()
    torch.cuda.synchronize(dev)
    _lib.prof_reset()
    _lib.prof_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        s, z = step()
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    _lib.prof_enable(False)
    stats = _lib.prof_read()
    if not (torch.isfinite(z.float()).all() and torch.isfinite(s.float()).all()):
        print("non-finite output", file=sys.stderr)
        return 1
    ms = elapsed * 1e3 / steps
    per = {k: {"avg_ms": round(v[0] / v[1], 4), "launches": v[1]} for k, v in stats.items() if v[1]}
    fl = sum(flops_block(n).values()) * layers
    what = "48-layer Pairformer trunk" if layers > 1 else "one Pairformer block, unchunked in HBM"
    print(json.dumps({
        "metric": f"ms per {what} @N={n} c_z=128 bf16",
        "value": round(ms, 3), "unit": "ms", "n_gpus": 1, "steps": steps, "higher_is_better": False,
        "ms_per_block": round(ms / layers, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 1), "dtype": "bf16",
        "data": "synthetic: z, s ~ N(0,1), random-init weights per layer",
        "config": {"workload": what, "n": n, "n_real": n_real, "layers": layers, "c_z": 128, "c_s": 384},
        "kernels": per,
    }))
    return 0


def main() -> int:
    a = _args()
    if a.gpus != 1:
        print(
            "bench.py measures one MI355X: this build has no multi-GPU path "
            f"(asked for --gpus {a.gpus}); run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    if a.config != "block":
        return run_config(a)

    import torch

    from foldjax_amd import _lib
    from foldjax_amd import synthetic as syn
    from foldjax_amd.pairformer import PairformerLayerWeights, flops_block, flops_triangle

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    n = a.n
    n_real = n - int(round(a.pad_frac * n))
    z0 = torch.from_numpy(syn.pair_input(n, 128, seed=0, batch=1)).to(dev, dtype)
    s0 = torch.from_numpy(syn.single_input(n, 384, seed=1, batch=1)).to(dev, dtype)
    tmask = torch.from_numpy(syn.token_mask(n, n_real)[None]).to(dev, dtype)
    pmask = torch.from_numpy(syn.pair_mask(n, n_real)[None]).to(dev, dtype)
    layer = PairformerLayerWeights.random(dtype, dev, seed=2)

    from foldjax_amd import kernels

    tri = layer.triangle
    steps_fn = {
        "block": lambda: layer.forward(s0, z0, tmask, pmask),
        "trimul": lambda: (s0, kernels.trimul(z0, pmask, tri.tri_mul_out, "outgoing", residual=z0)),
        "triattn": lambda: (s0, kernels.triattn(z0, pmask, tri.tri_att_start, starting=True, residual=z0)),
        "transition": lambda: (s0, kernels.transition(z0, layer.transition_z, residual=z0)),
        # a plain device copy of the pair tensor (N*N*128*2 bytes each way): the
        # calibration point for the FETCH_SIZE / WRITE_SIZE counters
        "copy": lambda: (s0, z0.clone()),
    }
    step = steps_fn[a.op]
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize(dev)

    # the timed steps run without per-kernel events (their markers cost about
    # 0.1 ms per block); the same number of steps is then repeated with the
    # events on for the per-kernel averages and the roofline
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    s, z = s0, z0
    for _ in range(a.steps):
        s, z = step()
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    if not (torch.isfinite(z.float()).all() and torch.isfinite(s.float()).all()):
        print("non-finite output", file=sys.stderr)
        return 1

    _lib.prof_reset()
    _lib.prof_enable(True)
    torch.cuda.synchronize(dev)
    t1 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize(dev)
    elapsed_prof = time.perf_counter() - t1
    _lib.prof_enable(False)
    stats = _lib.prof_read()

    ms_step = elapsed * 1e3 / a.steps
    if a.op != "block":
        per = {k: {"avg_ms": round(v[0] / v[1], 4), "launches": v[1]} for k, v in stats.items() if v[1]}
        print(json.dumps({"op": a.op, "n": n, "ms_per_step": round(ms_step, 4), "kernels": per}))
        return 0
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
        entry = {"avg_ms": round(avg, 4), "launches": cnt, "share": round(tot_ms / (elapsed_prof * 1e3), 4)}
        if name in per_launch:
            tf = per_launch[name] / (avg * 1e-3) / 1e12
            entry.update(tflops=round(tf, 1), mfma_frac=round(tf / PEAK_BF16_TFLOPS, 4))
        kern[name] = entry
    dominant = max(kern, key=lambda k: kern[k]["avg_ms"] * kern[k]["launches"])
    t_contract = kern["trimul_contract"]["avg_ms"] * 2
    t_flash = kern["triattn_flash"]["avg_ms"] * 2
    primary = (2 * fl["contraction"] + 2 * fl["attn_core"]) / ((t_contract + t_flash) * 1e-3) / 1e12 / PEAK_BF16_TFLOPS
    tri_kernels = ("trimul_prologue", "trimul_contract", "trimul_epilogue", "triattn_prologue", "triattn_flash",
                   "triattn_epilogue")
    sub_t = sum(kern[k]["avg_ms"] * kern[k]["launches"] for k in tri_kernels if k in kern) / a.steps
    secondary = (2 * fl["trimul"] + 2 * fl["triattn"]) / (sub_t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS
    block_tflops = sum(flops_block(n).values()) / (ms_step * 1e-3) / 1e12
    dom_flops = per_launch.get(dominant)
    traffic = measured_traffic(dominant, n)
    if dom_flops is not None:
        ach = dom_flops / (kern[dominant]["avg_ms"] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic, "kernel": dominant}
    else:
        roof = {"bound": "hbm", "achieved": None, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": None,
                "traffic": traffic, "kernel": dominant}

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
        "ms_per_step_profiled": round(elapsed_prof * 1e3 / a.steps, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: z, s ~ N(0,1) (PCG64 seeds 0, 1), Glorot-uniform random-init weights, 5% padded tail mask",
        "config": {
            "workload": "one Pairformer block (Boltz-2 layer): tri-mul out+in, tri-attn start+end, pair transition "
                        "4x SwiGLU, single attention with pair bias, single transition; residuals fused",
            "n": n, "n_real": n_real, "c_z": 128, "c_hidden": 128, "c_s": 384, "tri_heads": 4, "tri_head_dim": 32,
            "single_heads": 16,
        },
        "block_tflops": round(block_tflops, 1),
        "roofline": roof,
        "cpu_baseline": cpu,
        "mfma_frac": {"primary": round(primary, 4), "secondary": round(secondary, 4)},
        "kernels": kern,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
