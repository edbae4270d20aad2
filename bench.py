"""Benchmark of one Pairformer block on one MI355X.

One step = one Boltz-2-form Pairformer layer at N=1024, c_z=128, c_s=384:
tri-mul outgoing and incoming, tri-attn starting and ending node (4 heads x
32), the pair transition (4x SwiGLU), the single attention with pair bias (16
heads) and the single transition, every residual fused. The pair track runs
in bf16; the single track in fp32 by default, as the reference runs it
(``B2K/pairformer.py:182-199``). Inputs are synthetic (z, s ~ N(0,1), PCG64
seeds 0/1) with a 5% padded tail (973 real tokens) and random-init weights
(seed 2).

Prints one JSON line. ``value`` times the K steps with no instrumentation;
the same K steps then run again while the library records HIP events on its
launch stream around every kernel (``fjx_prof_*``), which gives the
per-kernel durations, ``ms_per_step_profiled`` and the roofline object (for
the kernel with the largest total time). ``other_configs_gpu`` times the
other baseline configurations the same way (no events); ``cpu_baseline``
times the float32 numpy restatement (``oracle/``) on a bounded sample of the
headline workload and on configs 1 and 2.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--n N] [--no-cpu] [--no-configs]
    python bench.py --op trimul|triattn|transition|transition_pb|copy   (one sublayer kind, a profiling aid)
    python bench.py --n 2048 --pad-frac 0 --layers 48 --no-cpu --no-configs   (config 4's trunk, per kernel)
    python bench.py --n 3072 --pad-frac 0.01953125 --no-cpu --no-configs      (config 5's block, per kernel)
    python bench.py --cpu-whole [--n N]   (the whole block on the CPU beside the sampled estimate)
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
    p.add_argument("--steps", type=int, default=30)
    p.add_argument("--warmup", type=int, default=20,
                   help="untimed steps first; the GPU clock needs some 100 ms of load to settle")
    p.add_argument("--n", type=int, default=1024)
    p.add_argument("--pad-frac", type=float, default=0.05)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--no-configs", action="store_true", help="skip the GPU timings of configs 1, 2, 4 and 5")
    p.add_argument("--single-dtype", default="fp32", choices=["fp32", "bf16"],
                   help="the single track's dtype: fp32 as the reference runs it over the bf16 pair track "
                        "(B2K/pairformer.py:182-199), or bf16")
    p.add_argument("--op", default="block",
                   choices=["block", "trimul", "triattn", "transition", "transition_pb", "copy", "mixprobe",
                            "hbmprobe"],
                   help="profiling aid: run only one sublayer kind per step instead of the whole block; mixprobe: "
                        "the issue rate of the flash attention's per-tile instruction mix alone; hbmprobe: the rate "
                        "of a plain HBM streaming kernel over the pair tensor's size")
    p.add_argument("--c-z", type=int, default=128,
                   help="with --op trimul|triattn|transition: the pair width (other than 128 runs the general-width "
                        "paths, e.g. 64 for the template stack, 384 for OpenDDE's structural pair track)")
    p.add_argument("--c-h", type=int, default=128, help="with --op trimul: the hidden width")
    p.add_argument("--heads", type=int, default=4, help="with --op triattn: heads of 32 channels")
    p.add_argument("--layers", type=int, default=1,
                   help="with --op block: layers per step, each with its own weights (48 at --n 2048 --pad-frac 0 is "
                        "BASELINE config 4's trunk; the per-kernel averages then cover the whole trunk)")
    p.add_argument("--cpu-whole", action="store_true",
                   help="no GPU work: time the whole block at --n on the CPU once, beside the sampled estimate "
                        "the bench line reports (checks the sample model)")
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


def _median_time(fn, budget_s: float, max_runs: int = 3) -> tuple[float, int]:
    import numpy as np

    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_runs or time.perf_counter() - t_start > budget_s:
            return float(np.median(times)), len(times)


def _rows_model(fn, r1: int, r2: int, n: int) -> float:
    """Time ``fn(rows)`` at r1 and r2 rows and extrapolate the linear model
    t = shared + rows * per_row (exact: attention rows are independent) to n."""
    t1, _ = _median_time(lambda: fn(r1), 0.0, 1)
    t2, _ = _median_time(lambda: fn(r2), 0.0, 1)
    per_row = max(t2 - t1, 0.0) / (r2 - r1)
    return t1 + (n - r1) * per_row


def cpu_baseline(n: int, n_real: int, with_configs: bool = True) -> dict:
    """The float32 numpy restatement (``oracle/``, the reference's XLA path in
    fp32) timed on this host's cores at the headline size. Every part runs
    whole on the block's own inputs except the two triangle attentions,
    which dominate and are sampled by rows:

    * tri-mul outgoing and incoming, whole;
    * tri-attn starting and ending node, each on r1 and r2 of its N rows,
      extrapolated linearly in rows (rows are independent; the LayerNorm and
      bias of the whole grid are in both samples, and the ending node samples
      its own transposed grid);
    * the pair transition, the single attention with pair bias and the
      single transition, whole.

    ``--cpu-whole`` checks this sample model against the whole block.
    Also times config 1 of the baseline table (tri-mul out+in at N=256 in
    fp32) and config 2 (tri-attn start+end at N=384, 346 real tokens),
    whole."""
    import numpy as np

    from foldjax_amd import synthetic as syn
    from oracle import triangle as O

    cores = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_info

        blas = max([int(i.get("num_threads", 1)) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover - informational only
        blas = cores
    w = syn.pairformer_layer_weights(seed=2)
    z = syn.pair_input(n, 128, seed=0, batch=1)
    s = syn.single_input(n, 384, seed=1, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    r1, r2 = 8, 56
    parts = {}
    with O.compute_dtype(np.float32):
        z = z.astype(np.float32)
        for key, d in (("tri_mul_out", "outgoing"), ("tri_mul_in", "incoming")):
            parts[key], _ = _median_time(lambda key=key, d=d: O.protenix_triangle_multiplication(z, pm, w[key], d),
                                         0.0, 1)
        for key, st in (("tri_att_start", True), ("tri_att_end", False)):
            parts[key] = _rows_model(lambda r, key=key, st=st: O.protenix_triangle_attention(
                z, pm, w[key], num_heads=4, starting=st, rows=np.arange(r)), r1, r2, n)
        parts["transition_z"], _ = _median_time(lambda: O.transition(z, w["transition_z"]), 0.0, 1)
        a = w["attention"]

        def single():
            s_ln = O.layer_norm(s, a["pre_norm_s"]["weight"], a["pre_norm_s"]["bias"])
            s2 = s + O.boltz2_attention_pair_bias(a, s_ln, z, tm)
            return s2 + O.transition(s2, w["transition_s"])

        parts["single_track"], _ = _median_time(single, 0.0, 1)
    total = sum(parts.values())
    out = {
        "value": round(total * 1e3, 1),
        "unit": "ms",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"float32 numpy restatement of the reference's XLA path (oracle/triangle.py) at N={n} ({n_real} real "
            f"tokens), BLAS on {blas} threads, elementwise numpy on one: tri-mul outgoing and incoming whole "
            f"({parts['tri_mul_out']:.1f} + {parts['tri_mul_in']:.1f} s); tri-attn starting and ending node each "
            f"on {r1} and {r2} of its rows, extrapolated linearly to {n} ({parts['tri_att_start']:.1f} + "
            f"{parts['tri_att_end']:.1f} s); pair transition whole ({parts['transition_z']:.1f} s); single track "
            f"whole ({parts['single_track']:.2f} s)"
        ),
        "parts_s": {k: round(v, 3) for k, v in parts.items()},
    }
    if not with_configs:
        return out
    with O.compute_dtype(np.float32):
        # configs 1 and 2, whole
        z1 = syn.pair_input(256, 128, seed=0, batch=1).astype(np.float32)
        def config1():
            z = z1 + O.protenix_triangle_multiplication(z1, None, w["tri_mul_out"], "outgoing")
            return z + O.protenix_triangle_multiplication(z, None, w["tri_mul_in"], "incoming")

        def config2():
            z = z2 + O.protenix_triangle_attention(z2, pm2, w["tri_att_start"], num_heads=4, starting=True)
            return z + O.protenix_triangle_attention(z, pm2, w["tri_att_end"], num_heads=4, starting=False)

        t_c1, _ = _median_time(config1, 0.0, 1)
        z2 = syn.pair_input(384, 128, seed=0, batch=1).astype(np.float32)
        pm2 = syn.pair_mask(384, 346)[None]
        t_c2, _ = _median_time(config2, 0.0, 1)
    out["configs"] = {
        "config1_trimul_out_in_n256_fp32_ms": round(t_c1 * 1e3, 1),
        "config2_triattn_start_end_n384_ms": round(t_c2 * 1e3, 1),
        "note": "configs 1 and 2 timed whole, each second sublayer on the first one's output",
    }
    return out


def cpu_whole_block(n: int, n_real: int) -> dict:
    """The whole block on the CPU once, against the sampled estimate of
    ``cpu_baseline`` at the same size: the float32 restatement of the Boltz-2
    layer (``oracle.boltz2_pairformer_layer``: tri-mul out and in, tri-attn
    start and end over the whole grid, 16 rows at a time, the pair transition,
    the single attention with pair bias and the single transition) on the
    same inputs. This checks the sample model; the default bench line keeps
    the bounded sample."""
    import numpy as np

    from foldjax_amd import synthetic as syn
    from oracle import triangle as O

    w = syn.pairformer_layer_weights(seed=2)
    z = syn.pair_input(n, 128, seed=0, batch=1)
    s = syn.single_input(n, 384, seed=1, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    with O.compute_dtype(np.float32):
        t0 = time.perf_counter()
        s_out, z_out = O.boltz2_pairformer_layer(w, s, z, tm, pm)
        whole = time.perf_counter() - t0
    if not (np.all(np.isfinite(z_out)) and np.all(np.isfinite(s_out))):
        raise RuntimeError("non-finite CPU block output")
    sampled = cpu_baseline(n, n_real, with_configs=False)
    return {
        "n": n, "n_real": n_real, "cores": len(os.sched_getaffinity(0)),
        "whole_ms": round(whole * 1e3, 1), "sampled_ms": sampled["value"],
        "sampled_over_whole": round(sampled["value"] / (whole * 1e3), 3),
        "sample": sampled["sample"],
    }


def hbm_bytes_per_launch(n: int, single_dtype) -> dict:
    """Algorithmic HBM bytes of one launch of the block's memory-bound
    kernels at size n (bf16 pair tensor, c = 128): each input and output
    element once. Pair row = 128 x 2 B.

    * tri-mul prologue: x and the mask in, a and b out (channel-major);
    * tri-mul epilogue: o and x in (x for the output gate and the residual),
      z out;
    * tri-attn prologue: x and the mask in; q, k, v, the [4, N, N] bias and
      the [N, N] fp32 mask bias out;
    * tri-attn epilogue: o and x in, z out;
    * pair transition: x in, z out, plus the single attention's [16, N, N]
      pair bias (fp32 for an fp32 single track)."""
    row = 128 * 2
    pos = n * n
    mask = pos * 2
    pb = 16 * pos * (4 if str(single_dtype).endswith("float32") else 2)
    return {
        "trimul_prologue": 3 * pos * row + mask,
        "trimul_epilogue": 3 * pos * row,
        "triattn_prologue": 4 * pos * row + mask + 4 * pos * 2 + pos * 4,
        "triattn_epilogue": 3 * pos * row,
        "transition": 2 * pos * row + pb,
    }


MIXES = {0: "flash tile: 10 MFMA + 16 exp + 24 VALU", 1: "without the bias widenings: 10 MFMA + 16 exp + 8 VALU",
         2: "10 MFMA alone", 3: "16 exp alone", 4: "24 VALU alone",
         5: "the flash tile on 32x32x16 MFMAs: 4 x 32x32x16 + 2 x 16x16x32 + 16 exp + 24 VALU",
         6: "4 x 32x32x16 + 2 x 16x16x32 MFMA alone"}


def mix_probe(n: int) -> dict:
    """``fjx_probe_issue_mix``: each mix at 1-4 waves per SIMD; ns for one
    SIMD to issue one tile's instructions, and that rate times the tiles one
    SIMD runs in a flash launch at size n (4 heads, 16 x 64 tiles over 256 CUs
    x 4 SIMDs) -- the issue floor of the launch."""
    import torch

    from foldjax_amd import _lib

    torch.zeros(1, device="cuda")  # the device context
    iters = 2000
    simds = torch.cuda.get_device_properties(0).multi_processor_count * 4
    tiles_per_simd = n * 4 * (n // 16) * (n // 64) / simds
    out = {"op": "mixprobe", "n": n, "iters": iters, "simds": simds, "tiles_per_simd": tiles_per_simd, "mixes": {}}
    for mix, what in MIXES.items():
        row = {"mix": what}
        for w in (1, 2, 3, 4):
            ms = _lib.probe_issue_mix(mix, w, iters)
            ns = ms * 1e6 / (iters * w)
            row[f"waves{w}"] = {"ns_per_tile": round(ns, 2), "floor_ms": round(ns * tiles_per_simd / 1e6, 4)}
        out["mixes"][str(mix)] = row
    return out


HBM_MODES = {0: "copy", 1: "copy, nontemporal loads and stores", 2: "read only", 3: "write only"}


def hbm_probe(n: int) -> dict:
    """``fjx_probe_hbm_stream`` over two buffers of the pair tensor's size at
    n (n * n * 128 bf16 values): each mode at 1, 2, 4 and 8 workgroups per
    CU, GB/s of bytes moved (a copy moves twice the buffer)."""
    import torch

    from foldjax_amd import _lib

    torch.zeros(1, device="cuda")  # the device context
    nbytes = n * n * 128 * 2
    out = {"op": "hbmprobe", "n": n, "bytes": nbytes, "modes": {}}
    for mode, what in HBM_MODES.items():
        row = {"mode": what}
        moved = nbytes * (2 if mode in (0, 1) else 1)
        for w in (1, 2, 4, 8):
            ms = min(_lib.probe_hbm_stream(mode, w, nbytes) for _ in range(3))
            row[f"wgs{w}"] = {"ms": round(ms, 4), "gbs": round(moved / (ms * 1e-3) / 1e9, 1)}
        out["modes"][str(mode)] = row
    return out


def _timed(fn, steps: int, warmup: int, dev) -> float:
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize(dev)
    return (time.perf_counter() - t0) * 1e3 / steps


def other_configs(single_dtype) -> dict:
    """GPU milliseconds of the other baseline configurations, timed like the
    headline (no per-kernel events): config 1 (tri-mul out+in, N=256, fp32,
    all-ones mask), config 2 (tri-attn start+end, N=384, bf16, 346 real
    tokens), config 4 (the 48-layer trunk at N=2048, all-ones mask, each
    layer with its own weights, stacked) and config 5 (one unchunked layer at N=3072,
    3012 real tokens)."""
    import torch

    from foldjax_amd import boltz2, kernels
    from foldjax_amd import synthetic as syn
    from foldjax_amd.pairformer import PairformerLayerWeights, flops_block
    from foldjax_amd.stacking import stacked_or_stack

    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    t = lambda a, dt: torch.from_numpy(a).to(dev, dt)  # noqa: E731
    out = {}
    layer32 = PairformerLayerWeights.random(torch.float32, dev, seed=2)
    z1 = t(syn.pair_input(256, 128, seed=0, batch=1), torch.float32)
    tri = layer32.triangle

    def config1():
        # z += tri-mul outgoing, then z += tri-mul incoming of that z
        z = kernels.trimul(z1, None, tri.tri_mul_out, "outgoing", residual=z1)
        return kernels.trimul(z, None, tri.tri_mul_in, "incoming", residual=z, out=z)

    out["config1_trimul_out_in_n256_fp32_ms"] = round(_timed(config1, 20, 3, dev), 4)
    del layer32, z1
    layer = PairformerLayerWeights.random(bf, dev, seed=2, single_dtype=single_dtype)
    tri = layer.triangle
    z2 = t(syn.pair_input(384, 128, seed=0, batch=1), bf)
    m2 = t(syn.pair_mask(384, 346)[None], bf)

    def config2():
        # z += tri-attn starting node, then z += tri-attn ending node of that z
        z = kernels.triattn(z2, m2, tri.tri_att_start, starting=True, residual=z2)
        return kernels.triattn(z, m2, tri.tri_att_end, starting=False, residual=z, out=z)

    out["config2_triattn_start_end_n384_bf16_ms"] = round(_timed(config2, 20, 3, dev), 4)
    del z2, m2
    for key, n, n_real, layers, steps in (("config5_block_n3072_ms", 3072, 3012, 1, 3),
                                          ("config4_trunk48_n2048_ms", 2048, 2048, 48, 2)):
        z0 = t(syn.pair_input(n, 128, seed=0, batch=1), bf)
        s0 = t(syn.single_input(n, 384, seed=1, batch=1), single_dtype)
        tmask = t(syn.token_mask(n, n_real)[None], single_dtype)
        pmask = t(syn.pair_mask(n, n_real)[None], bf)
        # the layers stacked once and run through Boltz-2's module forward
        # (donated s and z after the first layer), as a trunk's caller runs them
        trunk = {"layers": stacked_or_stack([PairformerLayerWeights.random(bf, dev, seed=2 + i,
                                                                           single_dtype=single_dtype)
                                             for i in range(layers)])}

        def step():
            return boltz2.pairformer_module_forward(trunk, s0, z0, tmask, pmask)

        ms = _timed(step, steps, 1, dev)
        s, z = step()
        torch.cuda.synchronize(dev)
        if not (torch.isfinite(z.float()).all() and torch.isfinite(s.float()).all()):
            raise RuntimeError(f"non-finite output in {key}")
        out[key] = round(ms, 3)
        out[key.replace("_ms", "_tflops")] = round(sum(flops_block(n).values()) * layers / (ms * 1e-3) / 1e12, 1)
        del z0, s0, trunk, s, z
        torch.cuda.empty_cache()
    return out


def main() -> int:
    a = _args()
    if a.gpus != 1:
        print(
            "bench.py measures one MI355X: this build has no multi-GPU path "
            f"(asked for --gpus {a.gpus}); run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    if a.cpu_whole:
        n_real = a.n - int(round(a.pad_frac * a.n))
        print(json.dumps({"cpu_whole_block": cpu_whole_block(a.n, n_real)}))
        return 0
    import torch

    from foldjax_amd import _lib
    from foldjax_amd import synthetic as syn
    from foldjax_amd.pairformer import PairformerLayerWeights, flops_block, flops_triangle

    if a.op == "mixprobe":
        print(json.dumps(mix_probe(a.n)))
        return 0
    if a.op == "hbmprobe":
        print(json.dumps(hbm_probe(a.n)))
        return 0

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    sdt = torch.float32 if a.single_dtype == "fp32" else torch.bfloat16
    n = a.n
    n_real = n - int(round(a.pad_frac * n))
    z0 = torch.from_numpy(syn.pair_input(n, 128, seed=0, batch=1)).to(dev, dtype)
    s0 = torch.from_numpy(syn.single_input(n, 384, seed=1, batch=1)).to(dev, sdt)
    tmask = torch.from_numpy(syn.token_mask(n, n_real)[None]).to(dev, sdt)
    pmask = torch.from_numpy(syn.pair_mask(n, n_real)[None]).to(dev, dtype)
    layer = PairformerLayerWeights.random(dtype, dev, seed=2, single_dtype=sdt)
    # further layers of a trunk (--layers), each with its own weights
    more = [PairformerLayerWeights.random(dtype, dev, seed=2 + i, single_dtype=sdt) for i in range(1, a.layers)]

    from foldjax_amd import kernels

    # a trunk (--layers > 1) runs as users run it: the layers stacked once
    # (one [L, ...] buffer per weight kind) through Boltz-2's module forward,
    # whose first layer writes new s and z (the inputs stay as they are for
    # the next step) and whose further layers update them in place
    from foldjax_amd import boltz2
    from foldjax_amd.stacking import stacked_or_stack

    trunk = {"layers": stacked_or_stack([layer] + more)} if more else None

    def block_step():
        if trunk is None:
            return layer.forward(s0, z0, tmask, pmask)
        return boltz2.pairformer_module_forward(trunk, s0, z0, tmask, pmask)

    tri = layer.triangle
    if a.op in ("trimul", "triattn", "transition") and (a.c_z, a.c_h, a.heads) != (128, 128, 4):
        # the general-width paths at another pair width
        z0 = torch.from_numpy(syn.pair_input(n, a.c_z, seed=0, batch=1)).to(dev, dtype)
        from foldjax_amd import params as PP
        tri.tri_mul_out = PP.pack_trimul_torch(PP.trimul_to_protenix(syn.trimul_weights(a.c_z, a.c_h, seed=3)), dtype, dev)
        tri.tri_att_start = PP.pack_triattn_protenix(
            PP.triattn_to_protenix(syn.triattn_weights(a.c_z, a.heads, 32, seed=4)), dtype, dev)
        layer.transition_z = PP.pack_transition_torch(syn.transition_weights(a.c_z, seed=5), dtype, dev)
    steps_fn = {
        "block": block_step,
        "trimul": lambda: (s0, kernels.trimul(z0, pmask, tri.tri_mul_out, "outgoing", residual=z0)),
        "triattn": lambda: (s0, kernels.triattn(z0, pmask, tri.tri_att_start, starting=True, residual=z0)),
        "transition": lambda: (s0, kernels.transition(z0, layer.transition_z, residual=z0)),
        # the block's form: the transition also writes the single attention's pair bias
        "transition_pb": lambda: (s0, kernels.transition(z0, layer.transition_z, residual=z0,
                                                         pair_bias_for=layer.attention)[0]),
        # one elementwise pass over the pair tensor (N*N*128*2 bytes read and
        # written by torch's neg kernel): the calibration point for the
        # FETCH_SIZE / WRITE_SIZE counters
        "copy": lambda: (s0, torch.neg(z0)),
    }
    step = steps_fn[a.op]
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize(dev)
    if a.op != "block":
        # a single-kernel op's few warm-up steps are a few ms of GPU work, too
        # short for the GPU's clock to settle: the timed loop then carried a
        # one-off ~40 ms ramp (0.64 -> 2.5 ms per step at 20 steps). The
        # profiling ops keep stepping until 0.5 s of warm-up have passed.
        t_w = time.perf_counter()
        while time.perf_counter() - t_w < 0.5:
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
        print(json.dumps({"op": a.op, "n": n, "c_z": a.c_z, "c_h": a.c_h, "heads": a.heads,
                          "ms_per_step": round(ms_step, 4), "kernels": per}))
        return 0
    fl = flops_triangle(n)
    per_launch = {
        "trimul_contract": fl["contraction"],
        "triattn_flash": fl["attn_core"],
        "transition": flops_block(n)["transition_z"],
    }
    hbm = hbm_bytes_per_launch(n, sdt)
    kern = {}
    for name, (tot_ms, cnt) in stats.items():
        if cnt == 0:
            continue
        avg = tot_ms / cnt
        entry = {"avg_ms": round(avg, 4), "launches": cnt, "share": round(tot_ms / (elapsed_prof * 1e3), 4)}
        if name in per_launch:
            tf = per_launch[name] / (avg * 1e-3) / 1e12
            entry.update(tflops=round(tf, 1), mfma_frac=round(tf / PEAK_BF16_TFLOPS, 4))
        if name in hbm:
            gbs = hbm[name] / (avg * 1e-3) / 1e9
            entry.update(alg_bytes=hbm[name], hbm_gbs=round(gbs, 1), hbm_frac=round(gbs / PEAK_HBM_GBS, 4))
        kern[name] = entry
    dominant = max(kern, key=lambda k: kern[k]["avg_ms"] * kern[k]["launches"])
    t_contract = kern["trimul_contract"]["avg_ms"] * 2
    t_flash = kern["triattn_flash"]["avg_ms"] * 2
    primary = (2 * fl["contraction"] + 2 * fl["attn_core"]) / ((t_contract + t_flash) * 1e-3) / 1e12 / PEAK_BF16_TFLOPS
    tri_kernels = ("trimul_prologue", "trimul_contract", "trimul_epilogue", "triattn_prologue", "triattn_flash",
                   "triattn_epilogue")
    sub_t = sum(kern[k]["avg_ms"] * kern[k]["launches"] for k in tri_kernels if k in kern) / a.steps
    secondary = a.layers * (2 * fl["trimul"] + 2 * fl["triattn"]) / (sub_t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS
    block_tflops = a.layers * sum(flops_block(n).values()) / (ms_step * 1e-3) / 1e12
    dom_flops = per_launch.get(dominant)
    traffic = measured_traffic(dominant, n)
    if dom_flops is not None:
        ach = dom_flops / (kern[dominant]["avg_ms"] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic, "kernel": dominant}
    else:
        roof = {"bound": "hbm", "achieved": None, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": None,
                "traffic": traffic, "kernel": dominant}

    configs = None if a.no_configs else other_configs(sdt)
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(n, n_real)

    out = {
        "metric": METRIC,
        "value": round(ms_step / a.layers, 4),  # ms per block (a step runs --layers blocks)
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
            "single_heads": 16, "pair_dtype": "bf16", "single_dtype": a.single_dtype, "layers": a.layers,
        },
        "block_tflops": round(block_tflops, 1),
        "roofline": roof,
        "cpu_baseline": cpu,
        "other_configs_gpu": configs,
        "mfma_frac": {"primary": round(primary, 4), "secondary": round(secondary, 4)},
        "kernels": kern,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
