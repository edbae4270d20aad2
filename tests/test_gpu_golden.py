"""The HIP path against the committed golden fixtures (tests/golden): every
fixture whose shape the kernels take (widths a multiple of 8, head width 32),
both directions and nodes; float32 fixtures at max-abs 1e-4, bf16-rounded
ones at relative 2e-2 (bf16 mode).

Attention rows whose every key is masked are checked for finiteness only:
their reference value depends on the arithmetic's precision (in float64 the
-1e9 mask bias cancels and the row's unmasked softmax remains, as in the
fixtures; in fp32 it rounds every score to the same multiple of 64)."""

from __future__ import annotations

import pytest
import torch

import numpy as np

from foldjax_amd import params as P
from foldjax_amd import protenix
from tests.golden import fixtures
from tests.gpu_util import assert_parity, device_tensor, say, to_np

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


def _supported_trimul(c):
    return c["z"].shape[-1] % 8 == 0 and c["w"]["layer_norm_out"]["weight"].shape[0] % 8 == 0


def _supported_triattn(c):
    hd = c["w"]["attention"]["linear_q"]["weight"].shape[0]
    return c["z"].shape[-1] % 8 == 0 and hd // c["heads"] == 32


@pytest.mark.parametrize("case", [c for c in fixtures.cases("trimul") if _supported_trimul(c)],
                         ids=lambda c: f"{c['tag']}-{c['name']}")
def test_trimul_golden(case):
    dt = DT[case["tag"]]
    z, m = device_tensor(case["z"], dt), device_tensor(case["mask"], dt)
    for d in ("outgoing", "incoming"):
        say(f"golden trimul {case['tag']} {case['name']} {d}")
        got = protenix.triangle_multiplication(z, m, P.trimul_to_protenix(case["w"]), d)
        torch.cuda.synchronize()
        assert_parity(to_np(got), case["out"][d], dt, f"{case['name']} {d}")


@pytest.mark.parametrize("case", [c for c in fixtures.cases("triattn") if _supported_triattn(c)],
                         ids=lambda c: f"{c['tag']}-{c['name']}")
def test_triattn_golden(case):
    dt = DT[case["tag"]]
    z, m = device_tensor(case["z"], dt), device_tensor(case["mask"], dt)
    for node in ("starting", "ending"):
        say(f"golden triattn {case['tag']} {case['name']} {node}")
        got = protenix.triangle_attention(z, m, P.triattn_to_protenix(case["w"]), num_heads=case["heads"],
                                          starting=node == "starting")
        torch.cuda.synchronize()
        g, want = to_np(got), case["out"][node]
        assert np.all(np.isfinite(g))
        if node == "starting":
            rows = np.flatnonzero(case["mask"].any(axis=1))
            g, want = g[rows], want[rows]
        else:
            cols = np.flatnonzero(case["mask"].any(axis=0))
            g, want = g[:, cols], want[:, cols]
        assert_parity(g, want, dt, f"{case['name']} {node}")
