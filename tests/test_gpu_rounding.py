"""Where the bfloat16 kernels sit relative to each port's own bfloat16 program.

The reference's ports round at different points in bfloat16 (oracle
``bf16_program``): Protenix stores bfloat16 logits and probabilities
(``PXT/triangle.py:850-860``) and rounds every LayerNorm op, Boltz-2 keeps its
attention scores, softmax and probability-value product in float32
(``B2T/triangle_attention.py:446-455``) and rounds the normalized value
before the LayerNorm affine (``B2P/_common.py:15-26``). The kernels have one
set of rounding points for all three ports. These tests show that their
output is within the bf16 bar (relative error 2e-2) of the exact result and
of both ports' emulated programs, and print the distances, including the
distance between the two programs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from foldjax_amd import params as P
from foldjax_amd import protenix
from foldjax_amd import synthetic as syn
from oracle import triangle as O
from tests.gpu_util import BF16_REL, device_tensor, mask_case, prep, prep_tree, rel_err, say, to_np

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _distances(got, run):
    exact = run()
    progs = {}
    for port in ("boltz2", "protenix"):
        with O.bf16_program(port):
            progs[port] = run()
    d = {
        "exact": rel_err(got, exact),
        "boltz2": rel_err(got, progs["boltz2"]),
        "protenix": rel_err(got, progs["protenix"]),
        "boltz2-vs-protenix": rel_err(progs["boltz2"], progs["protenix"]),
        "boltz2-vs-exact": rel_err(progs["boltz2"], exact),
        "protenix-vs-exact": rel_err(progs["protenix"], exact),
    }
    say("  " + ", ".join(f"{k} {v:.2e}" for k, v in d.items()))
    return d


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_bf16_within_bar_of_both_programs(starting):
    n, heads = 64, 4
    say(f"rounding programs: triattn n={n} starting={starting}")
    z = syn.pair_input(n, 128, seed=11)
    m = mask_case("tail", n)
    w = syn.triattn_weights(128, heads, 32, seed=12)
    got = to_np(protenix.triangle_attention(device_tensor(z, BF), device_tensor(m, BF), P.triattn_to_protenix(w),
                                            num_heads=heads, starting=starting))
    torch.cuda.synchronize()
    rows = (m if starting else m.T).max(axis=1) > 0
    sel = (lambda a: a[rows]) if starting else (lambda a: a[:, rows])
    d = _distances(sel(got), lambda: sel(O.protenix_triangle_attention(
        prep(z, BF), prep(m, BF), prep_tree(w, BF), num_heads=heads, starting=starting)))
    for k in ("exact", "boltz2", "protenix"):
        assert d[k] <= BF16_REL, (k, d)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_bf16_within_bar_of_both_programs(direction):
    n = 64
    say(f"rounding programs: trimul n={n} {direction}")
    z = syn.pair_input(n, 128, seed=13)
    m = mask_case("tail", n)
    w = syn.trimul_weights(128, 128, seed=14)
    got = to_np(protenix.triangle_multiplication(device_tensor(z, BF), device_tensor(m, BF),
                                                 P.trimul_to_protenix(w), direction))
    torch.cuda.synchronize()
    d = _distances(got, lambda: O.protenix_triangle_multiplication(prep(z, BF), prep(m, BF), prep_tree(w, BF),
                                                                   direction))
    for k in ("exact", "boltz2", "protenix"):
        assert d[k] <= BF16_REL, (k, d)
