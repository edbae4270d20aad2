"""Write the golden fixtures of the triangle operations (run once, by hand):

    python -m tests.golden.make_golden

Each case holds seeded inputs (pair tensor, pair mask, torch-layout weights)
and the expected output computed by the scalar loops of tests/_brute.py in
float64 -- code independent of the vectorised oracle -- so a fixture pins the
oracle (tests/test_oracle.py) and the HIP path (tests/test_gpu_golden.py).
The reference holds no numeric fixture for this path, so these are the
build's own known answers, at small shapes: N in {3, 5, 8, 17, 24, 33},
widths 4 .. 64, 1 to 4 heads, head widths 3 .. 32,
masks all-ones / random 0-1 / tail padding / one fully masked row, each once
with float32 values and once with bf16-rounded inputs and weights.
"""

from __future__ import annotations

import os

import numpy as np

from foldjax_amd import synthetic as syn
from tests import _brute as B

HERE = os.path.dirname(os.path.abspath(__file__))

# (name, n, c_z, c_h, mask kind)
TRIMUL = [
    ("n3c4", 3, 4, 4, "ones"),
    ("n5c8", 5, 8, 8, "random"),
    ("n8c8h16", 8, 8, 16, "tail"),
    ("n17c32", 17, 32, 32, "fullrow"),
    ("n33c8", 33, 8, 8, "random"),
]
# (name, n, c_z, heads, head_dim, mask kind)
TRIATTN = [
    ("n3c4h1d3", 3, 4, 1, 3, "ones"),
    ("n5c8h2d8", 5, 8, 2, 8, "random"),
    ("n8c8h4d3", 8, 8, 4, 3, "tail"),
    ("n17c32h1d32", 17, 32, 1, 32, "fullrow"),
    ("n24c64h2d32", 24, 64, 2, 32, "random"),
]


def _mask(rng, n, kind):
    if kind == "ones":
        return np.ones((n, n), np.float32)
    if kind == "random":
        return rng.integers(0, 2, size=(n, n)).astype(np.float32)
    if kind == "tail":
        return syn.pair_mask(n, n - max(1, n // 4))
    m = np.ones((n, n), np.float32)
    m[1, :] = 0.0  # one fully masked row
    return m


def _flat(prefix, tree, out):
    for k, v in tree.items():
        if isinstance(v, dict):
            _flat(f"{prefix}{k}.", v, out)
        elif v is not None:
            out[f"{prefix}{k}"] = np.asarray(v, np.float32)


def _cases(rounded: bool):
    r = syn.bf16_round if rounded else (lambda a: np.asarray(a, np.float32))
    tag = "bf16" if rounded else "fp32"
    tm, ta = {}, {}
    for i, (name, n, c, ch, kind) in enumerate(TRIMUL):
        rng = np.random.default_rng(100 + i)
        z = r(rng.standard_normal((n, n, c)).astype(np.float32))
        mask = _mask(rng, n, kind)
        w = syn.cast_tree(syn.trimul_weights(c, ch, seed=200 + i), r)
        key = f"{tag}.{name}"
        tm[f"{key}.z"] = z
        tm[f"{key}.mask"] = mask
        _flat(f"{key}.w.", w, tm)
        for d in ("outgoing", "incoming"):
            want = B.trimul(z.astype(np.float64).tolist(), mask.tolist(), B.tolist(w), d == "outgoing")
            tm[f"{key}.out.{d}"] = np.asarray(want, np.float64)
    for i, (name, n, c, h, dh, kind) in enumerate(TRIATTN):
        rng = np.random.default_rng(300 + i)
        z = r(rng.standard_normal((n, n, c)).astype(np.float32))
        mask = _mask(rng, n, kind)
        w = syn.cast_tree(syn.triattn_weights(c, h, dh, seed=400 + i), r)
        key = f"{tag}.{name}"
        ta[f"{key}.z"] = z
        ta[f"{key}.mask"] = mask
        _flat(f"{key}.w.", w, ta)
        ta[f"{key}.heads"] = np.asarray(h)
        for node in ("starting", "ending"):
            want = B.triattn(z.astype(np.float64).tolist(), mask.tolist(), B.tolist(w), h, node == "starting")
            ta[f"{key}.out.{node}"] = np.asarray(want, np.float64)
    return tm, ta


def main() -> None:
    tm, ta = {}, {}
    for rounded in (False, True):
        a, b = _cases(rounded)
        tm.update(a)
        ta.update(b)
    np.savez_compressed(os.path.join(HERE, "trimul_cases.npz"), **tm)
    np.savez_compressed(os.path.join(HERE, "triattn_cases.npz"), **ta)
    print(f"wrote {len(tm)} + {len(ta)} arrays")


if __name__ == "__main__":
    main()
