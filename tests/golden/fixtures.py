"""Loader of the golden fixtures written by tests/golden/make_golden.py."""

from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _nest(flat: dict) -> dict:
    out: dict = {}
    for key, value in flat.items():
        node = out
        parts = key.split(".")
        for p in parts[:-1]:
            node = node.setdefault(p, {})
        node[parts[-1]] = value
    return out


def cases(kind: str) -> list[dict]:
    """The cases of ``kind`` ("trimul" or "triattn"): dicts with ``tag``
    ("fp32" or "bf16"), ``name``, ``z`` [N, N, C], ``mask`` [N, N], ``w`` (the
    torch-layout weight tree of foldjax_amd.synthetic), ``out`` (per direction
    or node, float64) and, for triattn, ``heads``."""
    with np.load(os.path.join(HERE, f"{kind}_cases.npz")) as f:
        arrays = {k: f[k] for k in f.files}
    by_case: dict = {}
    for key, value in arrays.items():
        tag, name, rest = key.split(".", 2)
        by_case.setdefault((tag, name), {})[rest] = value
    out = []
    for (tag, name), flat in sorted(by_case.items()):
        c = _nest(flat)
        c["tag"], c["name"] = tag, name
        if "heads" in c:
            c["heads"] = int(c["heads"])
        out.append(c)
    return out
