"""Helpers shared by the GPU parity tests: seeded inputs, tolerances, printing."""

from __future__ import annotations

import sys

import numpy as np
import torch

from foldjax_amd import synthetic as syn

FP32_MAX_ABS = 1e-4  # north-star bar in fp32 mode
BF16_REL = 2e-2      # north-star bar in bf16 mode (vs an fp32 reference)


def say(msg: str) -> None:
    """Name the case before each GPU step, flushed, so a fault is attributable."""
    print(msg, file=sys.stderr, flush=True)


def device_tensor(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda").to(dtype)


def prep(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """The exact values the GPU sees, as float64 (bf16-rounded in bf16 mode)."""
    a = np.asarray(a, dtype=np.float32)
    if dtype == torch.bfloat16:
        a = syn.bf16_round(a)
    return a.astype(np.float64)


def prep_tree(tree, dtype):
    return syn.cast_tree(tree, lambda a: prep(a, dtype))


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().astype(np.float64)


def max_abs(got, want) -> float:
    return float(np.max(np.abs(np.asarray(got) - np.asarray(want))))


def rel_err(got, want) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def assert_parity(got, want, dtype, what=""):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    if dtype == torch.float32:
        err = max_abs(got, want)
        assert err <= FP32_MAX_ABS, f"{what}: fp32 max-abs error {err:.3e} > {FP32_MAX_ABS}"
    else:
        err = rel_err(got, want)
        assert err <= BF16_REL, f"{what}: bf16 relative error {err:.3e} > {BF16_REL}"
    return err


def mask_case(kind: str, n: int, seed: int = 3) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if kind == "ones":
        return np.ones((n, n), np.float32)
    if kind == "tail":
        return syn.pair_mask(n, max(1, n - max(1, n // 10)))
    if kind == "random":
        m = (rng.random((n, n)) > 0.25).astype(np.float32)
        m[:, 0] = 1.0
        return m
    if kind == "row0":  # one fully masked row
        m = np.ones((n, n), np.float32)
        m[min(1, n - 1), :] = 0.0
        return m
    raise ValueError(kind)


def spike_rows(rng: np.random.Generator, rows: int, c: int = 128) -> np.ndarray:
    """Every other row bf16-exact with its mean dwarfing its spread: a
    constant value (8-bit mantissa, 2^-4 to 2^15, either sign) with one or two
    entries one bf16 step away, mean^2 / variance up to about 10^6; ordinary
    rows in between."""
    x = rng.standard_normal((rows, c)).astype(np.float32)
    for r in range(0, rows, 2):
        base = float(syn.bf16_round(np.array(
            [2.0 ** rng.integers(-4, 15) * (1 + rng.integers(1, 128) / 128) * (1 if rng.random() < 0.5 else -1)],
            dtype=np.float32))[0])
        step = abs(base) * 2.0 ** -7
        x[r] = base
        for k in rng.choice(c, size=1 + r % 2, replace=False):
            x[r, k] = syn.bf16_round(np.array([base + step * (1 if rng.random() < 0.5 else -1)], dtype=np.float32))[0]
    return x
