"""Seeded synthetic inputs and random-init weights for the triangle path.

Inputs come from numpy PCG64 so that the CPU oracle, the GPU kernels and the
committed fixtures all see the same bits: seed 0 draws the pair tensor z,
seed 1 the single representation s, seed 2 the weights. Linears are
Glorot-uniform ``U(+-sqrt(6/(fan_in+fan_out)))``; LayerNorm weight is
``1 + 0.1 N(0,1)`` and bias ``0.1 N(0,1)`` so that neither is degenerate.

Weights are produced in the PyTorch ``[out, in]`` layout under the
Protenix/OpenFold3 field names (``layer_norm_in``, ``linear_a_p`` ...), as plain
nested dicts of float32 arrays; ``foldjax_amd.params`` turns them into each
port's own container.
"""

from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    # no finite value overflows 32 bits here (the largest, 0xFF7FFFFF, gains
    # at most 0x8000); NaN patterns may, and are restored below
    r = (u >> 16) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = x[nan]
    return out


def _glorot(rng, out_f: int, in_f: int) -> np.ndarray:
    lim = np.sqrt(6.0 / (in_f + out_f))
    return rng.uniform(-lim, lim, size=(out_f, in_f)).astype(np.float32)


def _ln(rng, c: int) -> dict:
    return {
        "weight": (1.0 + 0.1 * rng.standard_normal(c)).astype(np.float32),
        "bias": (0.1 * rng.standard_normal(c)).astype(np.float32),
    }


def trimul_weights(c_z: int = 128, c_h: int = 128, seed: int = 2) -> dict:
    """Tri-mul weights under the Protenix/OpenFold3 field names, torch layout."""
    rng = np.random.default_rng(seed)
    return {
        "layer_norm_in": _ln(rng, c_z),
        "linear_a_p": {"weight": _glorot(rng, c_h, c_z)},
        "linear_a_g": {"weight": _glorot(rng, c_h, c_z)},
        "linear_b_p": {"weight": _glorot(rng, c_h, c_z)},
        "linear_b_g": {"weight": _glorot(rng, c_h, c_z)},
        "layer_norm_out": _ln(rng, c_h),
        "linear_z": {"weight": _glorot(rng, c_z, c_h)},
        "linear_g": {"weight": _glorot(rng, c_z, c_z)},
    }


def triattn_weights(c_z: int = 128, heads: int = 4, head_dim: int = 32, seed: int = 2) -> dict:
    """Tri-attn weights under the Protenix field names (``linear``, ``attention``)."""
    rng = np.random.default_rng(seed)
    hd = heads * head_dim
    return {
        "layer_norm": _ln(rng, c_z),
        "linear": {"weight": _glorot(rng, heads, c_z)},
        "attention": {
            "linear_q": {"weight": _glorot(rng, hd, c_z)},
            "linear_k": {"weight": _glorot(rng, hd, c_z)},
            "linear_v": {"weight": _glorot(rng, hd, c_z)},
            "linear_o": {"weight": _glorot(rng, c_z, hd)},
            "linear_g": {"weight": _glorot(rng, hd, c_z)},
        },
    }


def transition_weights(c: int = 128, expansion: int = 4, seed: int = 2) -> dict:
    """Transition weights under the Protenix field names (``linear_a`` is the
    silu branch), torch layout."""
    rng = np.random.default_rng(seed)
    h = expansion * c
    return {
        "layer_norm": _ln(rng, c),
        "linear_a": {"weight": _glorot(rng, h, c)},
        "linear_b": {"weight": _glorot(rng, h, c)},
        "linear_out": {"weight": _glorot(rng, c, h)},
    }


def single_attention_weights(c_s: int = 384, c_z: int = 128, heads: int = 16, seed: int = 2) -> dict:
    """Boltz-2 ``AttentionPairBias`` weights plus the layer's ``pre_norm_s``,
    torch layout, Boltz-2 module names."""
    rng = np.random.default_rng(seed)
    return {
        "pre_norm_s": _ln(rng, c_s),
        "proj_q": {"weight": _glorot(rng, c_s, c_s), "bias": (0.1 * rng.standard_normal(c_s)).astype(np.float32)},
        "proj_k": {"weight": _glorot(rng, c_s, c_s)},
        "proj_v": {"weight": _glorot(rng, c_s, c_s)},
        "proj_g": {"weight": _glorot(rng, c_s, c_s)},
        "proj_o": {"weight": _glorot(rng, c_s, c_s)},
        "proj_z_norm": _ln(rng, c_z),
        "proj_z": {"weight": _glorot(rng, heads, c_z)},
    }


def single_input(n: int, c_s: int = 384, seed: int = 1, batch: int | None = None) -> np.ndarray:
    """``s ~ N(0,1)`` of shape ``[N, c_s]`` (or ``[B, N, c_s]``), float32."""
    rng = np.random.default_rng(seed)
    shape = (n, c_s) if batch is None else (batch, n, c_s)
    return rng.standard_normal(shape, dtype=np.float32)


def pair_input(n: int, c_z: int = 128, seed: int = 0, batch: int | None = None) -> np.ndarray:
    """``z ~ N(0,1)`` of shape ``[N, N, c_z]`` (or ``[B, N, N, c_z]``), float32."""
    rng = np.random.default_rng(seed)
    shape = (n, n, c_z) if batch is None else (batch, n, n, c_z)
    return rng.standard_normal(shape, dtype=np.float32)


def token_mask(n: int, n_real: int) -> np.ndarray:
    t = np.zeros(n, dtype=np.float32)
    t[:n_real] = 1.0
    return t


def pair_mask(n: int, n_real: int | None = None, batch: int | None = None) -> np.ndarray:
    """Pair mask ``t (x) t`` for a token mask with ``n_real`` leading ones."""
    t = token_mask(n, n if n_real is None else n_real)
    m = np.outer(t, t).astype(np.float32)
    return m if batch is None else np.broadcast_to(m, (batch, n, n)).copy()


def cast_tree(tree, fn):
    """Apply ``fn`` to every array leaf of a nested dict."""
    if isinstance(tree, dict):
        return {k: cast_tree(v, fn) for k, v in tree.items()}
    if tree is None:
        return None
    return fn(tree)


def pairformer_layer_weights(c_s: int = 384, c_z: int = 128, heads_pair: int = 4, heads_single: int = 16,
                             seed: int = 2) -> dict:
    """All weights of one Pairformer layer as torch-layout field dicts, each
    sublayer from its own seed (``seed``, ``seed + 1``, ...)."""
    return {
        "tri_mul_out": trimul_weights(c_z, c_z, seed=seed),
        "tri_mul_in": trimul_weights(c_z, c_z, seed=seed + 1),
        "tri_att_start": triattn_weights(c_z, heads_pair, c_z // heads_pair, seed=seed + 2),
        "tri_att_end": triattn_weights(c_z, heads_pair, c_z // heads_pair, seed=seed + 3),
        "transition_z": transition_weights(c_z, seed=seed + 4),
        "attention": single_attention_weights(c_s, c_z, heads_single, seed=seed + 5),
        "transition_s": transition_weights(c_s, seed=seed + 6),
    }
