"""Boltz-2 triangle entry points with the reference's call signatures.

Mirrors ``src/foldjax/models/boltz2/models/triangle/triangle.py:33`` and
``.../triangle_attention.py:79`` (plus the kernel-level
``triangle_cueq.py:47,72``). The selectors keep their names and values and
gain ``"hip"``, the backend this package provides:

* ``BOLTZ_JAX_TRIANGLE_MULTIPLICATION_BACKEND`` in {xla, cueq, hip}
  (reference: ``triangle.py:67-76``);
* ``triangle_backend`` argument in {xla, pallas, tokamax, cueq, hip}
  (reference: ``triangle_attention.py:384-418``).

Unknown values raise ``ValueError`` with the reference's messages. The JAX
backends (xla/cueq/pallas/tokamax) live in the reference, not here: selecting
one raises ``RuntimeError`` instead of silently running something else.
The default of both selectors in this package is ``"hip"``.
"""

from __future__ import annotations

import os

import torch

from foldjax_amd import kernels
from foldjax_amd.kernels import TriAttnWeights, TriMulWeights
from foldjax_amd.params import pack_triattn_boltz2, pack_trimul_boltz2

DEFAULT_BACKEND = "hip"
_REFERENCE_ONLY = "the {kind} backend {name!r} is a JAX backend of the reference; this package provides 'hip'"


def triangle_multiplication_forward(
    params,
    x: torch.Tensor,
    mask: torch.Tensor,
    direction: str,
    eps: float = 1e-5,
    chunk_size: int = 128,
    glu_backend: str = "xla",
    contraction_precision: str = "float32",
    *,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Boltz-2 triangle multiplication; returns the update (``residual +
    update`` when ``residual`` is given, fused into the epilogue).

    ``chunk_size`` is accepted and unused: the contraction is never chunked.
    Both ``contraction_precision`` values run bf16 operands with fp32
    accumulation, which is what the reference's fp32-upcast contraction of
    bf16 values computes (``triangle.py:95-101``).
    """
    backend = os.getenv("BOLTZ_JAX_TRIANGLE_MULTIPLICATION_BACKEND", DEFAULT_BACKEND)
    if backend not in ("xla", "cueq", "hip"):
        raise ValueError(f"Unsupported triangle multiplication backend: {backend!r}")
    if backend != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle multiplication", name=backend))
    if contraction_precision not in ("float32", "bf16"):
        raise ValueError(f"Unsupported contraction_precision: {contraction_precision!r}")
    if glu_backend not in ("xla", "tokamax"):
        raise ValueError(f"Unsupported glu backend: {glu_backend!r}")
    w = params if isinstance(params, TriMulWeights) else pack_trimul_boltz2(params, x.dtype, x.device)
    return kernels.trimul(x, mask, w, direction, eps=eps, residual=residual)


def resolve_matmul_precision(matmul_precision: str) -> str:
    """Validate like ``triangle_attention.py:61-76``; the HIP path always
    accumulates in fp32."""
    key = matmul_precision.lower()
    if key in ("highest", "float32", "fp32", "default", "tensorfloat32", "tf32"):
        return key
    raise ValueError(f"Unsupported matmul_precision: {matmul_precision!r}")


def triangle_attention_forward(
    params,
    x: torch.Tensor,
    mask: torch.Tensor | None = None,
    starting: bool = True,
    inf: float = 1e9,
    eps: float = 1e-5,
    chunk_size: int = 128,
    q_chunk_size: int | None = None,
    matmul_precision: str = "highest",
    triangle_backend: str = DEFAULT_BACKEND,
    *,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Boltz-2 triangle attention (starting or ending node); chunk sizes are
    accepted and unused (the flash kernel never forms the score tensor)."""
    resolve_matmul_precision(matmul_precision)
    if triangle_backend not in ("xla", "pallas", "tokamax", "cueq", "hip"):
        raise ValueError(f"Unsupported triangle_backend: {triangle_backend!r}")
    if triangle_backend != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle attention", name=triangle_backend))
    w = params if isinstance(params, TriAttnWeights) else pack_triattn_boltz2(params, x.dtype, x.device)
    return kernels.triattn(x, mask, w, starting=starting, inf=inf, eps=eps, residual=residual)


def hip_attention_core(q, k, v, tri_bias, mask_bias, *, scale: float, precision=None) -> torch.Tensor:
    """Drop-in for ``cueq_attention_core`` (``triangle_cueq.py:47-69``): the
    scale is applied inside, so callers must not pre-scale q."""
    return kernels.triattn_core(q, k, v, tri_bias, mask_bias, scale=scale)


def hip_triangle_multiplication_forward(params, x, mask, direction, eps: float = 1e-5) -> torch.Tensor:
    """Drop-in for ``cueq_triangle_multiplication_forward`` (``triangle_cueq.py:72-102``)."""
    w = params if isinstance(params, TriMulWeights) else pack_trimul_boltz2(params, x.dtype, x.device)
    return kernels.trimul(x, mask, w, direction, eps=eps)
