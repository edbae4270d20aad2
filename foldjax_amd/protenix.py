"""Protenix triangle entry points with the reference's call signatures.

Mirrors ``src/foldjax/models/protenix/models/triangle/triangle.py:98``
(``triangle_multiplication``) and ``:456`` (``triangle_attention``). Selectors
keep their names and values and gain ``"hip"``:

* ``PROTENIX_TRIANGLE_MULTIPLICATION_BACKEND`` in {cueq, xla, hip}
  (reference ``triangle.py:130-145``);
* ``PROTENIX_TRIANGLE_BACKEND`` / ``attention_backend`` in
  {xla, xla_jit, tokamax, cueq, cueq_jit, hip, hip_jit}, lower-cased
  (reference ``triangle.py:41-71``); ``_jit`` has no meaning here and maps to
  the same kernels.

Unknown values raise ``ValueError`` with the reference's messages; the JAX
backends raise ``RuntimeError``. Default: ``"hip"``.
"""

from __future__ import annotations

import os

import torch

from foldjax_amd import kernels
from foldjax_amd.kernels import TransitionWeights, TriAttnWeights, TriMulWeights
from foldjax_amd.params import pack_transition_torch, pack_triattn_protenix, pack_trimul_torch

DEFAULT_BACKEND = "hip"
_REFERENCE_ONLY = "the {kind} backend {name!r} is a JAX backend of the reference; this package provides 'hip'"


def _triangle_attention_backend() -> str:
    backend = os.environ.get("PROTENIX_TRIANGLE_BACKEND", DEFAULT_BACKEND).lower()
    if backend not in {"xla", "xla_jit", "tokamax", "cueq", "cueq_jit", "hip", "hip_jit"}:
        raise ValueError(f"unsupported triangle attention backend: {backend!r}")
    return backend


def triangle_multiplication(
    z: torch.Tensor,
    mask: torch.Tensor | None,
    params,
    direction: str,
    *,
    chunk_size: int | None = None,
    use_jit: bool = False,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Protenix triangle multiplication (update only, or ``residual + update``)."""
    backend = os.environ.get("PROTENIX_TRIANGLE_MULTIPLICATION_BACKEND", DEFAULT_BACKEND).lower()
    if backend not in {"cueq", "xla", "hip"}:
        raise ValueError(f"unsupported triangle multiplication backend: {backend!r}")
    if backend != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle multiplication", name=backend))
    w = params if isinstance(params, TriMulWeights) else pack_trimul_torch(params, z.dtype, z.device)
    return kernels.trimul(z, mask, w, direction, eps=1e-5, residual=residual)


def triangle_attention(
    x: torch.Tensor,
    mask: torch.Tensor | None,
    params,
    *,
    num_heads: int,
    starting: bool = True,
    inf: float = 1e9,
    q_chunk_size: int | None = None,
    attention_backend: str | None = None,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Protenix triangle attention (update only, or ``residual + update``)."""
    backend = _triangle_attention_backend() if attention_backend is None else attention_backend
    if backend not in {"xla", "xla_jit", "tokamax", "cueq", "cueq_jit", "hip", "hip_jit"}:
        raise ValueError(f"unsupported triangle attention backend: {backend!r}")
    if backend.removesuffix("_jit") != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle attention", name=backend))
    w = params if isinstance(params, TriAttnWeights) else pack_triattn_protenix(params, x.dtype, x.device)
    if w.heads != num_heads:
        raise ValueError(f"num_heads={num_heads} but the bias projection has {w.heads} heads")
    return kernels.triattn(x, mask, w, starting=starting, inf=inf, eps=1e-5, residual=residual)


def hip_attention_core(q, k, v, triangle_bias, mask_bias, *, scale: float) -> torch.Tensor:
    """Drop-in for ``PXT/triangle_cueq.py``'s ``cueq_attention_core`` (via
    ``src/foldjax/models/_cueq.py:66``)."""
    return kernels.triattn_core(q, k, v, triangle_bias, mask_bias, scale=scale)


def transition(
    x: torch.Tensor,
    params,
    *,
    chunk_size: int | None = None,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Protenix ``transition`` (``PXP/primitives.py:96-114``); ``chunk_size`` is
    accepted and unused (the widened form never leaves the chip)."""
    w = params if isinstance(params, TransitionWeights) else pack_transition_torch(params, x.dtype, x.device)
    return kernels.transition(x, w, residual=residual)
