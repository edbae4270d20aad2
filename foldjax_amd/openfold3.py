"""OpenFold3 triangle entry points with the reference's call signatures.

Mirrors ``src/foldjax/models/openfold3/models/triangle.py:82``
(``triangle_multiplication``, which has no backend switch upstream) and
``triangle_attention.py:95`` (``triangle_attention``). The attention selector
``OPENFOLD3_TRIANGLE_BACKEND`` / ``backend`` keeps its values {xla, cueq},
case-insensitive (reference ``triangle_attention.py:80,154-157``), and gains
``"hip"``, the default here.
"""

from __future__ import annotations

import os

import torch

from foldjax_amd import kernels
from foldjax_amd.kernels import TransitionWeights, TriAttnWeights, TriMulWeights
from foldjax_amd.params import OpenFold3PairBlockParams as PairBlockParams
from foldjax_amd.params import pack_transition_openfold3, pack_triattn_openfold3, pack_trimul_torch

DEFAULT_BACKEND = "hip"


def _default_backend() -> str:
    return os.environ.get("OPENFOLD3_TRIANGLE_BACKEND", DEFAULT_BACKEND).lower()


def triangle_multiplication(
    z: torch.Tensor,
    params,
    *,
    outgoing: bool,
    mask: torch.Tensor | None = None,
    eps: float = 1e-5,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """OpenFold3 triangle multiplication; ``mask=None`` means all ones."""
    w = params if isinstance(params, TriMulWeights) else pack_trimul_torch(params, z.dtype, z.device)
    return kernels.trimul(z, mask, w, "outgoing" if outgoing else "incoming", eps=eps, residual=residual)


def triangle_attention(
    x: torch.Tensor,
    params,
    *,
    no_heads: int,
    mask: torch.Tensor | None = None,
    starting: bool = True,
    inf: float = 1e9,
    eps: float = 1e-5,
    chunk_size: int | None = None,
    backend: str | None = None,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """OpenFold3 triangle attention; ``chunk_size`` is accepted and unused."""
    if backend is None:
        backend = _default_backend()
    backend = backend.lower()
    if backend not in {"xla", "cueq", "hip"}:
        raise ValueError(f"unsupported triangle attention backend: {backend!r}")
    if backend != "hip":
        raise RuntimeError(
            f"the triangle attention backend {backend!r} is a JAX backend of the reference; "
            "this package provides 'hip'"
        )
    w = params if isinstance(params, TriAttnWeights) else pack_triattn_openfold3(params, x.dtype, x.device)
    if w.heads != no_heads:
        raise ValueError(f"no_heads={no_heads} but the bias projection has {w.heads} heads")
    return kernels.triattn(x, mask, w, starting=starting, inf=inf, eps=eps, residual=residual)


def swiglu_transition(
    x: torch.Tensor,
    params,
    *,
    mask: torch.Tensor | None = None,
    eps: float = 1e-5,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """OpenFold3 ``swiglu_transition`` (``OF3/primitives.py:133-150``): the
    output is multiplied by ``mask`` over the last axis when given."""
    w = params if isinstance(params, TransitionWeights) else pack_transition_openfold3(params, x.dtype, x.device)
    return kernels.transition(x, w, row_mask=mask, residual=residual, eps=eps)


def pair_block(
    z: torch.Tensor,
    params: PairBlockParams,
    *,
    pair_mask: torch.Tensor,
    no_heads_pair: int,
    inf: float = 1e9,
    mask_transition: bool = True,
    tri_mul_first: bool = True,
    eps: float = 1e-5,
    chunk_size: int | None = None,
) -> torch.Tensor:
    """OpenFold3 ``pair_block`` (``OF3/pair_block.py:106-190``): the updated
    ``z`` after tri-mul out and in, tri-attn start and end (``tri_mul_first``
    orders the two pairs) and the SwiGLU transition, its output multiplied by
    ``pair_mask`` when ``mask_transition``. Every residual add is fused into
    the producing kernel. Upstream builds ``tri_att_end`` as a starting-node
    module and transposes ``z`` and the mask around it; the ending-node kernel
    here addresses the transposed grid directly, which is the same update
    without the two transposed copies. ``chunk_size`` is accepted for
    signature parity (the kernels stream rows with a fixed workspace)."""

    def mul_pair(z):
        z = triangle_multiplication(z, params.tri_mul_out, outgoing=True, mask=pair_mask, eps=eps, residual=z)
        return triangle_multiplication(z, params.tri_mul_in, outgoing=False, mask=pair_mask, eps=eps, residual=z)

    def att_pair(z):
        z = triangle_attention(z, params.tri_att_start, no_heads=no_heads_pair, mask=pair_mask, starting=True,
                               inf=inf, eps=eps, backend="hip", residual=z)
        return triangle_attention(z, params.tri_att_end, no_heads=no_heads_pair, mask=pair_mask, starting=False,
                                  inf=inf, eps=eps, backend="hip", residual=z)

    z = att_pair(mul_pair(z)) if tri_mul_first else mul_pair(att_pair(z))
    return swiglu_transition(z, params.pair_transition, mask=pair_mask if mask_transition else None, eps=eps,
                             residual=z)

