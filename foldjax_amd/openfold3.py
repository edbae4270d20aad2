"""OpenFold3 entry points of the Pairformer path with the reference's call signatures.

Mirrors ``src/foldjax/models/openfold3/models/triangle.py:82``
(``triangle_multiplication``, which has no backend switch upstream),
``triangle_attention.py:95`` (``triangle_attention``),
``primitives.py:133`` (``swiglu_transition``), ``pair_block.py:106``
(``pair_block``), ``attention_pair_bias.py:40`` (``attention_pair_bias``) and
``pairformer.py:42,105`` (``pairformer_block``, ``pairformer_stack``). The attention selector
``OPENFOLD3_TRIANGLE_BACKEND`` / ``backend`` keeps its values {xla, cueq},
case-insensitive (reference ``triangle_attention.py:80,154-157``), and gains
``"hip"``, the default here.
"""

from __future__ import annotations

import os

import torch

from foldjax_amd import kernels
from foldjax_amd.kernels import SingleAttentionWeights, TransitionWeights, TriAttnWeights, TriMulWeights
from foldjax_amd.pairformer import PairformerLayerWeights
from foldjax_amd.params import OpenFold3AttentionPairBiasParams as AttentionPairBiasParams
from foldjax_amd.params import OpenFold3PairBlockParams as PairBlockParams
from foldjax_amd.params import OpenFold3PairformerBlockParams as PairformerBlockParams
from foldjax_amd.params import OpenFold3PairformerStackParams as PairformerStackParams
from foldjax_amd.params import (
    pack_single_attention_openfold3,
    pack_transition_openfold3,
    pack_triattn_openfold3,
    pack_trimul_torch,
)
from foldjax_amd.stacking import StackedLayers, stackable, stacked_or_stack

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


def attention_pair_bias(
    a: torch.Tensor,
    z: torch.Tensor,
    params,
    *,
    no_heads: int,
    mask: torch.Tensor | None = None,
    inf: float = 1e9,
    eps: float = 1e-5,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """OpenFold3 trunk ``attention_pair_bias`` (``OF3/attention_pair_bias.py:40-75``):
    ``a = LN_a(a)``, key mask ``inf (mask - 1)``, pair bias ``LN_z(z) W_z^T``,
    gated attention. Returns the update (as upstream), or ``residual +
    update``."""
    w = params if isinstance(params, SingleAttentionWeights) else pack_single_attention_openfold3(params, a.dtype,
                                                                                                  a.device)
    if w.heads != no_heads:
        raise ValueError(f"no_heads={no_heads} but the pair-bias projection has {w.heads} heads")
    return kernels.single_attention(a, z, mask, w, inf=inf, eps=eps, residual=residual)


def _check_block_heads(block: PairformerLayerWeights, no_heads_pair: int, no_heads_pair_bias: int) -> None:
    for name, w in (("tri_att_start", block.triangle.tri_att_start), ("tri_att_end", block.triangle.tri_att_end)):
        if w.heads != no_heads_pair:
            raise ValueError(f"no_heads_pair={no_heads_pair} but {name} has {w.heads} heads")
    if block.attention.heads != no_heads_pair_bias:
        raise ValueError(f"no_heads_pair_bias={no_heads_pair_bias} but the pair-bias projection has "
                         f"{block.attention.heads} heads")


def pairformer_block(
    s: torch.Tensor,
    z: torch.Tensor,
    params,
    *,
    single_mask: torch.Tensor,
    pair_mask: torch.Tensor,
    no_heads_pair: int,
    no_heads_pair_bias: int,
    inf: float = 1e9,
    mask_transition: bool = True,
    eps: float = 1e-5,
    chunk_size: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """OpenFold3 ``pairformer_block`` (``OF3/pairformer.py:42-102``): z through
    the pair block, then s += attention with pair bias over the updated z
    and s += SwiGLU transition (update times ``single_mask`` when
    ``mask_transition``). ``params`` is a ``PairformerBlockParams`` or a packed
    ``PairformerLayerWeights``. When s and z share a dtype the attention's
    pair bias comes out of the pair transition's epilogue."""
    if chunk_size is not None and chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    return _block_forward(s, z, params, single_mask, pair_mask, no_heads_pair, no_heads_pair_bias, inf,
                          mask_transition, eps, donate=False)


def _block_forward(s, z, params, single_mask, pair_mask, no_heads_pair, no_heads_pair_bias, inf, mask_transition,
                   eps, *, donate):
    block = params if isinstance(params, PairformerLayerWeights) else PairformerLayerWeights.from_openfold3(
        params, z.dtype, z.device, single_dtype=s.dtype)
    _check_block_heads(block, no_heads_pair, no_heads_pair_bias)
    return block.forward_openfold3(s, z, single_mask, pair_mask, inf=inf, mask_transition=mask_transition, eps=eps,
                                   donate=donate)


def can_scan(blocks) -> bool:
    """``OF3/stacking.py:28-46``: two or more blocks of one structure and
    matching weight shapes."""
    blocks = list(blocks)
    return len(blocks) >= 2 and stackable(blocks)


def pairformer_stack(
    s: torch.Tensor,
    z: torch.Tensor,
    params,
    *,
    single_mask: torch.Tensor,
    pair_mask: torch.Tensor,
    no_heads_pair: int,
    no_heads_pair_bias: int,
    inf: float = 1e9,
    mask_transition: bool = True,
    eps: float = 1e-5,
    chunk_size: int | None = None,
    scan_blocks: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """OpenFold3 ``pairformer_stack`` (``OF3/pairformer.py:105-171``): every
    block in order. ``params`` is a ``PairformerStackParams`` or a
    ``StackedLayers`` of packed blocks. Blocks are packed once; with
    ``scan_blocks`` a stackable list runs from one pre-stacked set of weights
    (``_scan_blocks``), otherwise block by block. The kernels are the same."""
    blocks = params if isinstance(params, StackedLayers) else params.blocks
    if not isinstance(blocks, StackedLayers):
        blocks = [b if isinstance(b, PairformerLayerWeights)
                  else PairformerLayerWeights.from_openfold3(b, z.dtype, z.device, single_dtype=s.dtype)
                  for b in blocks]
        if scan_blocks and can_scan(blocks):
            blocks = stacked_or_stack(blocks)
    if chunk_size is not None and chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    # the first block writes new s and z, every later one updates them in
    # place (the reference's scan donates its carry)
    for idx, block in enumerate(blocks):
        s, z = _block_forward(s, z, block, single_mask, pair_mask, no_heads_pair, no_heads_pair_bias, inf,
                              mask_transition, eps, donate=idx > 0)
    return s, z
