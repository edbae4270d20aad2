"""Protenix entry points of the Pairformer path with the reference's call signatures.

Mirrors ``src/foldjax/models/protenix/models/triangle/triangle.py:98``
(``triangle_multiplication``) and ``:456`` (``triangle_attention``),
``primitives/attention.py:108`` (``attention_pair_bias``) and
``trunk_blocks/pairformer.py:49,183,237`` (``pairformer_block``,
``pairformer_stack``, ``stack_pairformer_block_params``). Selectors keep their
names and values and gain ``"hip"``:

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
from foldjax_amd.kernels import SingleAttentionWeights, TransitionWeights, TriAttnWeights, TriMulWeights
from foldjax_amd.pairformer import PairformerLayerWeights
from foldjax_amd.params import ProtenixAttentionPairBiasParams as AttentionPairBiasParams
from foldjax_amd.params import ProtenixPairformerBlockParams as PairformerBlockParams
from foldjax_amd.params import ProtenixPairformerStackParams as PairformerStackParams
from foldjax_amd.params import (
    pack_single_attention_protenix,
    pack_transition_torch,
    pack_triattn_protenix,
    pack_trimul_torch,
)
from foldjax_amd.stacking import StackedLayers, stacked_or_stack

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


# the single attention's backends of ``PXP/attention.py:60-99,361-424``; they
# choose among JAX implementations of one function, which here is one HIP path
_SINGLE_BACKENDS = {"xla", "xla_jit", "xla_sdpa", "cudnn", "hip"}


def _single_backend(name: str) -> None:
    if name not in _SINGLE_BACKENDS:
        raise ValueError(f"unsupported attention backend: {name!r}")


def attention_pair_bias(
    a: torch.Tensor,
    s: torch.Tensor | None,
    z: torch.Tensor,
    params,
    *,
    num_heads: int,
    q_chunk_size: int | None = None,
    attention_backend: str = "xla",
    z_is_normalized: bool = False,
    extra_attn_bias: torch.Tensor | None = None,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Protenix ``attention_pair_bias`` (``PXP/attention.py:108-169``) in the
    trunk form the Pairformer uses: ``q_x = LN_a(a)``, ``bias = LN_z(z) W_z^T``
    plus ``extra_attn_bias`` (``[..., N, N]`` or ``[..., H, N, N]``, aligned as
    :140-150), gated attention over ``q_x``. Returns the update, or
    ``residual + update``. ``q_chunk_size`` is accepted and unused (the
    kernel streams keys). The diffusion forms (``has_s``, cross attention,
    ``z_is_normalized``) are not on this path and raise ``ValueError``."""
    _single_backend(attention_backend)
    if z_is_normalized:
        raise ValueError("z_is_normalized=True is the diffusion conditioning form; the hip path takes the trunk form")
    w = params if isinstance(params, SingleAttentionWeights) else pack_single_attention_protenix(params, a.dtype,
                                                                                                 a.device)
    if w.heads != num_heads:
        raise ValueError(f"num_heads={num_heads} but the pair-bias projection has {w.heads} heads")
    extra = None
    if extra_attn_bias is not None:
        n = int(a.shape[-2])
        if tuple(extra_attn_bias.shape[-2:]) != (n, n):
            raise ValueError("extra attention bias pair axes must match projected pair bias: "
                             f"{tuple(extra_attn_bias.shape[-2:])} != {(n, n)}")
        bias_ndim = a.dim() + 1  # [..., H, N, N]
        extra = extra_attn_bias
        while extra.dim() < bias_ndim - 1:
            extra = extra.unsqueeze(0)
        if extra.dim() == bias_ndim - 1:
            extra = extra.unsqueeze(-3)
        if a.dim() == 2:
            extra = extra.unsqueeze(0)
    return kernels.single_attention(a, z, None, w, eps=1e-5, residual=residual, extra_bias=extra)


def pairformer_block(
    s: torch.Tensor | None,
    z: torch.Tensor,
    pair_mask: torch.Tensor | None,
    params,
    *,
    triangle_mul_chunk_size: int | None = None,
    triangle_att_q_chunk_size: int | None = None,
    single_att_q_chunk_size: int | None = None,
    single_attention_backend: str = "xla",
    triangle_attention_backend: str | None = None,
) -> tuple[torch.Tensor | None, torch.Tensor]:
    """Protenix ``pairformer_block`` (``PXK/pairformer.py:49-180``): z through
    tri-mul out and in, tri-attn start and end, pair transition, each output
    multiplied by ``bool(pair_mask)`` inside its kernel; then s += attention
    with pair bias (keys masked by the pair mask's diagonal) and s += single
    transition, each gated by that diagonal. ``params`` is a
    ``PairformerBlockParams`` (fields the reference's containers or packed
    weights) or a packed ``PairformerLayerWeights``. Chunk sizes are accepted
    and unused; the backend selectors are validated as upstream."""
    _check_block_selectors(single_attention_backend, triangle_attention_backend)
    return _packed_block(params, s, z).forward_protenix(s, z, pair_mask)


def _check_block_selectors(single_attention_backend: str, triangle_attention_backend: str | None) -> None:
    _single_backend(single_attention_backend)
    backend = _triangle_attention_backend() if triangle_attention_backend is None else triangle_attention_backend
    if backend not in {"xla", "xla_jit", "tokamax", "cueq", "cueq_jit", "hip", "hip_jit"}:
        raise ValueError(f"unsupported triangle attention backend: {backend!r}")
    if backend.removesuffix("_jit") != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle attention", name=backend))
    mul = os.environ.get("PROTENIX_TRIANGLE_MULTIPLICATION_BACKEND", DEFAULT_BACKEND).lower()
    if mul not in {"cueq", "xla", "hip"}:
        raise ValueError(f"unsupported triangle multiplication backend: {mul!r}")
    if mul != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle multiplication", name=mul))


def _packed_block(params, s: torch.Tensor | None, z: torch.Tensor) -> PairformerLayerWeights:
    sd = s.dtype if s is not None else z.dtype
    return params if isinstance(params, PairformerLayerWeights) else PairformerLayerWeights.from_protenix(
        params, z.dtype, z.device, single_dtype=sd)


def stack_pairformer_block_params(blocks, dtype: torch.dtype | None = None, device=None) -> StackedLayers:
    """``PXK/pairformer.py:237-245``: the blocks' weights on a leading layer
    axis, packed once (``dtype``/``device`` for blocks given as the
    reference's containers; packed blocks keep theirs)."""
    if not blocks:
        raise ValueError("stack_pairformer_block_params requires at least one block")
    if isinstance(blocks, StackedLayers):
        return blocks
    packed = [b if isinstance(b, PairformerLayerWeights) else PairformerLayerWeights.from_protenix(b, dtype, device)
              for b in blocks]
    return stacked_or_stack(packed)


def pairformer_stack(
    s: torch.Tensor | None,
    z: torch.Tensor,
    pair_mask: torch.Tensor | None,
    params,
    *,
    use_scan: bool = True,
    triangle_mul_chunk_size: int | None = None,
    triangle_att_q_chunk_size: int | None = None,
    single_att_q_chunk_size: int | None = None,
    single_attention_backend: str = "xla",
    triangle_attention_backend: str | None = None,
) -> tuple[torch.Tensor | None, torch.Tensor]:
    """Protenix ``pairformer_stack`` (``PXK/pairformer.py:183-234``): the
    blocks in order. ``params`` is a ``PairformerStackParams`` or a
    ``StackedLayers`` of packed blocks. With ``use_scan`` the blocks are
    stacked once (``stack_pairformer_block_params``) and run from the stacked
    weights; either way every block is the same chain of kernel launches."""
    blocks = params if isinstance(params, StackedLayers) else params.blocks
    if not blocks:
        raise ValueError("PairformerStack requires at least one block")
    sd = s.dtype if s is not None else z.dtype
    if use_scan and not isinstance(blocks, StackedLayers):
        blocks = stacked_or_stack([b if isinstance(b, PairformerLayerWeights)
                                   else PairformerLayerWeights.from_protenix(b, z.dtype, z.device, single_dtype=sd)
                                   for b in blocks])
    _check_block_selectors(single_attention_backend, triangle_attention_backend)
    # the first block writes new s and z, every later one updates them in
    # place (the reference's scan donates its carry)
    for idx, block in enumerate(blocks):
        s, z = _packed_block(block, s, z).forward_protenix(s, z, pair_mask, donate=idx > 0)
    return s, z
