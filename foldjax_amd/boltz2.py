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
from foldjax_amd.kernels import SingleAttentionWeights, TransitionWeights, TriAttnWeights, TriMulWeights
from foldjax_amd.params import (
    pack_single_attention_boltz2,
    pack_transition_boltz2,
    pack_triattn_boltz2,
    pack_trimul_boltz2,
)

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


def transition_forward(
    params,
    x: torch.Tensor,
    chunk_size: int | None = None,
    eps: float = 1e-5,
    row_chunk_size: int | None = None,
    glu_backend: str = "xla",
    *,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Boltz-2 ``transition_forward`` (``B2P/transition.py:39-122``): the fused
    kernel never forms the widened hidden tensor, so both chunk sizes are
    accepted and unused (a non-positive ``chunk_size`` still raises, as there)."""
    if chunk_size is not None and chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    if glu_backend not in ("xla", "tokamax"):
        raise ValueError(f"Unsupported glu backend: {glu_backend!r}")
    w = params if isinstance(params, TransitionWeights) else pack_transition_boltz2(params, x.dtype, x.device)
    return kernels.transition(x, w, residual=residual, eps=eps)


def attention_pair_bias_forward(
    params,
    s: torch.Tensor,
    z: torch.Tensor,
    mask: torch.Tensor,
    k_in: torch.Tensor | None = None,
    multiplicity: int = 1,
    inf: float = 1e6,
    eps: float = 1e-5,
    chunk_size: int | None = None,
    attention_backend: str = "xla",
    *,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """Boltz-2 ``attention_pair_bias_forward`` (``B2P/attention.py:19-115``) in
    the self-attention form the Pairformer layer uses (``k_in`` is ``s``).
    ``s`` is the normalised single representation; returns the update."""
    if k_in is not None and k_in is not s:
        raise ValueError("the hip attention with pair bias supports k_in=None or k_in=s only")
    if multiplicity != 1:
        raise ValueError("the hip attention with pair bias supports multiplicity=1 only")
    if attention_backend not in ("xla", "tokamax", "flash", "hip"):
        raise ValueError(f"Unsupported attention backend: {attention_backend!r}")
    w = params if isinstance(params, SingleAttentionWeights) else pack_single_attention_boltz2(params, s.dtype, s.device)
    return kernels.single_attention(s, z, mask, w, inf=inf, eps=eps, residual=residual)


def pairformer_layer_forward(
    params,
    s: torch.Tensor,
    z: torch.Tensor,
    mask: torch.Tensor,
    pair_mask: torch.Tensor,
    eps: float = 1e-5,
    chunk_size: int = 128,
    triangle_attention_chunk: int | None = None,
    triangle_attention_q_chunk: int | None = None,
    transition_hidden_chunk: int | None = None,
    matmul_precision: str = "highest",
    attention_backend: str = "xla",
    triangle_backend: str = DEFAULT_BACKEND,
    glu_backend: str = "xla",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Boltz-2 ``pairformer_layer_forward`` (``B2K/pairformer.py:100-206``):
    every residual is fused into the producing kernel. ``params`` is the
    Boltz-2 layer dict, or a ``foldjax_amd.pairformer.PairformerLayerWeights``."""
    w = _packed_layer(params, s, z)
    _check_layer_selectors(matmul_precision, triangle_backend)
    return w.forward(s, z, mask, pair_mask, eps=eps)


def _packed_layer(params, s: torch.Tensor, z: torch.Tensor):
    from foldjax_amd.pairformer import PairformerLayerWeights

    return params if isinstance(params, PairformerLayerWeights) else PairformerLayerWeights.from_boltz2(
        params, z.dtype, z.device, single_dtype=s.dtype)


def _check_layer_selectors(matmul_precision: str, triangle_backend: str) -> None:
    """Selector validation as the reference's layer entry point does it."""
    resolve_matmul_precision(matmul_precision)
    if triangle_backend not in ("xla", "pallas", "tokamax", "cueq", "hip"):
        raise ValueError(f"Unsupported triangle_backend: {triangle_backend!r}")
    if triangle_backend != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle attention", name=triangle_backend))


def pairformer_no_seq_layer_forward(
    params,
    z: torch.Tensor,
    pair_mask: torch.Tensor,
    eps: float = 1e-5,
    chunk_size: int = 128,
    triangle_attention_chunk: int | None = None,
    triangle_attention_q_chunk: int | None = None,
    transition_hidden_chunk: int | None = None,
    matmul_precision: str = "highest",
    triangle_backend: str = DEFAULT_BACKEND,
    glu_backend: str = "xla",
) -> torch.Tensor:
    """Boltz-2 ``pairformer_no_seq_layer_forward`` (``B2K/msa.py:467-539``),
    the MSA module's pair block: z += tri-mul outgoing, incoming, tri-attn
    starting, ending (all with ``pair_mask``) and the unmasked pair
    transition, each residual fused into its kernel. ``params`` is the
    Boltz-2 dict with ``tri_mul_out``, ``tri_mul_in``, ``tri_att_start``,
    ``tri_att_end`` and ``transition_z``; the chunk arguments are accepted for
    signature parity (the kernels stream with a fixed workspace)."""
    from foldjax_amd.pairformer import TriangleSublayers

    resolve_matmul_precision(matmul_precision)
    if triangle_backend not in ("xla", "pallas", "tokamax", "cueq", "hip"):
        raise ValueError(f"Unsupported triangle_backend: {triangle_backend!r}")
    if triangle_backend != "hip":
        raise RuntimeError(_REFERENCE_ONLY.format(kind="triangle attention", name=triangle_backend))
    dt, dev = z.dtype, z.device
    tri = TriangleSublayers(
        pack_trimul_boltz2(params["tri_mul_out"], dt, dev),
        pack_trimul_boltz2(params["tri_mul_in"], dt, dev),
        pack_triattn_boltz2(params["tri_att_start"], dt, dev),
        pack_triattn_boltz2(params["tri_att_end"], dt, dev),
    )
    z = tri.forward(z, pair_mask)  # a new tensor, updated in place from here on
    return kernels.transition(z, pack_transition_boltz2(params["transition_z"], dt, dev), residual=z, eps=eps,
                              out=z)


def stack_layer_params(layer_list, dtype: torch.dtype | None = None, device=None, single_dtype=None):
    """``B2P/_scan_utils.py:18-27``: the layers' weights on a leading layer
    axis (``foldjax_amd.stacking.StackedLayers``), packed once. Layers given
    as Boltz-2 dicts are packed in ``dtype`` on ``device`` (the single track
    in ``single_dtype``, default ``dtype``)."""
    from foldjax_amd.pairformer import PairformerLayerWeights
    from foldjax_amd.stacking import StackedLayers, stacked_or_stack

    if not layer_list:
        raise ValueError("stack_layer_params requires at least one layer")
    if isinstance(layer_list, StackedLayers):
        return layer_list
    return stacked_or_stack([
        lay if isinstance(lay, PairformerLayerWeights)
        else PairformerLayerWeights.from_boltz2(lay, dtype, device, single_dtype=single_dtype)
        for lay in layer_list
    ])


def pairformer_module_forward(
    params,
    s: torch.Tensor,
    z: torch.Tensor,
    mask: torch.Tensor,
    pair_mask: torch.Tensor,
    eps: float = 1e-5,
    use_scan: bool = True,
    chunk_size: int = 128,
    triangle_attention_chunk: int | None = None,
    triangle_attention_q_chunk: int | None = None,
    transition_hidden_chunk: int | None = None,
    matmul_precision: str = "highest",
    attention_backend: str = "xla",
    triangle_backend: str = DEFAULT_BACKEND,
    glu_backend: str = "xla",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Boltz-2 ``pairformer_module_forward`` (``B2K/pairformer.py:30-97``):
    the layers of ``params["layers"]`` applied in order, each one
    ``pairformer_layer_forward``. A layer entry is the Boltz-2 layer dict or a
    pre-packed ``PairformerLayerWeights``; ``params["layers"]`` may also be a
    ``StackedLayers`` (``stack_layer_params``). With ``use_scan`` the layers
    are packed and stacked once, as the reference stacks them for its scan;
    without it each layer is used as given. The chunk arguments are accepted
    for signature parity: the reference uses them to bound XLA's memory,
    while every layer here streams through fused kernels with a fixed
    workspace. As the reference's scan donates its carry
    (``B2K/pairformer.py:74-96``), the first layer writes new s and z and
    every later layer updates those in place."""
    layers = params["layers"]
    if use_scan:
        layers = stack_layer_params(layers, z.dtype, z.device, single_dtype=s.dtype)
    _check_layer_selectors(matmul_precision, triangle_backend)
    for idx, layer in enumerate(layers):
        s, z = _packed_layer(layer, s, z).forward(s, z, mask, pair_mask, eps=eps, donate=idx > 0)
    return s, z
