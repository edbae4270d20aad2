"""Parameter containers of the three ports and their packing into ABI weights.

The containers mirror the reference's own types so that mapped checkpoints
drop in unchanged:

* Boltz-2 uses nested dicts with ``[in, out]`` kernels
  (``src/foldjax/models/boltz2/bridge/torch_mapping.py:513-600``).
* Protenix uses NamedTuples with PyTorch ``[out, in]`` weights
  (``src/foldjax/models/protenix/models/primitives/primitives.py:11-28``,
  ``.../triangle/triangle.py:77-95``, ``.../primitives/attention.py:21-29``).
* OpenFold3 uses its own NamedTuples (``src/foldjax/models/openfold3/models/
  triangle.py:40-54``, ``triangle_attention.py:83-92``, ``attention.py``).

Every triangle projection is bias-free upstream; a container carrying a
projection bias is rejected rather than silently ignored.
"""

from __future__ import annotations

from typing import Any, NamedTuple

import numpy as np
import torch

from foldjax_amd.kernels import SingleAttentionWeights, TransitionWeights, TriAttnWeights, TriMulWeights


class LinearParams(NamedTuple):
    """PyTorch-layout linear: ``weight [out, in]``, optional ``bias [out]``."""

    weight: Any
    bias: Any = None


class LayerNormParams(NamedTuple):
    weight: Any = None
    bias: Any = None


class AttentionParams(NamedTuple):
    """Protenix/OpenFold3 ``Attention`` projections."""

    linear_q: LinearParams
    linear_k: LinearParams
    linear_v: LinearParams
    linear_o: LinearParams
    linear_g: LinearParams | None


class ProtenixTriangleMultiplicationParams(NamedTuple):
    layer_norm_in: LayerNormParams
    layer_norm_out: LayerNormParams
    linear_a_p: LinearParams
    linear_a_g: LinearParams
    linear_b_p: LinearParams
    linear_b_g: LinearParams
    linear_z: LinearParams
    linear_g: LinearParams


class ProtenixTriangleAttentionParams(NamedTuple):
    layer_norm: LayerNormParams
    linear: LinearParams
    attention: AttentionParams


class OpenFold3TriangleMultiplicationParams(NamedTuple):
    layer_norm_in: LayerNormParams
    layer_norm_out: LayerNormParams
    linear_a_p: LinearParams
    linear_a_g: LinearParams
    linear_b_p: LinearParams
    linear_b_g: LinearParams
    linear_g: LinearParams
    linear_z: LinearParams


class OpenFold3TriangleAttentionParams(NamedTuple):
    layer_norm: LayerNormParams
    linear_z: LinearParams
    mha: AttentionParams


class OpenFold3PairBlockParams(NamedTuple):
    """OpenFold3 ``PairBlockParams`` (``OF3/pair_block.py:35-46``): the
    AF3 SwiGLU / non-fused layout. Each field is that sublayer's parameter
    container (or a pre-packed weight object of ``foldjax_amd.kernels``)."""

    tri_mul_out: object
    tri_mul_in: object
    tri_att_start: object
    tri_att_end: object
    pair_transition: object


class ProtenixAttentionPairBiasParams(NamedTuple):
    """Protenix ``AttentionPairBiasParams`` (``PXP/attention.py:32-41``)."""

    layernorm_a: Any
    layernorm_kv: Any
    attention: AttentionParams
    layernorm_z: LayerNormParams
    linear_z: LinearParams
    linear_a_last: Any = None
    has_s: bool = False
    cross_attention_mode: bool = False


class ProtenixTransitionParams(NamedTuple):
    """Protenix ``TransitionParams`` (``PXP/primitives.py:30-36``)."""

    layer_norm: LayerNormParams
    linear_a: LinearParams
    linear_b: LinearParams
    linear_out: LinearParams


class ProtenixPairformerBlockParams(NamedTuple):
    """Protenix ``PairformerBlockParams`` (``PXK/pairformer.py:31-41``). Each
    field is the reference's container or a pre-packed weight object of
    ``foldjax_amd.kernels``."""

    tri_mul_out: Any
    tri_mul_in: Any
    tri_att_start: Any
    tri_att_end: Any
    pair_transition: Any
    attention_pair_bias: Any = None
    single_transition: Any = None


class ProtenixPairformerStackParams(NamedTuple):
    """Protenix ``PairformerStackParams`` (``PXK/pairformer.py:44-47``)."""

    blocks: tuple


class OpenFold3AttentionPairBiasParams(NamedTuple):
    """OpenFold3 trunk ``AttentionPairBiasParams`` (``OF3/attention_pair_bias.py:30-37``)."""

    layer_norm_a: LayerNormParams
    layer_norm_z: LayerNormParams
    linear_z: LinearParams
    mha: AttentionParams


class OpenFold3PairformerBlockParams(NamedTuple):
    """OpenFold3 ``PairformerBlockParams`` (``OF3/pairformer.py:27-33``)."""

    pair_stack: Any
    attn_pair_bias: Any
    single_transition: Any


class OpenFold3PairformerStackParams(NamedTuple):
    """OpenFold3 ``PairformerStackParams`` (``OF3/pairformer.py:36-39``)."""

    blocks: tuple


def _t(x) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x
    return torch.as_tensor(np.asarray(x))


def _get(obj, name):
    if isinstance(obj, dict):
        return obj.get(name)
    return getattr(obj, name, None)


def _weight(lin, what: str) -> torch.Tensor:
    if lin is None:
        raise ValueError(f"missing linear {what}")
    if _get(lin, "bias") is not None:
        raise ValueError(f"{what} carries a bias; the triangle projections are bias-free")
    return _t(_get(lin, "weight"))


def _ln(p, c: int):
    w = _get(p, "weight") if p is not None else None
    b = _get(p, "bias") if p is not None else None
    w = torch.ones(c) if w is None else _t(w)
    b = torch.zeros(c) if b is None else _t(b)
    return w, b


# ----------------------------------------------------------------- tri-mul


def pack_trimul_boltz2(params, dtype: torch.dtype, device) -> TriMulWeights:
    """Boltz-2 dict (kernels ``[in, out]``) -> ABI weights: every projection is
    transposed, as the reference's cuEquivariance adapter does
    (``B2T/triangle_cueq.py:92-99``)."""
    k = lambda name: _t(params[name]["kernel"]).T  # noqa: E731
    w = TriMulWeights(
        norm_in_weight=_t(params["norm_in"]["scale"]),
        norm_in_bias=_t(params["norm_in"]["bias"]),
        p_in_weight=k("p_in"),
        g_in_weight=k("g_in"),
        norm_out_weight=_t(params["norm_out"]["scale"]),
        norm_out_bias=_t(params["norm_out"]["bias"]),
        p_out_weight=k("p_out"),
        g_out_weight=k("g_out"),
    )
    return w.to(dtype, device)


def pack_trimul_torch(params, dtype: torch.dtype, device) -> TriMulWeights:
    """Protenix/OpenFold3 tri-mul fields -> ABI weights: a and b projections
    are stacked a-first, as ``PXT/triangle_cueq.py:28-47`` does for cuEq."""
    a_p = _weight(_get(params, "linear_a_p"), "linear_a_p")
    c_h, c_z = a_p.shape
    ln_in = _ln(_get(params, "layer_norm_in"), c_z)
    ln_out = _ln(_get(params, "layer_norm_out"), c_h)
    w = TriMulWeights(
        norm_in_weight=ln_in[0],
        norm_in_bias=ln_in[1],
        p_in_weight=torch.cat([a_p, _weight(_get(params, "linear_b_p"), "linear_b_p")], 0),
        g_in_weight=torch.cat(
            [_weight(_get(params, "linear_a_g"), "linear_a_g"), _weight(_get(params, "linear_b_g"), "linear_b_g")], 0
        ),
        norm_out_weight=ln_out[0],
        norm_out_bias=ln_out[1],
        p_out_weight=_weight(_get(params, "linear_z"), "linear_z"),
        g_out_weight=_weight(_get(params, "linear_g"), "linear_g"),
    )
    return w.to(dtype, device)


# ---------------------------------------------------------------- tri-attn


def pack_triattn_boltz2(params, dtype: torch.dtype, device) -> TriAttnWeights:
    """Boltz-2 tri-attn dict -> ABI weights (all kernels transposed)."""
    mha = params["mha"]
    k = lambda p: _t(p["kernel"]).T  # noqa: E731
    w = TriAttnWeights(
        norm_weight=_t(params["layer_norm"]["scale"]),
        norm_bias=_t(params["layer_norm"]["bias"]),
        bias_weight=k(params["linear"]),
        q_weight=k(mha["linear_q"]),
        k_weight=k(mha["linear_k"]),
        v_weight=k(mha["linear_v"]),
        g_weight=k(mha["linear_g"]),
        o_weight=k(mha["linear_o"]),
    )
    return w.to(dtype, device)


def _pack_triattn_torch(ln, bias_lin, att, dtype, device) -> TriAttnWeights:
    q = _weight(_get(att, "linear_q"), "linear_q")
    c_z = q.shape[1]
    lw, lb = _ln(ln, c_z)
    g = _get(att, "linear_g")
    w = TriAttnWeights(
        norm_weight=lw,
        norm_bias=lb,
        bias_weight=_weight(bias_lin, "triangle bias linear"),
        q_weight=q,
        k_weight=_weight(_get(att, "linear_k"), "linear_k"),
        v_weight=_weight(_get(att, "linear_v"), "linear_v"),
        g_weight=None if g is None else _weight(g, "linear_g"),
        o_weight=_weight(_get(att, "linear_o"), "linear_o"),
    )
    return w.to(dtype, device)


def pack_triattn_protenix(params, dtype: torch.dtype, device) -> TriAttnWeights:
    """Protenix ``TriangleAttentionParams(layer_norm, linear, attention)``."""
    return _pack_triattn_torch(_get(params, "layer_norm"), _get(params, "linear"), _get(params, "attention"), dtype, device)


def pack_triattn_openfold3(params, dtype: torch.dtype, device) -> TriAttnWeights:
    """OpenFold3 ``TriangleAttentionParams(layer_norm, linear_z, mha)``."""
    return _pack_triattn_torch(_get(params, "layer_norm"), _get(params, "linear_z"), _get(params, "mha"), dtype, device)


# ------------------------------------------------ synthetic-weight adapters


def _lin(d):
    return LinearParams(weight=d["weight"], bias=d.get("bias"))


def _lnp(d):
    return LayerNormParams(weight=d.get("weight"), bias=d.get("bias"))


def trimul_to_protenix(w: dict) -> ProtenixTriangleMultiplicationParams:
    """Field dict (``foldjax_amd.synthetic.trimul_weights``) -> Protenix container."""
    return ProtenixTriangleMultiplicationParams(
        layer_norm_in=_lnp(w["layer_norm_in"]), layer_norm_out=_lnp(w["layer_norm_out"]),
        linear_a_p=_lin(w["linear_a_p"]), linear_a_g=_lin(w["linear_a_g"]),
        linear_b_p=_lin(w["linear_b_p"]), linear_b_g=_lin(w["linear_b_g"]),
        linear_z=_lin(w["linear_z"]), linear_g=_lin(w["linear_g"]),
    )


def trimul_to_openfold3(w: dict) -> OpenFold3TriangleMultiplicationParams:
    return OpenFold3TriangleMultiplicationParams(
        layer_norm_in=_lnp(w["layer_norm_in"]), layer_norm_out=_lnp(w["layer_norm_out"]),
        linear_a_p=_lin(w["linear_a_p"]), linear_a_g=_lin(w["linear_a_g"]),
        linear_b_p=_lin(w["linear_b_p"]), linear_b_g=_lin(w["linear_b_g"]),
        linear_g=_lin(w["linear_g"]), linear_z=_lin(w["linear_z"]),
    )


def trimul_to_boltz2(w: dict) -> dict:
    """Field dict -> Boltz-2 dict (``p_in``/``g_in`` ``[c_z, 2c_h]``, a first)."""
    cat = lambda a, b: np.concatenate([np.asarray(w[a]["weight"]), np.asarray(w[b]["weight"])], 0).T  # noqa: E731
    return {
        "norm_in": {"scale": w["layer_norm_in"]["weight"], "bias": w["layer_norm_in"]["bias"]},
        "p_in": {"kernel": cat("linear_a_p", "linear_b_p")},
        "g_in": {"kernel": cat("linear_a_g", "linear_b_g")},
        "norm_out": {"scale": w["layer_norm_out"]["weight"], "bias": w["layer_norm_out"]["bias"]},
        "p_out": {"kernel": np.asarray(w["linear_z"]["weight"]).T},
        "g_out": {"kernel": np.asarray(w["linear_g"]["weight"]).T},
    }


def _attn(d) -> AttentionParams:
    g = d.get("linear_g")
    return AttentionParams(
        linear_q=_lin(d["linear_q"]), linear_k=_lin(d["linear_k"]), linear_v=_lin(d["linear_v"]),
        linear_o=_lin(d["linear_o"]), linear_g=None if g is None else _lin(g),
    )


def triattn_to_protenix(w: dict) -> ProtenixTriangleAttentionParams:
    """Field dict (``foldjax_amd.synthetic.triattn_weights``) -> Protenix container."""
    return ProtenixTriangleAttentionParams(
        layer_norm=_lnp(w["layer_norm"]), linear=_lin(w["linear"]), attention=_attn(w["attention"])
    )


def triattn_to_openfold3(w: dict) -> OpenFold3TriangleAttentionParams:
    return OpenFold3TriangleAttentionParams(
        layer_norm=_lnp(w["layer_norm"]), linear_z=_lin(w["linear"]), mha=_attn(w["attention"])
    )


def triattn_to_boltz2(w: dict) -> dict:
    att = w["attention"]
    return {
        "layer_norm": {"scale": w["layer_norm"]["weight"], "bias": w["layer_norm"]["bias"]},
        "linear": {"kernel": np.asarray(w["linear"]["weight"]).T},
        "mha": {n: {"kernel": np.asarray(att[n]["weight"]).T} for n in ("linear_q", "linear_k", "linear_v", "linear_o", "linear_g")},
    }


# -------------------------------------------------------------- transition


def pack_transition_torch(params, dtype: torch.dtype, device) -> TransitionWeights:
    """Protenix ``TransitionParams(layer_norm, linear_a, linear_b, linear_out)``
    (``PXP/primitives.py:30-36``); ``linear_a`` is the silu branch."""
    a = _weight(_get(params, "linear_a"), "linear_a")
    lw, lb = _ln(_get(params, "layer_norm"), a.shape[1])
    w = TransitionWeights(
        norm_weight=lw, norm_bias=lb, w_a=a,
        w_b=_weight(_get(params, "linear_b"), "linear_b"),
        w_o=_weight(_get(params, "linear_out"), "linear_out"),
    )
    return w.to(dtype, device)


def pack_transition_openfold3(params, dtype: torch.dtype, device) -> TransitionWeights:
    """OpenFold3 ``SwiGLUTransitionParams(layer_norm, swiglu, linear_out)``
    (``OF3/primitives.py:67-72``)."""
    sw = _get(params, "swiglu")
    a = _weight(_get(sw, "linear_a"), "swiglu.linear_a")
    lw, lb = _ln(_get(params, "layer_norm"), a.shape[1])
    w = TransitionWeights(
        norm_weight=lw, norm_bias=lb, w_a=a,
        w_b=_weight(_get(sw, "linear_b"), "swiglu.linear_b"),
        w_o=_weight(_get(params, "linear_out"), "linear_out"),
    )
    return w.to(dtype, device)


def pack_transition_boltz2(params, dtype: torch.dtype, device) -> TransitionWeights:
    """Boltz-2 ``{norm, fc1, fc2, fc3}`` with ``[in, out]`` kernels
    (``M/boltz2/bridge/torch_mapping.py:63-71``)."""
    k = lambda name: _t(params[name]["kernel"]).T  # noqa: E731
    w = TransitionWeights(
        norm_weight=_t(params["norm"]["scale"]), norm_bias=_t(params["norm"]["bias"]),
        w_a=k("fc1"), w_b=k("fc2"), w_o=k("fc3"),
    )
    return w.to(dtype, device)


def pack_single_attention_boltz2(params, dtype: torch.dtype, device, pre_norm=None) -> SingleAttentionWeights:
    """Boltz-2 ``AttentionPairBias`` dict (``M/boltz2/bridge/torch_mapping.py:
    74-113``, kernels ``[in, out]``) plus an optional ``pre_norm_s`` dict."""
    k = lambda name: _t(params[name]["kernel"]).T  # noqa: E731
    qb = params["proj_q"].get("bias")
    w = SingleAttentionWeights(
        pre_norm_weight=None if pre_norm is None else _t(pre_norm["scale"]),
        pre_norm_bias=None if pre_norm is None else _t(pre_norm["bias"]),
        z_norm_weight=_t(params["proj_z_norm"]["scale"]),
        z_norm_bias=_t(params["proj_z_norm"]["bias"]),
        z_weight=k("proj_z"),
        q_weight=k("proj_q"),
        q_bias=None if qb is None else _t(qb),
        k_weight=k("proj_k"), v_weight=k("proj_v"), g_weight=k("proj_g"), o_weight=k("proj_o"),
    )
    return w.to(dtype, device)


def transition_to_boltz2(w: dict) -> dict:
    """Field dict (``foldjax_amd.synthetic.transition_weights``) -> Boltz-2 dict."""
    return {
        "norm": {"scale": w["layer_norm"]["weight"], "bias": w["layer_norm"]["bias"]},
        "fc1": {"kernel": np.asarray(w["linear_a"]["weight"]).T},
        "fc2": {"kernel": np.asarray(w["linear_b"]["weight"]).T},
        "fc3": {"kernel": np.asarray(w["linear_out"]["weight"]).T},
    }


def single_attention_to_boltz2(w: dict) -> tuple[dict, dict]:
    """Torch-layout dict (``foldjax_amd.synthetic.single_attention_weights``) ->
    (Boltz-2 ``attention`` dict, ``pre_norm_s`` dict)."""
    k = lambda name: {"kernel": np.asarray(w[name]["weight"]).T}  # noqa: E731
    att = {
        "proj_q": {"kernel": np.asarray(w["proj_q"]["weight"]).T, "bias": w["proj_q"]["bias"]},
        "proj_k": k("proj_k"), "proj_v": k("proj_v"), "proj_g": k("proj_g"), "proj_o": k("proj_o"),
        "proj_z_norm": {"scale": w["proj_z_norm"]["weight"], "bias": w["proj_z_norm"]["bias"]},
        "proj_z": k("proj_z"),
    }
    pre = {"scale": w["pre_norm_s"]["weight"], "bias": w["pre_norm_s"]["bias"]}
    return att, pre


def pairformer_layer_to_boltz2(w: dict) -> dict:
    """Field dicts of one layer -> Boltz-2 ``PairformerLayerParams`` dict
    (``M/boltz2/bridge/torch_mapping.py:603-650`` key names)."""
    att, pre = single_attention_to_boltz2(w["attention"])
    return {
        "tri_mul_out": trimul_to_boltz2(w["tri_mul_out"]),
        "tri_mul_in": trimul_to_boltz2(w["tri_mul_in"]),
        "tri_att_start": triattn_to_boltz2(w["tri_att_start"]),
        "tri_att_end": triattn_to_boltz2(w["tri_att_end"]),
        "transition_z": transition_to_boltz2(w["transition_z"]),
        "pre_norm_s": pre,
        "attention": att,
        "transition_s": transition_to_boltz2(w["transition_s"]),
    }


# --------------------------------------- single attention, Protenix / OpenFold3


def _pack_single_attention_torch(ln_a, att, ln_z, lin_z, dtype, device) -> SingleAttentionWeights:
    """The gated attention with pair bias of the Protenix and OpenFold3 trunks:
    ``linear_q`` may carry a bias (both ports map it so,
    ``M/protenix/bridge/torch_mapping.py:175-198``,
    ``M/openfold3/bridge/torch_mapping.py:153-177``); every other projection is
    bias-free. A LayerNorm without weight or bias packs ones or zeros."""
    if att is None:
        raise ValueError("missing attention parameters")
    if ln_a is None:
        raise ValueError("missing attention pair-bias normalization params")
    if _get(att, "linear_g") is None:
        raise ValueError("the hip attention with pair bias needs a gated attention (linear_g)")
    lq = _get(att, "linear_q")
    q = _t(_get(lq, "weight"))
    c_s = q.shape[1]
    qb = _get(lq, "bias")
    z_w = _weight(lin_z, "linear_z")
    pw, pb = _ln(ln_a, c_s)
    zw, zb = _ln(ln_z, z_w.shape[1])
    w = SingleAttentionWeights(
        pre_norm_weight=pw, pre_norm_bias=pb, z_norm_weight=zw, z_norm_bias=zb, z_weight=z_w,
        q_weight=q, q_bias=None if qb is None else _t(qb),
        k_weight=_weight(_get(att, "linear_k"), "linear_k"), v_weight=_weight(_get(att, "linear_v"), "linear_v"),
        g_weight=_weight(_get(att, "linear_g"), "linear_g"), o_weight=_weight(_get(att, "linear_o"), "linear_o"),
    )
    return w.to(dtype, device)


def pack_single_attention_protenix(params, dtype: torch.dtype, device) -> SingleAttentionWeights:
    """Protenix ``AttentionPairBiasParams`` in its trunk form (``has_s=False``,
    no cross attention, ``PXK/pairformer.py:150-154``): ``layernorm_a`` is the
    attention's own pre-norm, ``linear_z`` the pair-bias projection."""
    if _get(params, "has_s") or _get(params, "cross_attention_mode"):
        raise ValueError("the hip attention with pair bias supports the trunk form "
                         "(has_s=False, cross_attention_mode=False)")
    return _pack_single_attention_torch(_get(params, "layernorm_a"), _get(params, "attention"),
                                        _get(params, "layernorm_z"), _get(params, "linear_z"), dtype, device)


def pack_single_attention_openfold3(params, dtype: torch.dtype, device) -> SingleAttentionWeights:
    """OpenFold3 trunk ``AttentionPairBiasParams(layer_norm_a, layer_norm_z,
    linear_z, mha)``."""
    return _pack_single_attention_torch(_get(params, "layer_norm_a"), _get(params, "mha"),
                                        _get(params, "layer_norm_z"), _get(params, "linear_z"), dtype, device)


def single_attention_to_protenix(w: dict) -> ProtenixAttentionPairBiasParams:
    """Torch-layout dict (``synthetic.single_attention_weights``) -> Protenix
    container: ``pre_norm_s`` becomes ``layernorm_a``."""
    return ProtenixAttentionPairBiasParams(
        layernorm_a=_lnp(w["pre_norm_s"]), layernorm_kv=None,
        attention=AttentionParams(linear_q=_lin(w["proj_q"]), linear_k=_lin(w["proj_k"]), linear_v=_lin(w["proj_v"]),
                                  linear_o=_lin(w["proj_o"]), linear_g=_lin(w["proj_g"])),
        layernorm_z=_lnp(w["proj_z_norm"]), linear_z=_lin(w["proj_z"]),
    )


def single_attention_to_openfold3(w: dict) -> OpenFold3AttentionPairBiasParams:
    px = single_attention_to_protenix(w)
    return OpenFold3AttentionPairBiasParams(layer_norm_a=px.layernorm_a, layer_norm_z=px.layernorm_z,
                                            linear_z=px.linear_z, mha=px.attention)


def transition_to_protenix(w: dict) -> ProtenixTransitionParams:
    return ProtenixTransitionParams(layer_norm=_lnp(w["layer_norm"]), linear_a=_lin(w["linear_a"]),
                                    linear_b=_lin(w["linear_b"]), linear_out=_lin(w["linear_out"]))


def transition_to_openfold3(w: dict) -> dict:
    """Field dict -> OpenFold3 ``SwiGLUTransitionParams`` shape
    (``layer_norm``, ``swiglu.linear_a/b``, ``linear_out``)."""
    return {"layer_norm": _lnp(w["layer_norm"]),
            "swiglu": {"linear_a": _lin(w["linear_a"]), "linear_b": _lin(w["linear_b"])},
            "linear_out": _lin(w["linear_out"])}


def pairformer_block_to_protenix(w: dict) -> ProtenixPairformerBlockParams:
    """Field dicts of one layer (``synthetic.pairformer_layer_weights``) ->
    Protenix ``PairformerBlockParams``."""
    return ProtenixPairformerBlockParams(
        tri_mul_out=trimul_to_protenix(w["tri_mul_out"]), tri_mul_in=trimul_to_protenix(w["tri_mul_in"]),
        tri_att_start=triattn_to_protenix(w["tri_att_start"]), tri_att_end=triattn_to_protenix(w["tri_att_end"]),
        pair_transition=transition_to_protenix(w["transition_z"]),
        attention_pair_bias=single_attention_to_protenix(w["attention"]),
        single_transition=transition_to_protenix(w["transition_s"]),
    )


def pairformer_block_to_openfold3(w: dict) -> OpenFold3PairformerBlockParams:
    """Field dicts of one layer -> OpenFold3 ``PairformerBlockParams``."""
    return OpenFold3PairformerBlockParams(
        pair_stack=OpenFold3PairBlockParams(
            tri_mul_out=trimul_to_openfold3(w["tri_mul_out"]), tri_mul_in=trimul_to_openfold3(w["tri_mul_in"]),
            tri_att_start=triattn_to_openfold3(w["tri_att_start"]), tri_att_end=triattn_to_openfold3(w["tri_att_end"]),
            pair_transition=transition_to_openfold3(w["transition_z"]),
        ),
        attn_pair_bias=single_attention_to_openfold3(w["attention"]),
        single_transition=transition_to_openfold3(w["transition_s"]),
    )
