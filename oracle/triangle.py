"""Float64 numpy restatement of the reference's jnp/XLA triangle path.

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never the thing
measured or shipped. The product package does not import it.

Every function restates one reference function, cited as ``path:line``
relative to the eightmm/FoldJAX checkout. All arithmetic is float64, so the
result stands for the reference's fp32 computation (the parity bar in fp32
mode is max-abs 1e-4; in bf16 mode the HIP output is compared with this on the
same bf16-valued inputs and weights, relative error 2e-2).

Parameter containers are plain dicts. Boltz-2 uses its own nested dict with
``[in, out]`` kernels; Protenix and OpenFold3 use dicts keyed by the field
names of their NamedTuples, with PyTorch ``[out, in]`` weights. Attribute
access (NamedTuples) is accepted too, via ``_get``.

Pinning (tests/test_oracle.py): brute-force Python loops on tiny shapes, the
torch CPU library routines ``layer_norm`` and ``scaled_dot_product_attention``
for the special cases that reduce to them, the three ports agreeing with one
another under the documented weight mappings, and the reference's own
invariants (incoming == transposed outgoing with a/b swapped, ending ==
transposed starting, row-chunk invariance, padding isolation).
"""

from __future__ import annotations

import contextlib

import numpy as np

F64 = np.float64
_DT = [F64]  # the element type every function converts its inputs to


@contextlib.contextmanager
def compute_dtype(dtype):
    """Run the restatements in ``dtype`` instead of float64 (the CPU baseline
    times them in float32, the reference's fp32 arithmetic). Parity checks
    always use the float64 default."""
    _DT.append(np.dtype(dtype).type)
    try:
        yield
    finally:
        _DT.pop()


# ---------------------------------------------------------------------------
# bfloat16 programs (analysis mode)
# ---------------------------------------------------------------------------

_PROGRAM = [None]  # the port whose bfloat16 program is emulated, or None

#: Where each port's jnp program, run on bfloat16 inputs and weights, stores a
#: bfloat16 result: a jnp op on bfloat16 operands returns bfloat16. Points not
#: listed stay exact.
#:   Boltz-2 takes LayerNorm statistics in float32 and rounds the normalized
#:   value before the affine (``B2P/_common.py:15-26``); its attention core
#:   upcasts q, k, v and both biases and keeps scores, softmax and the
#:   probability-value product in float32 (``B2T/triangle_attention.py:446-455``).
#:   Protenix runs every LayerNorm op in bfloat16 (``PXP/primitives.py:57-72``),
#:   multiplies bfloat16 q and k into bfloat16 logits, adds the float32 mask
#:   bias and the triangle bias, takes softmax in float32 and rounds the
#:   probabilities to bfloat16 before the value product (``PXT/triangle.py:850-860``).
#: Both store every projection, the scaled q, the sigmoid gates, the gated
#: products and the triangle contraction (Protenix accumulates it in float32
#: and casts, ``PXT/triangle.py:174``) in bfloat16.
_POINTS = {
    "boltz2": frozenset({"ln_normed", "ln_affine", "linear", "q_scale", "sigmoid", "gated", "contract", "attn_out"}),
    "protenix": frozenset(
        {"ln_ops", "ln_affine", "linear", "q_scale", "sigmoid", "gated", "contract", "logits", "probs", "attn_out"}
    ),
}


@contextlib.contextmanager
def bf16_program(port):
    """Round where ``port``'s bfloat16 program stores bfloat16 (``_POINTS``).

    Analysis mode, used to measure how far apart the ports' own bfloat16
    results are and where the HIP kernels sit between them; no parity bar
    rests on it (XLA's fusion may keep some of these values in float32, which
    only running the reference could settle). Inputs and weights should be
    bfloat16 values already. ``port=None`` is the exact default."""
    if port is not None and port not in _POINTS:
        raise ValueError(f"unknown port {port!r}; expected one of {tuple(_POINTS)}")
    _PROGRAM.append(port)
    try:
        yield
    finally:
        _PROGRAM.pop()


def bf16(x):
    """Round to the nearest bfloat16 value (ties to even), as float64."""
    b = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    r = r.astype(np.uint32).view(np.float32).astype(F64)
    x32 = np.asarray(x, dtype=np.float32)
    return np.where(np.isfinite(x32), r, x32.astype(F64))  # inf stays inf, NaN stays NaN


def _st(x, point):
    """``x`` as the emulated program stores it at ``point``."""
    port = _PROGRAM[-1]
    if port is None or point not in _POINTS[port]:
        return x
    return bf16(x)


def _get(obj, name):
    """Field access for dict- or NamedTuple-shaped parameter containers."""
    if isinstance(obj, dict):
        return obj.get(name)
    return getattr(obj, name, None)


def _f(x):
    return None if x is None else np.asarray(x, dtype=_DT[-1])


# ---------------------------------------------------------------------------
# Leaf primitives
# ---------------------------------------------------------------------------


def layer_norm(x, weight, bias, eps=1e-5):
    """LayerNorm over the last axis.

    Boltz-2 ``B2P/_common.py:15-26`` (fp32 stats, ``rsqrt``), Protenix
    ``PXP/primitives.py:57-72`` and OpenFold3 ``OF3/primitives.py:81-97``
    (``1/sqrt``) are the same function in exact arithmetic; the optional
    weight/bias follow the Protenix/OpenFold3 containers.
    """
    x = _f(x)
    if _PROGRAM[-1] is not None and "ln_ops" in _POINTS[_PROGRAM[-1]]:
        # every op of the LayerNorm rounded to bfloat16
        mean = _st(x.mean(axis=-1, keepdims=True), "ln_ops")
        d = _st(x - mean, "ln_ops")
        var = _st(_st(np.square(d), "ln_ops").mean(axis=-1, keepdims=True), "ln_ops")
        r = _st(1.0 / _st(np.sqrt(_st(var + eps, "ln_ops")), "ln_ops"), "ln_ops")
        y = _st(d * r, "ln_ops")
    else:
        mean = x.mean(axis=-1, keepdims=True)
        var = np.square(x - mean).mean(axis=-1, keepdims=True)
        y = _st((x - mean) / np.sqrt(var + eps), "ln_normed")
    if weight is not None:
        y = _st(y * _f(weight), "ln_affine")
    if bias is not None:
        y = _st(y + _f(bias), "ln_affine")
    return y


def sigmoid(x):
    """Logistic sigmoid, evaluated stably.

    ``jax.nn.sigmoid`` (Boltz-2), ``1/(1+exp(-x))`` (``PXP/primitives.py:81-84``)
    and the branchwise form (``OF3/primitives.py:105-111``) agree in float64.
    """
    x = _f(x)
    e = np.exp(-np.abs(x))
    return _st(np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e)), "sigmoid")


def silu(x):
    """``x * sigmoid(x)`` (``PXP/primitives.py:75-78``, ``jax.nn.silu``)."""
    x = _f(x)
    return x * sigmoid(x)


def _mm(x, w_in_out):
    """``x @ W`` over the last axis, as one contiguous 2-D BLAS call."""
    x = _f(x)
    w = np.ascontiguousarray(_f(w_in_out))
    y = np.ascontiguousarray(x).reshape(-1, x.shape[-1]) @ w
    return _st(y.reshape(x.shape[:-1] + (w.shape[-1],)), "linear")


def linear_torch(x, lin):
    """PyTorch-layout linear ``x @ W.T + b`` (``PXP/primitives.py:48-54``)."""
    y = _mm(x, _f(_get(lin, "weight")).T)
    b = _get(lin, "bias")
    if b is not None:
        y = _st(y + _f(b), "linear")
    return y


def _ln_params(p):
    return _get(p, "weight"), _get(p, "bias")


def softmax(x, axis=-1):
    """Max-subtracted softmax, as ``jax.nn.softmax``."""
    x = _f(x)
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


# ---------------------------------------------------------------------------
# Triangle contraction
# ---------------------------------------------------------------------------


def triangle_contract(a, b, direction):
    """Per-channel contraction of two ``[..., N, N, C]`` projections.

    outgoing: ``out[i,j,c] = sum_k a[i,k,c] b[j,k,c]``
    incoming: ``out[i,j,c] = sum_k a[k,i,c] b[k,j,c]``
    (``B2T/triangle.py:215-254``, ``PXT/triangle.py:399-416``,
    ``OF3/triangle.py:64-79``). Written as a batched matmul over the channel
    axis moved to the front, which is how OpenFold3 spells it.
    """
    a = _f(a)
    b = _f(b)
    ac = np.moveaxis(a, -1, -3)  # [..., C, N, N]
    bc = np.moveaxis(b, -1, -3)
    if direction == "outgoing":
        out = np.ascontiguousarray(ac) @ np.ascontiguousarray(np.swapaxes(bc, -1, -2))
    elif direction == "incoming":
        out = np.ascontiguousarray(np.swapaxes(ac, -1, -2)) @ np.ascontiguousarray(bc)
    else:
        raise ValueError(f"Unsupported triangle multiplication direction: {direction!r}")
    return np.moveaxis(out, -3, -1)


# ---------------------------------------------------------------------------
# Triangle multiplicative update
# ---------------------------------------------------------------------------


def boltz2_triangle_multiplication(params, x, mask, direction, eps=1e-5):
    """Boltz-2 ``triangle_multiplication_forward`` XLA path.

    ``B2T/triangle.py:78-129``: LN_in; sigmoid GLU ``sigmoid(x@g_in)*(x@p_in)``
    (``B2P/glu_backend.py:73-74``); times mask; split into a (first c_h) and b;
    contraction; LN_out; ``@p_out``; times ``sigmoid(x_ln @ g_out)``. Kernels
    are ``[in, out]``. Returns the update; the caller adds it.
    """
    x = layer_norm(x, params["norm_in"]["scale"], params["norm_in"]["bias"], eps)
    mask = _f(mask)
    proj = _st(sigmoid(_mm(x, params["g_in"]["kernel"])) * _mm(x, params["p_in"]["kernel"]), "gated")
    proj = _st(proj * mask[..., None], "gated")
    a, b = np.split(proj, 2, axis=-1)
    out = _st(triangle_contract(a, b, direction), "contract")
    out = layer_norm(out, params["norm_out"]["scale"], params["norm_out"]["bias"], eps)
    out = _mm(out, params["p_out"]["kernel"])
    gate = sigmoid(_mm(x, params["g_out"]["kernel"]))
    return _st(out * gate, "gated")


def protenix_triangle_multiplication(z, mask, params, direction):
    """Protenix ``triangle_multiplication`` XLA path.

    ``PXT/triangle.py:166-228``: ``b = mask*sigmoid(lin(z_ln, b_g))*lin(z_ln, b_p)``,
    a likewise (``project_a``, :198-200), contraction in float32, cast, LN_out,
    ``linear_z``, times ``sigmoid(linear(z_ln, linear_g))``. LN eps is 1e-5.
    """
    z = _f(z)
    if mask is None:
        mask = np.ones(z.shape[:-1])
    m = _f(mask)[..., None]
    zn = layer_norm(z, *_ln_params(_get(params, "layer_norm_in")))
    b = _st(m * sigmoid(linear_torch(zn, _get(params, "linear_b_g"))), "gated")
    b = _st(b * linear_torch(zn, _get(params, "linear_b_p")), "gated")
    a = _st(m * sigmoid(linear_torch(zn, _get(params, "linear_a_g"))), "gated")
    a = _st(a * linear_torch(zn, _get(params, "linear_a_p")), "gated")
    out = _st(triangle_contract(a, b, direction), "contract")
    out = layer_norm(out, *_ln_params(_get(params, "layer_norm_out")))
    out = linear_torch(out, _get(params, "linear_z"))
    return _st(out * sigmoid(linear_torch(zn, _get(params, "linear_g"))), "gated")


def openfold3_triangle_multiplication(z, params, *, outgoing, mask=None, eps=1e-5):
    """OpenFold3 ``triangle_multiplication`` (``OF3/triangle.py:82-134``).

    Same function, with ``gate_mask = 1`` when the mask is ``None``; the
    contraction is the channel-major matmul of ``combine_projections``
    (``OF3/triangle.py:64-79``).
    """
    zn = layer_norm(z, *_ln_params(_get(params, "layer_norm_in")), eps=eps)
    gm = 1.0 if mask is None else _f(mask)[..., None]
    a = gm * sigmoid(linear_torch(zn, _get(params, "linear_a_g"))) * linear_torch(
        zn, _get(params, "linear_a_p")
    )
    b = gm * sigmoid(linear_torch(zn, _get(params, "linear_b_g"))) * linear_torch(
        zn, _get(params, "linear_b_p")
    )
    x = triangle_contract(a, b, "outgoing" if outgoing else "incoming")
    x = layer_norm(x, *_ln_params(_get(params, "layer_norm_out")), eps=eps)
    x = linear_torch(x, _get(params, "linear_z"))
    return x * sigmoid(linear_torch(zn, _get(params, "linear_g")))


# ---------------------------------------------------------------------------
# Triangle attention
# ---------------------------------------------------------------------------


def attention_rows(q, k, v, mask_bias, tri_bias, row_block=16):
    """Biased softmax attention for independent rows.

    ``q, k, v``: ``[..., I, H, J, D]`` with q already scaled;
    ``mask_bias``: ``[..., I, 1, 1, J]``; ``tri_bias``: ``[..., 1, H, J, J]``.
    ``scores = q k^T + mask_bias + tri_bias``; softmax over keys; ``p v``
    (``B2T/triangle_attention.py:428-455``, ``PXT/triangle.py:850-860``,
    ``OF3/attention.py:54-67``). Rows are processed in blocks of
    ``row_block``, which the reference shows is exact
    (``B2T/triangle_attention.py:458-493``).
    """
    q, k, v = _f(q), _f(k), _f(v)
    mask_bias, tri_bias = _f(mask_bias), _f(tri_bias)
    n_rows = q.shape[-4]
    out = np.empty(q.shape[:-1] + (v.shape[-1],), dtype=_DT[-1])
    for s in range(0, n_rows, row_block):
        e = min(n_rows, s + row_block)
        qs, ks, vs = q[..., s:e, :, :, :], k[..., s:e, :, :, :], v[..., s:e, :, :, :]
        mb = mask_bias[..., s:e, :, :, :] if mask_bias.shape[-4] > 1 else mask_bias
        scores = _st(np.ascontiguousarray(qs) @ np.ascontiguousarray(np.swapaxes(ks, -1, -2)), "logits")
        scores = scores + mb + tri_bias
        probs = _st(softmax(scores, axis=-1), "probs")
        out[..., s:e, :, :, :] = _st(probs @ np.ascontiguousarray(vs), "attn_out")
    return out


def _split_heads_torch(x, lin, heads):
    """``[..., J, C] -> [..., H, J, D]`` (``PXT/triangle.py:863-870``)."""
    y = linear_torch(x, lin)
    y = y.reshape(y.shape[:-1] + (heads, -1))
    return np.swapaxes(y, -2, -3)


def boltz2_triangle_attention(params, x, mask=None, starting=True, inf=1e9, eps=1e-5):
    """Boltz-2 ``triangle_attention_forward`` XLA path.

    ``B2T/triangle_attention.py:125-162`` and ``_attention`` :346-425: ending
    node swaps the two pair axes of x and mask in and out; LN; fp32
    ``mask_bias = inf*(mask-1)`` as ``[..., I, 1, 1, J]``; ``tri_bias = x @ W``
    moved to ``[..., 1, H, J, J]``; q,g from ``[W_q|W_g]``, k,v from
    ``[W_k|W_v]``; ``q /= sqrt(D)``; softmax attention; ``sigmoid(g)`` gate;
    ``@ W_o``. Kernels are ``[in, out]``.
    """
    x = _f(x)
    if mask is None:
        mask = np.ones(x.shape[:-1])
    mask = _f(mask)
    if not starting:
        x = np.swapaxes(x, -2, -3)
        mask = np.swapaxes(mask, -1, -2)
    x = layer_norm(x, params["layer_norm"]["scale"], params["layer_norm"]["bias"], eps)
    mask_bias = (inf * (mask - 1.0))[..., :, None, None, :]
    tri_bias = _mm(x, params["linear"]["kernel"])  # [..., I, J, H]
    tri_bias = np.moveaxis(tri_bias, -1, -3)[..., None, :, :, :]
    mha = params["mha"]
    heads = tri_bias.shape[-3]
    d = _f(mha["linear_g"]["kernel"]).shape[-1] // heads

    def proj(name):
        y = _mm(x, mha[name]["kernel"])
        y = y.reshape(y.shape[:-1] + (heads, d))
        return np.swapaxes(y, -2, -3)

    q = _st(proj("linear_q") / np.sqrt(d), "q_scale")
    k = proj("linear_k")
    v = proj("linear_v")
    o = attention_rows(q, k, v, mask_bias, tri_bias)
    o = np.swapaxes(o, -2, -3)  # [..., I, J, H, D]
    gate = sigmoid(_mm(x, mha["linear_g"]["kernel"])).reshape(o.shape)
    o = _st(o * gate, "gated").reshape(o.shape[:-2] + (heads * d,))
    out = _mm(o, mha["linear_o"]["kernel"])
    if not starting:
        out = np.swapaxes(out, -2, -3)
    return out


def protenix_triangle_attention(x, mask, params, *, num_heads, starting=True, inf=1e9, rows=None):
    """Protenix ``triangle_attention`` dense path.

    ``PXT/triangle.py:509-535`` and ``_triangle_attention_dense`` :732-847:
    same math as Boltz-2 with torch-layout weights, ``scale = D**-0.5``
    multiplied into q (:792), and an optional ``linear_g``.

    ``rows``: compute only these rows of the attention grid (rows i of x for
    the starting node, columns for the ending node) and return them as
    ``[..., len(rows), N, C]`` in that grid (not swapped back); the
    reference's row blocking shows rows are independent
    (``PXT/triangle.py:850-860``). The bias still comes from the whole grid.
    """
    x = _f(x)
    if mask is None:
        mask = np.ones(x.shape[:-1])
    mask = _f(mask)
    if not starting:
        # the transposed grid as its own array: numpy runs every later op of
        # the whole-grid computation on it at the speed of a contiguous one
        x = np.ascontiguousarray(np.swapaxes(x, -2, -3))
        mask = np.ascontiguousarray(np.swapaxes(mask, -1, -2))
    x = layer_norm(x, *_ln_params(_get(params, "layer_norm")))
    mask_bias = (inf * (mask - 1.0))[..., :, None, None, :]
    tri_bias = linear_torch(x, _get(params, "linear"))
    tri_bias = np.moveaxis(tri_bias, -1, -3)[..., None, :, :, :]
    if rows is not None:
        rows = np.asarray(rows)
        x = x[..., rows, :, :]
        mask_bias = mask_bias[..., rows, :, :, :]
    att = _get(params, "attention")
    d = _f(_get(_get(att, "linear_k"), "weight")).shape[0] // num_heads
    q = _st(_split_heads_torch(x, _get(att, "linear_q"), num_heads) * (float(d) ** -0.5), "q_scale")
    k = _split_heads_torch(x, _get(att, "linear_k"), num_heads)
    v = _split_heads_torch(x, _get(att, "linear_v"), num_heads)
    o = np.swapaxes(attention_rows(q, k, v, mask_bias, tri_bias), -2, -3)
    if _get(att, "linear_g") is not None:
        o = _st(o * sigmoid(linear_torch(x, _get(att, "linear_g"))).reshape(o.shape), "gated")
    o = o.reshape(o.shape[:-2] + (-1,))
    out = linear_torch(o, _get(att, "linear_o"))
    if not starting and rows is None:
        out = np.ascontiguousarray(np.swapaxes(out, -2, -3))
    return out


def openfold3_triangle_attention(x, params, *, no_heads, mask=None, starting=True, inf=1e9, eps=1e-5):
    """OpenFold3 ``triangle_attention`` (``OF3/triangle_attention.py:159-195``).

    Biases are added in the order ``(mask_bias, triangle_bias)``
    (``OF3/attention.py:64-66``); ``query / sqrt(D)`` (``OF3/attention.py:100``);
    the gate multiplies the ``[..., J, H, D]`` output (:106-108).
    """
    x = _f(x)
    if mask is None:
        mask = np.ones(x.shape[:-1])
    mask = _f(mask)
    if not starting:
        x = np.swapaxes(x, -2, -3)
        mask = np.swapaxes(mask, -1, -2)
    x = layer_norm(x, *_ln_params(_get(params, "layer_norm")), eps=eps)
    mask_bias = (inf * (mask - 1.0))[..., :, None, None, :]
    tri_bias = np.moveaxis(linear_torch(x, _get(params, "linear_z")), -1, -3)[..., None, :, :, :]
    mha = _get(params, "mha")
    q = _split_heads_torch(x, _get(mha, "linear_q"), no_heads)
    q = q / np.sqrt(q.shape[-1])
    k = _split_heads_torch(x, _get(mha, "linear_k"), no_heads)
    v = _split_heads_torch(x, _get(mha, "linear_v"), no_heads)
    o = np.swapaxes(attention_rows(q, k, v, mask_bias, tri_bias), -2, -3)
    if _get(mha, "linear_g") is not None:
        o = o * sigmoid(linear_torch(x, _get(mha, "linear_g"))).reshape(o.shape)
    out = linear_torch(o.reshape(o.shape[:-2] + (-1,)), _get(mha, "linear_o"))
    if not starting:
        out = np.swapaxes(out, -2, -3)
    return out


def attention_core(q, k, v, tri_bias, mask_bias, scale):
    """The kernel-boundary core: ``cueq_attention_core`` semantics.

    ``M/_cueq.py:66-121``: q/k/v ``[B, I, H, J, D]``, ``tri_bias``
    ``[B, 1, H, J, J]``, additive ``mask_bias`` ``[B, I, 1, 1, J]``; ``scale``
    applied inside. Returns ``[B, I, H, J, D]``.
    """
    return attention_rows(_f(q) * scale, k, v, mask_bias, tri_bias)


# ---------------------------------------------------------------------------
# Weight mappings between the three ports (test helpers)
# ---------------------------------------------------------------------------


def trimul_torch_to_boltz2(p):
    """Protenix/OpenFold3 tri-mul fields -> Boltz-2 dict.

    Boltz-2's fused ``p_in``/``g_in`` are ``[c_z, 2c_h]`` with the a half first
    (``B2T/triangle.py:102``; torch layout ``[2c_h, c_z]`` per
    ``B2T/triangle_cueq.py:94-95``).
    """
    w = lambda name: _f(_get(_get(p, name), "weight"))  # noqa: E731
    lin = _get(p, "layer_norm_in")
    lout = _get(p, "layer_norm_out")
    return {
        "norm_in": {"scale": _f(_get(lin, "weight")), "bias": _f(_get(lin, "bias"))},
        "p_in": {"kernel": np.concatenate([w("linear_a_p"), w("linear_b_p")], 0).T},
        "g_in": {"kernel": np.concatenate([w("linear_a_g"), w("linear_b_g")], 0).T},
        "norm_out": {"scale": _f(_get(lout, "weight")), "bias": _f(_get(lout, "bias"))},
        "p_out": {"kernel": w("linear_z").T},
        "g_out": {"kernel": w("linear_g").T},
    }


def triattn_torch_to_boltz2(p, *, bias_name="linear", mha_name="attention"):
    """Protenix (``linear``/``attention``) or OpenFold3 (``linear_z``/``mha``)
    tri-attn fields -> Boltz-2 dict (``M/boltz2/bridge/torch_mapping.py:553-600``)."""
    ln = _get(p, "layer_norm")
    mha = _get(p, mha_name)
    k = lambda lin: _f(_get(lin, "weight")).T  # noqa: E731
    return {
        "layer_norm": {"scale": _f(_get(ln, "weight")), "bias": _f(_get(ln, "bias"))},
        "linear": {"kernel": k(_get(p, bias_name))},
        "mha": {n: {"kernel": k(_get(mha, n))} for n in ("linear_q", "linear_k", "linear_v", "linear_o", "linear_g")},
    }


# ---------------------------------------------------------------------------
# The rest of a Pairformer block: transition and single-track attention
# ---------------------------------------------------------------------------


def transition(x, p, *, mask=None, eps=1e-5):
    """SwiGLU transition: ``(silu(LN(x) Wa^T) * (LN(x) Wb^T)) Wo^T [* mask]``.

    Protenix ``_transition_block`` (``PXP/primitives.py:88-93``), Boltz-2
    ``transition_forward`` (``B2P/transition.py:112-116``: fc1 = a, fc2 = b,
    fc3 = out), OpenFold3 ``swiglu_transition`` (``OF3/primitives.py:133-150``,
    optional mask over the last axis).
    """
    y = layer_norm(x, *_ln_params(_get(p, "layer_norm")), eps=eps)
    h = silu(linear_torch(y, _get(p, "linear_a"))) * linear_torch(y, _get(p, "linear_b"))
    out = linear_torch(h, _get(p, "linear_out"))
    if mask is not None:
        out = out * _f(mask)[..., None]
    return out


def boltz2_attention_pair_bias(p, s, z, mask, *, inf=1e6, eps=1e-5):
    """Boltz-2 ``attention_pair_bias_forward`` XLA path with ``k_in = s``.

    ``B2P/attention.py:44-115``: q/g from ``s`` (q with bias), k/v from ``s``;
    ``bias = LN_z(z) W_z^T`` as ``[B, H, N, N]``; scores
    ``q k^T / sqrt(d) + bias + (1 - mask[b, key]) * (-inf)``; softmax; gate
    ``sigmoid(g)``; ``@ W_o``. ``s`` is the already normalised single
    representation; weights are torch-layout under the Boltz-2 module names.
    """
    s = _f(s)
    z = _f(z)
    mask = _f(mask)
    b, n, c_s = s.shape
    heads = _f(p["proj_z"]["weight"]).shape[0]
    d = c_s // heads
    q = linear_torch(s, p["proj_q"]).reshape(b, n, heads, d)
    g = sigmoid(linear_torch(s, {"weight": p["proj_g"]["weight"]}))
    k = linear_torch(s, {"weight": p["proj_k"]["weight"]}).reshape(b, n, heads, d)
    v = linear_torch(s, {"weight": p["proj_v"]["weight"]}).reshape(b, n, heads, d)
    bias = linear_torch(layer_norm(z, p["proj_z_norm"]["weight"], p["proj_z_norm"]["bias"], eps), {"weight": p["proj_z"]["weight"]})
    bias = np.transpose(bias, (0, 3, 1, 2))  # [B, H, N, N]
    mask_bias = (1.0 - mask[:, None, None, :]) * -inf
    qh = np.ascontiguousarray(np.transpose(q, (0, 2, 1, 3)))
    kh = np.ascontiguousarray(np.transpose(k, (0, 2, 3, 1)))
    vh = np.ascontiguousarray(np.transpose(v, (0, 2, 1, 3)))
    attn = qh @ kh / np.sqrt(d) + bias + mask_bias
    o = softmax(attn, axis=-1) @ vh  # [B, H, N, d]
    o = np.transpose(o, (0, 2, 1, 3)).reshape(b, n, c_s)
    return linear_torch(g * o, {"weight": p["proj_o"]["weight"]})


def boltz2_pairformer_no_seq_layer(p, z, pair_mask, *, eps=1e-5):
    """The pair half of a Boltz-2 layer, which is also the MSA module's
    ``pairformer_no_seq_layer_forward`` (``B2K/msa.py:467-539``): z +=
    tri_mul_out, tri_mul_in, tri_att_start, tri_att_end (all with the pair
    mask), then the unmasked transition_z. Field dicts as in
    ``boltz2_pairformer_layer``."""
    heads = _f(p["tri_att_start"]["linear"]["weight"]).shape[0]
    z = _f(z) + protenix_triangle_multiplication(z, pair_mask, p["tri_mul_out"], "outgoing")
    z = z + protenix_triangle_multiplication(z, pair_mask, p["tri_mul_in"], "incoming")
    z = z + protenix_triangle_attention(z, pair_mask, p["tri_att_start"], num_heads=heads, starting=True)
    z = z + protenix_triangle_attention(z, pair_mask, p["tri_att_end"], num_heads=heads, starting=False)
    return z + transition(z, p["transition_z"], eps=eps)


def boltz2_pairformer_layer(p, s, z, mask, pair_mask, *, eps=1e-5):
    """One Boltz-2 ``pairformer_layer_forward`` (``B2K/pairformer.py:100-206``):
    z += tri_mul_out, tri_mul_in, tri_att_start, tri_att_end, transition_z;
    s += attention_pair_bias(LN(s), z, mask); s += transition_s.

    ``p`` holds torch-layout field dicts: ``tri_mul_out``/``tri_mul_in``
    (``linear_a_p`` ...), ``tri_att_start``/``tri_att_end`` (``layer_norm``,
    ``linear``, ``attention``), ``transition_z``/``transition_s``
    (``layer_norm``, ``linear_a``, ``linear_b``, ``linear_out``), ``attention``
    (``pre_norm_s``, ``proj_*``). Returns ``(s, z)``.
    """
    z = boltz2_pairformer_no_seq_layer(p, z, pair_mask, eps=eps)
    a = p["attention"]
    s_ln = layer_norm(s, a["pre_norm_s"]["weight"], a["pre_norm_s"]["bias"], eps)
    s = _f(s) + boltz2_attention_pair_bias(a, s_ln, z, mask, eps=eps)
    s = s + transition(s, p["transition_s"], eps=eps)
    return s, z


# ---------------------------------------------------------------------------
# Sampled output positions at full size (configs 3-5)
# ---------------------------------------------------------------------------
#
# At N = 1024 .. 3072 the full float64 restatements above need tens of GB.
# Each output position of a triangle sublayer depends on only a few lines of
# the pair tensor, so the same formulas are restated here per position:
# ``z`` and ``mask`` are anything indexable as ``z[i]`` (row i, ``[N, C]``) and
# ``z[:, j]`` (column j), e.g. a numpy array or a test-side view of a device
# tensor; every line is converted to float64. Pinned against the full
# functions on small shapes (tests/test_oracle.py).


def _line(z, idx, transposed):
    return _f(z[:, idx] if transposed else z[idx])


def triangle_multiplication_at(z, mask, params, direction, positions, eps=1e-5):
    """Protenix/OpenFold3-form tri-mul update (torch-layout field names) at
    ``positions`` ``[(i, j), ...]`` of a ``[N, N, C]`` pair tensor.

    The formula of ``protenix_triangle_multiplication`` (``PXT/triangle.py:166-228``):
    outgoing ``o[i,j] = sum_k a[i,k] b[j,k]`` reads rows i and j of z and the
    mask, incoming ``o[i,j] = sum_k a[k,i] b[k,j]`` reads columns i and j, with
    ``a = m * sigmoid(LN(z) A_g^T) * (LN(z) A_p^T)`` (b likewise); then
    ``LN_out(o) W_z^T * sigmoid(LN(z[i,j]) W_g^T)``. Returns ``[len(positions), C]``.
    """
    t = direction == "incoming"
    if direction not in ("outgoing", "incoming"):
        raise ValueError(f"Unsupported triangle multiplication direction: {direction!r}")
    ln_in = _ln_params(_get(params, "layer_norm_in"))
    cache = {}

    def proj(idx):
        if idx not in cache:
            zl = _line(z, idx, t)
            m = np.ones(zl.shape[0]) if mask is None else _line(mask, idx, t)
            zn = layer_norm(zl, *ln_in, eps=eps)
            a = m[:, None] * sigmoid(linear_torch(zn, _get(params, "linear_a_g"))) * linear_torch(
                zn, _get(params, "linear_a_p"))
            b = m[:, None] * sigmoid(linear_torch(zn, _get(params, "linear_b_g"))) * linear_torch(
                zn, _get(params, "linear_b_p"))
            cache[idx] = (a, b, zl)
        return cache[idx]

    out = []
    for i, j in positions:
        a_i, _, zl_i = proj(i)
        _, b_j, zl_j = proj(j)
        o = (a_i * b_j).sum(axis=0)
        o = layer_norm(o, *_ln_params(_get(params, "layer_norm_out")), eps=eps)
        y = linear_torch(o, _get(params, "linear_z"))
        x_ij = zl_j[i] if t else zl_i[j]  # z[i, j]: row i at column j, or column j at row i
        xn = layer_norm(x_ij, *ln_in, eps=eps)
        out.append(y * sigmoid(linear_torch(xn, _get(params, "linear_g"))))
    return np.stack(out)


def triangle_attention_at(z, mask, params, *, num_heads, starting, positions, inf=1e9, eps=1e-5):
    """Protenix-form tri-attn update (``linear`` / ``attention`` field names) at
    ``positions`` ``[(i, q), ...]`` of the attention grid.

    The formula of ``protenix_triangle_attention`` (``PXT/triangle.py:509-535,
    732-847``) for one attention row i and one query q: keys, values, the
    mask bias ``inf * (m[i, k] - 1)`` come from line i of the grid, the query
    and gate from its entry q, and the triangle bias ``LN(x)[q, k] . w_b`` from
    line q. Starting node: the grid is z (lines are rows), and the result is
    the update at ``[i, q]``; ending node: the grid is z transposed (lines are
    columns), and the result is the update at ``[q, i]``. Returns
    ``[len(positions), C]``.
    """
    t = not starting
    ln = _ln_params(_get(params, "layer_norm"))
    att = _get(params, "attention")
    cache = {}

    def line(idx):
        if idx not in cache:
            cache[idx] = layer_norm(_line(z, idx, t), *ln, eps=eps)
        return cache[idx]

    out = []
    for i, q in positions:
        xi = line(i)  # [N, C]
        n = xi.shape[0]
        m = np.ones(n) if mask is None else _line(mask, i, t)
        k = linear_torch(xi, _get(att, "linear_k")).reshape(n, num_heads, -1)
        v = linear_torch(xi, _get(att, "linear_v")).reshape(n, num_heads, -1)
        d = k.shape[-1]
        qv = linear_torch(xi[q], _get(att, "linear_q")).reshape(num_heads, d) * (float(d) ** -0.5)
        bias = linear_torch(line(q), _get(params, "linear"))  # [N(k), H]
        s = np.einsum("hd,khd->hk", qv, k) + (inf * (m - 1.0))[None, :] + bias.T
        o = np.einsum("hk,khd->hd", softmax(s, axis=-1), v)
        if _get(att, "linear_g") is not None:
            o = o * sigmoid(linear_torch(xi[q], _get(att, "linear_g"))).reshape(num_heads, d)
        out.append(linear_torch(o.reshape(-1), _get(att, "linear_o")))
    return np.stack(out)


def boltz2_attention_pair_bias_at(p, s, z, mask, queries, *, inf=1e6, eps=1e-5):
    """``boltz2_attention_pair_bias`` (``B2P/attention.py:44-115``) for one batch
    item at the query rows ``queries``: ``s`` ``[N, c_s]`` normalised single
    representation, ``z`` indexable by row (row i gives the bias row
    ``LN_z(z[i, :]) W_z^T``), ``mask`` ``[N]``. Returns ``[len(queries), c_s]``."""
    s = _f(s)
    mask = _f(mask)
    n, c_s = s.shape
    heads = _f(p["proj_z"]["weight"]).shape[0]
    d = c_s // heads
    k = linear_torch(s, {"weight": p["proj_k"]["weight"]}).reshape(n, heads, d)
    v = linear_torch(s, {"weight": p["proj_v"]["weight"]}).reshape(n, heads, d)
    out = []
    for i in queries:
        q = linear_torch(s[i], p["proj_q"]).reshape(heads, d)
        g = sigmoid(linear_torch(s[i], {"weight": p["proj_g"]["weight"]}))
        bias = linear_torch(layer_norm(_f(z[i]), p["proj_z_norm"]["weight"], p["proj_z_norm"]["bias"], eps),
                            {"weight": p["proj_z"]["weight"]})  # [N(j), H]
        sc = np.einsum("hd,jhd->hj", q, k) / np.sqrt(d) + bias.T + ((1.0 - mask) * -inf)[None, :]
        o = np.einsum("hj,jhd->hd", softmax(sc, axis=-1), v).reshape(-1)
        out.append(linear_torch(g * o, {"weight": p["proj_o"]["weight"]}))
    return np.stack(out)


def pair_bias_at(p, z, positions, *, eps=1e-5):
    """The single attention's pair bias ``LN_z(z[i, j]) W_z^T`` (``B2P/attention.py:69-75``)
    at ``positions`` ``[(i, j), ...]``; returns ``[len(positions), H]``."""
    rows = np.stack([_f(z[i])[j] for i, j in positions])
    return linear_torch(layer_norm(rows, p["proj_z_norm"]["weight"], p["proj_z_norm"]["bias"], eps),
                        {"weight": p["proj_z"]["weight"]})


# ---------------------------------------------------------------------------
# Protenix and OpenFold3 single attention with pair bias, and their blocks
# ---------------------------------------------------------------------------


def gated_attention(q_x, kv_x, att, num_heads, biases=()):
    """Gated multi-head attention of the Protenix and OpenFold3 ports.

    Protenix ``attention`` (``PXP/attention.py:60-99``: ``prepare_qkv`` :43-57
    splits heads and divides q by ``sqrt(d)``, ``_attention_qkv_chunk``
    :374-378 adds the bias and softmaxes, the gate is
    ``sigmoid(linear(q_x, linear_g))`` per head) and OpenFold3 ``attention``
    (``OF3/attention.py:71-112``, the same steps with the biases added in
    order). ``biases`` broadcast against ``[..., H, Q, K]``.
    """
    q_x = _f(q_x)
    kv_x = _f(kv_x)
    q = _split_heads_torch(q_x, _get(att, "linear_q"), num_heads)  # [..., H, Q, D]
    k = _split_heads_torch(kv_x, _get(att, "linear_k"), num_heads)
    v = _split_heads_torch(kv_x, _get(att, "linear_v"), num_heads)
    q = q / np.sqrt(q.shape[-1])
    logits = np.ascontiguousarray(q) @ np.ascontiguousarray(np.swapaxes(k, -1, -2))
    for b in biases:
        logits = logits + _f(b)
    o = np.swapaxes(softmax(logits, axis=-1) @ np.ascontiguousarray(v), -2, -3)  # [..., Q, H, D]
    if _get(att, "linear_g") is not None:
        o = o * sigmoid(linear_torch(q_x, _get(att, "linear_g"))).reshape(o.shape)
    return linear_torch(o.reshape(o.shape[:-2] + (-1,)), _get(att, "linear_o"))


def protenix_attention_pair_bias(a, z, params, *, num_heads, extra_attn_bias=None, eps=1e-5):
    """Protenix ``attention_pair_bias`` (``PXP/attention.py:108-169``), trunk
    form (``has_s=False``, no cross attention, ``z`` not pre-normalised):
    ``q_x = LN_a(a)``; ``bias = LN_z(z) W_z^T`` moved to ``[..., H, N, N]``;
    ``extra_attn_bias`` (``[..., N, N]`` or ``[..., H, N, N]``) is added after
    the rank alignment of :140-150; then ``gated_attention(q_x, q_x, ...)``.
    Returns the update."""
    q_x = layer_norm(a, *_ln_params(_get(params, "layernorm_a")), eps=eps)
    bias = np.moveaxis(linear_torch(layer_norm(z, *_ln_params(_get(params, "layernorm_z")), eps=eps),
                                    _get(params, "linear_z")), -1, -3)
    if extra_attn_bias is not None:
        e = _f(extra_attn_bias)
        while e.ndim < bias.ndim - 1:
            e = e[None]
        if e.ndim == bias.ndim - 1:
            e = np.expand_dims(e, -3)
        bias = bias + e
    return gated_attention(q_x, q_x, _get(params, "attention"), num_heads, (bias,))


def openfold3_attention_pair_bias(a, z, params, *, no_heads, mask=None, inf=1e9, eps=1e-5):
    """OpenFold3 trunk ``attention_pair_bias`` (``OF3/attention_pair_bias.py:40-75``):
    ``a = LN_a(a)``; ``mask_bias = inf (mask - 1)`` over keys; ``pair_bias =
    LN_z(z) W_z^T`` as ``[..., H, N, N]``; ``attention(a, a, mha, biases=(mask_bias,
    pair_bias))``. Returns the update."""
    a = layer_norm(a, *_ln_params(_get(params, "layer_norm_a")), eps=eps)
    if mask is None:
        mask = np.ones(a.shape[:-1])
    mask_bias = (inf * (_f(mask) - 1.0))[..., None, None, :]
    pair_bias = np.moveaxis(linear_torch(layer_norm(z, *_ln_params(_get(params, "layer_norm_z")), eps=eps),
                                         _get(params, "linear_z")), -1, -3)
    return gated_attention(a, a, _get(params, "mha"), no_heads, (mask_bias, pair_bias))


def protenix_pairformer_block(s, z, pair_mask, params):
    """Protenix ``pairformer_block`` (``PXK/pairformer.py:49-180``).

    With a pair mask: ``pair_gate = bool(pair_mask)`` multiplies z at entry and
    after every sublayer (:74-77, 99-149); ``single_valid`` is the diagonal of
    the boolean pair mask, ``single_gate`` gates s at entry and after each
    single-track sublayer, and the single attention gets the extra bias
    ``-1e10`` wherever query or key is invalid (:80-87). The ending-node
    attention is a starting module between two transposes (:123-140). Heads
    come from the weight shapes (:112, :157). ``params`` is a dict (or
    NamedTuple) with the fields of ``PairformerBlockParams`` (:31-41), the
    triangle sublayers in the Protenix field names. Returns ``(s, z)``.
    """
    z = _f(z)
    s = None if s is None else _f(s)
    pair_gate = single_gate = extra = None
    if pair_mask is not None:
        valid = _f(pair_mask) != 0
        pair_gate = valid.astype(F64)[..., None]
        z = z * pair_gate
        single_valid = np.diagonal(valid, axis1=-2, axis2=-1)
        single_gate = single_valid.astype(F64)[..., None]
        extra = np.where(single_valid[..., :, None] & single_valid[..., None, :], 0.0, -1.0e10)
        if s is not None:
            s = s * single_gate

    def gate(z):
        return z if pair_gate is None else z * pair_gate

    z = gate(z + protenix_triangle_multiplication(z, pair_mask, _get(params, "tri_mul_out"), "outgoing"))
    z = gate(z + protenix_triangle_multiplication(z, pair_mask, _get(params, "tri_mul_in"), "incoming"))
    heads = _f(_get(_get(_get(params, "tri_att_start"), "linear"), "weight")).shape[0]
    z = gate(z + protenix_triangle_attention(z, pair_mask, _get(params, "tri_att_start"), num_heads=heads))
    zt = np.swapaxes(z, -2, -3)
    mt = None if pair_mask is None else np.swapaxes(_f(pair_mask), -1, -2)
    zt = zt + protenix_triangle_attention(zt, mt, _get(params, "tri_att_end"), num_heads=heads)
    z = gate(np.swapaxes(zt, -2, -3))
    z = gate(z + transition(z, _get(params, "pair_transition")))
    apb = _get(params, "attention_pair_bias")
    if apb is not None:
        if s is None:
            raise ValueError("PairformerBlock single path requires s")
        heads_s = _f(_get(_get(apb, "linear_z"), "weight")).shape[0]
        s = s + protenix_attention_pair_bias(s, z, apb, num_heads=heads_s, extra_attn_bias=extra)
        if single_gate is not None:
            s = s * single_gate
        s = s + transition(s, _get(params, "single_transition"))
        if single_gate is not None:
            s = s * single_gate
    return s, z


def openfold3_pair_block(z, params, *, pair_mask, no_heads_pair, inf=1e9, mask_transition=True,
                         tri_mul_first=True, eps=1e-5):
    """OpenFold3 ``pair_block`` (``OF3/pair_block.py:106-190``): tri-mul out and
    in, tri-attn start and end (the ending node a starting module between two
    transposes, :65-103), ``tri_mul_first`` ordering the two pairs, then the
    SwiGLU transition multiplied by ``pair_mask`` when ``mask_transition``.
    Each sublayer is a residual add."""
    z = _f(z)

    def mul_pair(z):
        z = z + openfold3_triangle_multiplication(z, _get(params, "tri_mul_out"), outgoing=True, mask=pair_mask,
                                                  eps=eps)
        return z + openfold3_triangle_multiplication(z, _get(params, "tri_mul_in"), outgoing=False, mask=pair_mask,
                                                     eps=eps)

    def att_pair(z):
        z = z + openfold3_triangle_attention(z, _get(params, "tri_att_start"), no_heads=no_heads_pair,
                                             mask=pair_mask, inf=inf, eps=eps)
        zt = np.swapaxes(z, -2, -3)
        mt = None if pair_mask is None else np.swapaxes(_f(pair_mask), -1, -2)
        zt = zt + openfold3_triangle_attention(zt, _get(params, "tri_att_end"), no_heads=no_heads_pair, mask=mt,
                                               inf=inf, eps=eps)
        return np.swapaxes(zt, -2, -3)

    z = att_pair(mul_pair(z)) if tri_mul_first else mul_pair(att_pair(z))
    return z + transition(z, _get(params, "pair_transition"), mask=pair_mask if mask_transition else None, eps=eps)


def openfold3_pairformer_block(s, z, params, *, single_mask, pair_mask, no_heads_pair, no_heads_pair_bias, inf=1e9,
                               mask_transition=True, eps=1e-5):
    """OpenFold3 ``pairformer_block`` (``OF3/pairformer.py:42-102``): z through
    ``pair_block``; ``s += attention_pair_bias(s, z, mask=single_mask)``;
    ``s += swiglu_transition(s, mask=single_mask if mask_transition)``.
    ``params`` has ``pair_stack``, ``attn_pair_bias`` and ``single_transition``
    (``OF3/pairformer.py:27-33``). Returns ``(s, z)``."""
    z = openfold3_pair_block(z, _get(params, "pair_stack"), pair_mask=pair_mask, no_heads_pair=no_heads_pair,
                             inf=inf, mask_transition=mask_transition, eps=eps)
    s = _f(s) + openfold3_attention_pair_bias(s, z, _get(params, "attn_pair_bias"), no_heads=no_heads_pair_bias,
                                              mask=single_mask, inf=inf, eps=eps)
    s = s + transition(s, _get(params, "single_transition"), mask=single_mask if mask_transition else None, eps=eps)
    return s, z
