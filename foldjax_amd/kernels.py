"""Tensor-level entry points of the HIP triangle kernels.

Torch tensors are used only as device-memory handles: every call passes raw
device pointers, sizes and the current HIP stream through the C ABI of
``include/fjx_tri.h``. There is no other code path -- if the library is
missing, the call raises.

Weights are packed once into the PyTorch ``[out, in]`` layout of the ABI
(``TriMulWeights`` / ``TriAttnWeights``); ``foldjax_amd.params`` builds them
from each port's parameter containers.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields
from typing import ClassVar

import torch

from foldjax_amd import _lib

_DTYPES = {torch.float32: _lib.FJX_DTYPE_F32, torch.bfloat16: _lib.FJX_DTYPE_BF16}


def _code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"the hip triangle kernels take float32 or bfloat16, got {dtype}") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dev(x: torch.Tensor) -> None:
    if x.device.type != "cuda":
        raise ValueError(f"the hip backend needs device tensors, got a tensor on {x.device}")


def _stream(x: torch.Tensor) -> int:
    return torch.cuda.current_stream(x.device).cuda_stream


def _prep(t: torch.Tensor | None, dtype: torch.dtype, device) -> torch.Tensor | None:
    if t is None:
        return None
    return t.to(device=device, dtype=dtype).contiguous()


def _same_device(x: torch.Tensor, **operands) -> None:
    """Every operand must live on ``x``'s device: a host tensor's pointer
    handed to a kernel would be read as device memory."""
    for name, t in operands.items():
        if t is not None and t.device != x.device:
            raise ValueError(f"{name} is on {t.device} but the input is on {x.device}; "
                             "every operand must be on the input's device")


def _need_shape(name: str, t: torch.Tensor | None, shape) -> None:
    if t is not None and tuple(t.shape) != tuple(int(v) for v in shape):
        raise ValueError(f"{name} must have shape {tuple(int(v) for v in shape)}, got {tuple(t.shape)}")


def _rows_of(m: torch.Tensor | None, shape, dtype: torch.dtype, name: str) -> torch.Tensor | None:
    """A per-row (per-position) mask broadcast to ``shape`` in ``dtype``,
    contiguous, as the kernels index it."""
    if m is None:
        return None
    try:
        m = torch.broadcast_to(m, tuple(shape))
    except RuntimeError:
        raise ValueError(f"{name} of shape {tuple(m.shape)} does not broadcast to {tuple(shape)}") from None
    return m.to(dtype=dtype).contiguous()


@dataclass(frozen=True)
class TriMulWeights:
    """Tri-mul weights in the ABI layout (PyTorch ``[out, in]``, a rows first)."""

    norm_in_weight: torch.Tensor  # [c_z]
    norm_in_bias: torch.Tensor  # [c_z]
    p_in_weight: torch.Tensor  # [2 c_h, c_z]
    g_in_weight: torch.Tensor  # [2 c_h, c_z]
    norm_out_weight: torch.Tensor  # [c_h]
    norm_out_bias: torch.Tensor  # [c_h]
    p_out_weight: torch.Tensor  # [c_z, c_h]
    g_out_weight: torch.Tensor  # [c_z, c_z]

    def to(self, dtype: torch.dtype, device) -> "TriMulWeights":
        return TriMulWeights(**{f.name: _prep(getattr(self, f.name), dtype, device) for f in fields(self)})

    def check(self, c_z: int) -> int:
        """Shapes against the pair width ``c_z``; returns ``c_h``."""
        c_h = int(self.norm_out_weight.shape[0])
        for name, shape in (("norm_in_weight", (c_z,)), ("norm_in_bias", (c_z,)), ("p_in_weight", (2 * c_h, c_z)),
                            ("g_in_weight", (2 * c_h, c_z)), ("norm_out_bias", (c_h,)), ("p_out_weight", (c_z, c_h)),
                            ("g_out_weight", (c_z, c_z))):
            _need_shape(f"tri-mul weight {name}", getattr(self, name), shape)
        return c_h


@dataclass(frozen=True)
class TriAttnWeights:
    """Tri-attn weights in the ABI layout (PyTorch ``[out, in]``)."""

    norm_weight: torch.Tensor  # [c_z]
    norm_bias: torch.Tensor  # [c_z]
    bias_weight: torch.Tensor  # [H, c_z]
    q_weight: torch.Tensor  # [H D, c_z]
    k_weight: torch.Tensor
    v_weight: torch.Tensor
    g_weight: torch.Tensor | None  # [H D, c_z] or None (ungated)
    o_weight: torch.Tensor  # [c_z, H D]

    @property
    def heads(self) -> int:
        return int(self.bias_weight.shape[0])

    def to(self, dtype: torch.dtype, device) -> "TriAttnWeights":
        return TriAttnWeights(**{f.name: _prep(getattr(self, f.name), dtype, device) for f in fields(self)})

    def check(self, c_z: int) -> int:
        """Shapes against the pair width ``c_z``; returns ``heads * head_dim``."""
        hd = int(self.q_weight.shape[0])
        if hd % self.heads:
            raise ValueError(f"q projection width {hd} is not divisible by {self.heads} heads")
        for name, shape in (("norm_weight", (c_z,)), ("norm_bias", (c_z,)), ("bias_weight", (self.heads, c_z)),
                            ("q_weight", (hd, c_z)), ("k_weight", (hd, c_z)), ("v_weight", (hd, c_z)),
                            ("g_weight", (hd, c_z)), ("o_weight", (c_z, hd))):
            _need_shape(f"tri-attn weight {name}", getattr(self, name), shape)
        return hd


@dataclass(frozen=True)
class TransitionWeights:
    """Transition weights, PyTorch ``[out, in]``: ``w_a``/``w_b`` ``[hidden, c]``
    (silu and linear branches), ``w_o`` ``[c, hidden]``; hidden is 4c in every
    port."""

    norm_weight: torch.Tensor
    norm_bias: torch.Tensor
    w_a: torch.Tensor
    w_b: torch.Tensor
    w_o: torch.Tensor

    def to(self, dtype: torch.dtype, device) -> "TransitionWeights":
        return TransitionWeights(**{f.name: _prep(getattr(self, f.name), dtype, device) for f in fields(self)})

    def check(self, c: int) -> int:
        """Shapes against the width ``c``; returns the hidden width."""
        hidden = int(self.w_a.shape[0])
        for name, shape in (("norm_weight", (c,)), ("norm_bias", (c,)), ("w_a", (hidden, c)), ("w_b", (hidden, c)),
                            ("w_o", (c, hidden))):
            _need_shape(f"transition weight {name}", getattr(self, name), shape)
        return hidden


@dataclass(frozen=True)
class SingleAttentionWeights:
    """Boltz-2 ``AttentionPairBias`` weights (PyTorch ``[out, in]``) plus the
    layer's ``pre_norm_s`` (None when the caller passes a normalised s)."""

    # fields a packed layer keeps back to back in one buffer (one projection
    # GEMM); stacking layers keeps them so (foldjax_amd.stacking)
    STACK_GROUPS: ClassVar[tuple[tuple[str, ...], ...]] = (("q_weight", "k_weight", "v_weight", "g_weight"),)

    pre_norm_weight: torch.Tensor | None
    pre_norm_bias: torch.Tensor | None
    z_norm_weight: torch.Tensor  # [c_z]
    z_norm_bias: torch.Tensor
    z_weight: torch.Tensor  # [H, c_z]
    q_weight: torch.Tensor  # [c_s, c_s]
    q_bias: torch.Tensor | None  # [c_s]
    k_weight: torch.Tensor
    v_weight: torch.Tensor
    g_weight: torch.Tensor
    o_weight: torch.Tensor

    @property
    def heads(self) -> int:
        return int(self.z_weight.shape[0])

    def to(self, dtype: torch.dtype, device) -> "SingleAttentionWeights":
        """Each weight in ``dtype`` on ``device``; q, k, v and g are stored back
        to back in one ``[4 c_s, c_s]`` buffer (the library then runs their four
        projections as one GEMM)."""
        f = {fl.name: _prep(getattr(self, fl.name), dtype, device) for fl in fields(self)}
        parts = [f[k] for k in ("q_weight", "k_weight", "v_weight", "g_weight")]
        if len({tuple(t.shape) for t in parts}) == 1:
            qkvg = torch.cat(parts, 0)
            f["q_weight"], f["k_weight"], f["v_weight"], f["g_weight"] = qkvg.chunk(4, 0)
        return SingleAttentionWeights(**f)

    def check(self, c_s: int, c_z: int | None) -> None:
        """Shapes against the single width ``c_s`` and (when z is read) the
        pair width ``c_z``."""
        for name in ("q_weight", "k_weight", "v_weight", "g_weight", "o_weight"):
            _need_shape(f"single attention weight {name}", getattr(self, name), (c_s, c_s))
        for name in ("q_bias", "pre_norm_weight", "pre_norm_bias"):
            _need_shape(f"single attention weight {name}", getattr(self, name), (c_s,))
        if c_z is not None:
            for name, shape in (("z_norm_weight", (c_z,)), ("z_norm_bias", (c_z,)), ("z_weight", (self.heads, c_z))):
                _need_shape(f"single attention weight {name}", getattr(self, name), shape)


def transition(
    x: torch.Tensor,
    w: TransitionWeights,
    *,
    row_mask: torch.Tensor | None = None,
    residual: torch.Tensor | None = None,
    eps: float = 1e-5,
    pair_bias_for: SingleAttentionWeights | None = None,
    pair_bias_eps: float = 1e-5,
    out_mask: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
):
    """``((silu(LN(x) w_a^T) * (LN(x) w_b^T)) w_o^T [* row_mask] [+ residual])
    [* (out_mask != 0)]`` over the last axis (``fjx_transition_fwd``);
    ``row_mask`` and ``out_mask`` broadcast to ``x.shape[:-1]``.

    ``pair_bias_for``: the weights of the single attention that reads this
    pair transition's output next (``x`` is then ``[..., N, N, 128]``). The
    call returns ``(out, pair_bias)``, ``pair_bias`` being that attention's
    bias ``LN_z(out) w_z^T`` (eps ``pair_bias_eps``) prepared in the
    library's ``[B, H, Np, Np]`` layout, for ``single_attention(...,
    pair_bias=...)``; with 128 channels, a 4x hidden width and at most 16
    heads it is computed in the transition's epilogue, so the pair tensor is
    not read again. The bias takes the attention's dtype: a float32
    attention over a bfloat16 pair track gets a float32 bias computed to
    float32 accuracy.

    ``out``: write the result into this tensor (x's shape, dtype and device,
    contiguous) instead of a new one; it may be ``x`` and/or ``residual``
    (in place)."""
    c = int(x.shape[-1])
    w.check(c)
    _same_device(x, row_mask=row_mask, residual=residual, out_mask=out_mask)
    if residual is not None:
        _need_shape("residual", residual, x.shape)
    if pair_bias_for is not None:
        _same_device(x, pair_bias_for=pair_bias_for.z_weight)
        _need_shape("pair-bias weight z_norm_weight", pair_bias_for.z_norm_weight, (c,))
        _need_shape("pair-bias weight z_norm_bias", pair_bias_for.z_norm_bias, (c,))
        _need_shape("pair-bias weight z_weight", pair_bias_for.z_weight, (pair_bias_for.heads, c))
    _dev(x)
    rows = x.numel() // max(c, 1)
    xf = x.contiguous()
    lib = _lib.load()
    out = _out_buffer(out, x, xf)
    pb = None
    pb_n = pb_heads = 0
    pb_f32 = False
    if pair_bias_for is not None:
        if x.dim() < 3 or x.shape[-3] != x.shape[-2]:
            raise ValueError(f"a pair-bias output needs a pair tensor [..., N, N, C], got {tuple(x.shape)}")
        pb_dtype = pair_bias_for.z_weight.dtype
        pb_f32 = pb_dtype == torch.float32 and x.dtype == torch.bfloat16
        if pb_dtype != x.dtype and not pb_f32:
            raise ValueError(f"a {pb_dtype} pair bias over a {x.dtype} transition is not supported")
        pb_n, pb_heads = int(x.shape[-2]), pair_bias_for.heads
        np_ = (pb_n + 63) // 64 * 64
        pb = torch.empty((rows // (pb_n * pb_n), pb_heads, np_, np_), dtype=pb_dtype, device=x.device)
    rm = _rows_of(row_mask, x.shape[:-1], x.dtype, "row_mask")
    om = _rows_of(out_mask, x.shape[:-1], x.dtype, "out_mask")
    res = None if residual is None else residual.to(dtype=x.dtype).contiguous()
    hidden = int(w.w_a.shape[0])
    ws_bytes = lib.fjx_transition_workspace_size(rows, c, hidden, _code(x.dtype))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    a = _lib.TransitionArgs(
        rows=rows, c=c, dtype=_code(x.dtype), eps=float(eps),
        x=_ptr(xf), norm_weight=_ptr(w.norm_weight), norm_bias=_ptr(w.norm_bias),
        w_a=_ptr(w.w_a), w_b=_ptr(w.w_b), w_o=_ptr(w.w_o),
        row_mask=_ptr(rm), residual=_ptr(res), out=_ptr(out),
        hidden=hidden, workspace=_ptr(ws), workspace_bytes=ws_bytes, out_mask=_ptr(om),
    )
    if pb is not None:
        a.pb_n, a.pb_heads, a.pb_eps = pb_n, pb_heads, float(pair_bias_eps)
        a.pb_norm_weight = _ptr(pair_bias_for.z_norm_weight)
        a.pb_norm_bias = _ptr(pair_bias_for.z_norm_bias)
        a.pb_weight = _ptr(pair_bias_for.z_weight)
        a.pb_out = _ptr(pb)
        a.pb_f32 = 1 if pb_f32 else 0
        _check_weights(pb, pair_bias_for)
    _check_weights(x, w)
    _lib.check(lib.fjx_transition_fwd(ctypes.byref(a), _stream(x)))
    return out if pb is None else (out, pb)


def single_attention(
    s: torch.Tensor,
    z: torch.Tensor | None,
    mask: torch.Tensor | None,
    w: SingleAttentionWeights,
    *,
    inf: float = 1e6,
    eps: float = 1e-5,
    residual: torch.Tensor | None = None,
    pair_bias: torch.Tensor | None = None,
    out_mask: torch.Tensor | None = None,
    extra_bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Single-track attention with pair bias (``fjx_single_attention_fwd``).
    ``s`` ``[B, N, c_s]`` (or ``[N, c_s]``), ``z`` ``[B, N, N, c_z]``, ``mask``
    ``[B, N]`` token mask. Returns the update, or ``residual + update``, times
    ``out_mask != 0`` per row when ``out_mask`` (``[B, N]``) is given.
    ``s`` and the weights share one dtype; ``z`` may be float32 or bfloat16
    independently (the Boltz-2 single track runs in float32 over a bfloat16
    pair tensor). ``pair_bias``: the bias ``transition(..., pair_bias_for=w)``
    prepared from this ``z`` in ``s``'s dtype; ``z`` is then not read (and may
    be None). ``extra_bias``: an additive bias broadcasting to ``[B, H, N, N]``
    from a 4-D tensor whose last two axes are ``[N, N]`` (Protenix's
    ``extra_attn_bias``). ``out``: write the result into this tensor (s's
    shape, dtype and device, contiguous); it may be ``s`` when ``residual`` is
    ``s`` (in place)."""
    _same_device(s, z=z, mask=mask, residual=residual, pair_bias=pair_bias, out_mask=out_mask,
                 extra_bias=extra_bias)
    if residual is not None:
        _need_shape("residual", residual, s.shape)
    w.check(int(s.shape[-1]), None if z is None else int(z.shape[-1]))
    squeeze = s.dim() == 2
    sb = s.unsqueeze(0) if squeeze else s
    batch, n, c_s = (int(v) for v in sb.shape)
    zb = None
    c_z = 0
    if z is not None:
        zb = z.unsqueeze(0) if z.dim() == 3 else z
        c_z = int(zb.shape[-1])
        if tuple(zb.shape[:3]) != (batch, n, n):
            raise ValueError(f"z must be [{batch}, {n}, {n}, c_z], got {tuple(z.shape)}")
        _code(zb.dtype)
        zb = zb.contiguous()
    if pair_bias is not None:
        np_ = (n + 63) // 64 * 64
        if (tuple(pair_bias.shape) != (batch, w.heads, np_, np_) or pair_bias.dtype != s.dtype
                or pair_bias.device != s.device or not pair_bias.is_contiguous()):
            raise ValueError(f"pair_bias must be the prepared [{batch}, {w.heads}, {np_}, {np_}] {s.dtype} bias, "
                             f"got {tuple(pair_bias.shape)} {pair_bias.dtype}")
    elif zb is None:
        raise ValueError("single_attention needs z or a prepared pair_bias")
    sb = sb.contiguous()
    mb = _rows_of(mask, (batch, n), s.dtype, "mask")
    om = _rows_of(out_mask, (batch, n), s.dtype, "out_mask")
    eb, eb_sb, eb_sh = None, 0, 0
    if extra_bias is not None:
        if extra_bias.dim() != 4 or tuple(extra_bias.shape[-2:]) != (n, n):
            raise ValueError(f"extra_bias must be a 4-D tensor [B or 1, H or 1, {n}, {n}], got {tuple(extra_bias.shape)}")
        eb = extra_bias.to(dtype=s.dtype)
        if eb.stride(-1) != 1 or eb.stride(-2) != n:
            eb = eb.contiguous()
        try:
            eb = torch.broadcast_to(eb, (batch, w.heads, n, n))
        except RuntimeError:
            raise ValueError(f"extra_bias of shape {tuple(extra_bias.shape)} does not broadcast to "
                             f"[{batch}, {w.heads}, {n}, {n}]") from None
        eb_sb, eb_sh = int(eb.stride(0)), int(eb.stride(1))
    _dev(s)
    res = None
    if residual is not None:
        res = (residual.unsqueeze(0) if squeeze else residual).to(dtype=s.dtype).contiguous()
    lib = _lib.load()
    code = _code(s.dtype)
    if out is not None and out.data_ptr() == s.data_ptr() and (residual is None or residual.data_ptr() != s.data_ptr()):
        raise ValueError("out may be s only when residual is s")
    out = _out_buffer(out, s, sb)
    ws_bytes = lib.fjx_single_attention_workspace_size(batch, n, c_s, w.heads, code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=s.device)
    a = _lib.SingleAttentionArgs(
        batch=batch, n=n, c_s=c_s, c_z=c_z, heads=w.heads, dtype=code, eps=float(eps), inf=float(inf),
        s=_ptr(sb), z=_ptr(zb), mask=_ptr(mb),
        pre_norm_weight=_ptr(w.pre_norm_weight), pre_norm_bias=_ptr(w.pre_norm_bias),
        z_norm_weight=_ptr(w.z_norm_weight), z_norm_bias=_ptr(w.z_norm_bias), z_weight=_ptr(w.z_weight),
        q_weight=_ptr(w.q_weight), q_bias=_ptr(w.q_bias), k_weight=_ptr(w.k_weight), v_weight=_ptr(w.v_weight),
        g_weight=_ptr(w.g_weight), o_weight=_ptr(w.o_weight),
        residual=_ptr(res), out=_ptr(out), workspace=_ptr(ws), workspace_bytes=ws_bytes,
        pair_bias=_ptr(pair_bias), z_dtype=_code(s.dtype if zb is None else zb.dtype), out_mask=_ptr(om),
        extra_bias=_ptr(eb), extra_bias_stride_b=eb_sb, extra_bias_stride_h=eb_sh,
    )
    _check_weights(s, w)
    _lib.check(lib.fjx_single_attention_fwd(ctypes.byref(a), _stream(s)))
    return out[0] if squeeze else out


def _out_buffer(out: torch.Tensor | None, x: torch.Tensor, flat: torch.Tensor) -> torch.Tensor:
    """The output buffer of a call on ``x`` (flattened as ``flat``): a new
    tensor, or the caller's ``out``, which must be a contiguous tensor of x's
    shape, dtype and device and may be x itself and/or the residual (every
    kernel reads an output position's inputs before it writes it, and only
    the workgroup that writes a position reads it)."""
    if out is None:
        return torch.empty_like(flat)
    if tuple(out.shape) != tuple(x.shape) or out.dtype != x.dtype or out.device != x.device:
        raise ValueError(f"out must be a {x.dtype} tensor of shape {tuple(x.shape)} on {x.device}, "
                         f"got {out.dtype} {tuple(out.shape)} on {out.device}")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    return out.reshape(flat.shape)


def _flatten_pair(x: torch.Tensor, mask: torch.Tensor | None):
    if x.dim() < 3:
        raise ValueError(f"pair tensor must be [..., N, N, C], got shape {tuple(x.shape)}")
    _same_device(x, mask=mask)
    n, n2, c = x.shape[-3:]
    if n != n2:
        raise ValueError(f"pair tensor must be square in its two pair axes, got {tuple(x.shape)}")
    lead = x.shape[:-3]
    batch = 1
    for s in lead:
        batch *= int(s)
    xf = x.contiguous().reshape(batch, n, n, c)
    mf = None
    if mask is not None:
        if tuple(mask.shape[-2:]) != (n, n):
            raise ValueError(f"mask must be [..., {n}, {n}], got {tuple(mask.shape)}")
        mf = torch.broadcast_to(mask, tuple(lead) + (n, n)).to(dtype=x.dtype).contiguous().reshape(batch, n, n)
    return xf, mf, lead, batch, n, c


def trimul(
    x: torch.Tensor,
    mask: torch.Tensor | None,
    w: TriMulWeights,
    direction: str,
    eps: float = 1e-5,
    residual: torch.Tensor | None = None,
    *,
    no_alloc: bool = False,
    out_mask: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Triangle multiplicative update (``fjx_trimul_fwd``); returns the update,
    or ``residual + update`` when ``residual`` is given, times
    ``out_mask != 0`` per position when ``out_mask`` (``[..., N, N]``) is given.

    ``no_alloc``: run ``fjx_trimul_fwd_noalloc`` instead, whose workspace is
    the library's static per-GPU scratch (shapes up to
    ``_lib.NOALLOC_SCRATCH_BYTES`` of workspace; calls on one GPU must not
    overlap). Only the output is allocated here, unless ``out`` is given:
    the result then goes into that tensor (x's shape, dtype and device,
    contiguous), which may be ``x`` and/or ``residual`` (in place)."""
    if direction not in ("outgoing", "incoming"):
        raise ValueError(f"Unsupported triangle multiplication direction: {direction!r}")
    _same_device(x, residual=residual, out_mask=out_mask)
    if residual is not None:
        _need_shape("residual", residual, x.shape)
    c_h = w.check(int(x.shape[-1]))
    xf, mf, lead, batch, n, c = _flatten_pair(x, mask)
    om = _rows_of(out_mask, x.shape[:-1], x.dtype, "out_mask")
    _dev(x)
    lib = _lib.load()
    code = _code(x.dtype)
    out = _out_buffer(out, x, xf)
    res = None if residual is None else residual.to(dtype=x.dtype).contiguous().reshape(batch, n, n, c)
    ws_bytes = 0 if no_alloc else lib.fjx_trimul_workspace_size(batch, n, c, c_h, code)
    ws = None if no_alloc else torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    a = _lib.TriMulArgs(
        batch=batch, n=n, c_z=c, c_h=c_h,
        direction=_lib.FJX_OUTGOING if direction == "outgoing" else _lib.FJX_INCOMING,
        dtype=code, eps=float(eps),
        x=_ptr(xf), mask=_ptr(mf),
        norm_in_weight=_ptr(w.norm_in_weight), norm_in_bias=_ptr(w.norm_in_bias),
        p_in_weight=_ptr(w.p_in_weight), g_in_weight=_ptr(w.g_in_weight),
        norm_out_weight=_ptr(w.norm_out_weight), norm_out_bias=_ptr(w.norm_out_bias),
        p_out_weight=_ptr(w.p_out_weight), g_out_weight=_ptr(w.g_out_weight),
        residual=_ptr(res), out=_ptr(out),
        workspace=_ptr(ws), workspace_bytes=ws_bytes, out_mask=_ptr(om),
    )
    _check_weights(x, w)
    entry = lib.fjx_trimul_fwd_noalloc if no_alloc else lib.fjx_trimul_fwd
    _lib.check(entry(ctypes.byref(a), _stream(x)))
    return out.reshape(tuple(lead) + (n, n, c))


def triattn(
    x: torch.Tensor,
    mask: torch.Tensor | None,
    w: TriAttnWeights,
    starting: bool = True,
    inf: float = 1e9,
    eps: float = 1e-5,
    residual: torch.Tensor | None = None,
    out_mask: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Triangle attention, starting or ending node (``fjx_triattn_fwd``);
    ``out_mask`` (``[..., N, N]``, indexed like the output) and ``out`` (may
    be ``x`` and/or ``residual``: in place) as for ``trimul``."""
    _same_device(x, residual=residual, out_mask=out_mask)
    if residual is not None:
        _need_shape("residual", residual, x.shape)
    hd = w.check(int(x.shape[-1]))
    heads = w.heads
    xf, mf, lead, batch, n, c = _flatten_pair(x, mask)
    om = _rows_of(out_mask, x.shape[:-1], x.dtype, "out_mask")
    _dev(x)
    lib = _lib.load()
    code = _code(x.dtype)
    out = _out_buffer(out, x, xf)
    res = None if residual is None else residual.to(dtype=x.dtype).contiguous().reshape(batch, n, n, c)
    ws_bytes = lib.fjx_triattn_workspace_size(batch, n, c, heads, hd // heads, code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    a = _lib.TriAttnArgs(
        batch=batch, n=n, c_z=c, heads=heads, head_dim=hd // heads,
        starting=1 if starting else 0, dtype=code, eps=float(eps), inf=float(inf),
        x=_ptr(xf), mask=_ptr(mf),
        norm_weight=_ptr(w.norm_weight), norm_bias=_ptr(w.norm_bias), bias_weight=_ptr(w.bias_weight),
        q_weight=_ptr(w.q_weight), k_weight=_ptr(w.k_weight), v_weight=_ptr(w.v_weight),
        g_weight=_ptr(w.g_weight), o_weight=_ptr(w.o_weight),
        residual=_ptr(res), out=_ptr(out),
        workspace=_ptr(ws), workspace_bytes=ws_bytes, out_mask=_ptr(om),
    )
    _check_weights(x, w)
    _lib.check(lib.fjx_triattn_fwd(ctypes.byref(a), _stream(x)))
    return out.reshape(tuple(lead) + (n, n, c))


def triattn_core(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    tri_bias: torch.Tensor,
    mask_bias: torch.Tensor | None,
    *,
    scale: float,
) -> torch.Tensor:
    """``cueq_attention_core`` semantics (``src/foldjax/models/_cueq.py:66-121``).

    q/k/v ``[..., I, H, J, D]``; ``tri_bias`` ``[..., 1, H, J, J]``; additive
    ``mask_bias`` ``[..., I, 1, 1, J]`` (or None); ``scale`` applied inside.
    Leading axes are broadcast and folded into one batch axis.
    """
    _same_device(q, k=k, v=v, tri_bias=tri_bias, mask_bias=mask_bias)
    if q.dim() < 4 or k.shape[-4:] != q.shape[-4:] or v.shape[-4:] != q.shape[-4:]:
        raise ValueError(f"q, k, v must share [..., I, H, J, D], got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if tri_bias.dim() < 4 or tuple(tri_bias.shape[-3:]) != (q.shape[-3], q.shape[-2], q.shape[-2]):
        raise ValueError(f"tri_bias must be [..., 1, H, J, J] for q {tuple(q.shape)}, got {tuple(tri_bias.shape)}")
    if mask_bias is not None and (mask_bias.dim() < 4 or tuple(mask_bias.shape[-4:]) not in
                                  ((q.shape[-4], 1, 1, q.shape[-2]), (1, 1, 1, q.shape[-2]))):
        raise ValueError(f"mask_bias must be [..., I, 1, 1, J] for q {tuple(q.shape)}, got {tuple(mask_bias.shape)}")
    _dev(q)
    lead = torch.broadcast_shapes(q.shape[:-4], tri_bias.shape[:-4],
                                  () if mask_bias is None else mask_bias.shape[:-4])
    rows, heads, n, d = q.shape[-4:]
    batch = 1
    for s in lead:
        batch *= int(s)
    dt = q.dtype

    def fold(t, shape):
        return torch.broadcast_to(t, tuple(lead) + tuple(shape)).to(dtype=dt).contiguous().reshape((batch,) + tuple(shape))

    qf = fold(q, (rows, heads, n, d))
    kf = fold(k, (rows, heads, n, d))
    vf = fold(v, (rows, heads, n, d))
    if tri_bias.shape[-4] != 1:
        raise ValueError("tri_bias must be [..., 1, H, J, J]: the kernel shares one bias across rows")
    bf = fold(tri_bias, (1, heads, n, n)).reshape(batch, heads, n, n)
    mb = None
    if mask_bias is not None:
        mb = torch.broadcast_to(mask_bias, tuple(lead) + (rows, 1, 1, n)).to(torch.float32).contiguous()
        mb = mb.reshape(batch, rows, n)
    lib = _lib.load()
    code = _code(dt)
    out = torch.empty_like(qf)
    ws_bytes = lib.fjx_triattn_core_workspace_size(batch, rows, heads, n, d, code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    a = _lib.TriAttnCoreArgs(
        batch=batch, rows=rows, heads=heads, n=n, head_dim=d, dtype=code, scale=float(scale),
        q=_ptr(qf), k=_ptr(kf), v=_ptr(vf), tri_bias=_ptr(bf), mask_bias=_ptr(mb),
        out=_ptr(out), workspace=_ptr(ws), workspace_bytes=ws_bytes,
    )
    _lib.check(lib.fjx_triattn_core(ctypes.byref(a), _stream(q)))
    return out.reshape(tuple(lead) + (rows, heads, n, d))


def _check_weights(x: torch.Tensor, w) -> None:
    for f in fields(w):
        t = getattr(w, f.name)
        if t is None:
            continue
        if t.dtype != x.dtype or t.device != x.device or not t.is_contiguous():
            raise ValueError(
                f"weight {f.name} must be a contiguous {x.dtype} tensor on {x.device}; "
                "pack weights with .to(dtype, device) first"
            )
