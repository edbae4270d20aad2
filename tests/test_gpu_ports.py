"""GPU parity of the Protenix and OpenFold3 single attention with pair bias,
their Pairformer blocks and stacks, the fused output masks, and the float32
single track over a bfloat16 pair tensor (Boltz-2's precision split).

Each case compares the HIP path with the float64 oracle on the same
(bf16-rounded in bf16 mode) inputs: max-abs 1e-4 in fp32, relative 2e-2 in
bf16. The oracle functions used here are pinned in tests/test_oracle.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from foldjax_amd import boltz2, kernels, openfold3, protenix
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn
from foldjax_amd.pairformer import PairformerLayerWeights
from foldjax_amd.stacking import StackedLayers
from oracle import triangle as O
from tests.gpu_util import FP32_MAX_ABS, assert_parity, device_tensor, max_abs, prep, prep_tree, say, to_np
from tests.port_fields import of3_apb_fields, of3_block_fields, px_apb_fields, px_block_fields

pytestmark = pytest.mark.gpu

DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16}


def _holey_pair_mask(n, n_real):
    """A token pair mask with one extra hole between valid tokens and one
    fractional entry (gated as True)."""
    pm = syn.pair_mask(n, n_real)
    pm[1, 3] = 0.0
    pm[2, 4] = 0.5
    return pm[None]


# ------------------------------------------------------ attention with pair bias


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("extra", ["none", "keys", "dense"])
def test_protenix_attention_pair_bias(dt, extra):
    dtype = DTYPES[dt]
    n, n_real, h = 50, 44, 16
    say(f"protenix attention_pair_bias n={n} extra={extra} {dt}")
    rng = np.random.default_rng(60)
    s = syn.single_input(n, 384, seed=61, batch=1)
    z = syn.pair_input(n, 128, seed=62, batch=1)
    w = syn.single_attention_weights(heads=h, seed=63)
    valid = syn.token_mask(n, n_real)
    e = None
    if extra == "keys":  # the block's form, rank 2: [N, N]
        e = np.where(valid[:, None] * valid[None, :] > 0, 0.0, -1e10).astype(np.float32)
    elif extra == "dense":  # a general [B, H, N, N] bias
        e = (0.5 * rng.standard_normal((1, h, n, n))).astype(np.float32)
    got = protenix.attention_pair_bias(device_tensor(s, dtype), None, device_tensor(z, dtype),
                                       P.single_attention_to_protenix(w), num_heads=h,
                                       extra_attn_bias=None if e is None else device_tensor(e, dtype))
    torch.cuda.synchronize()
    want = O.protenix_attention_pair_bias(prep(s, dtype), prep(z, dtype), px_apb_fields(prep_tree(w, dtype)),
                                          num_heads=h, extra_attn_bias=None if e is None else prep(e, dtype))
    rows = slice(0, n_real) if extra == "keys" else slice(0, n)
    assert_parity(to_np(got)[:, rows], want[:, rows], dtype, f"protenix apb extra={extra}")


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("n,n_real", [(37, 37), (70, 61)])
def test_openfold3_attention_pair_bias(dt, n, n_real):
    dtype = DTYPES[dt]
    say(f"openfold3 attention_pair_bias n={n} {dt}")
    s = syn.single_input(n, 384, seed=64, batch=1)
    z = syn.pair_input(n, 128, seed=65, batch=1)
    m = syn.token_mask(n, n_real)[None]
    w = syn.single_attention_weights(heads=16, seed=66)
    st = device_tensor(s, dtype)
    got = openfold3.attention_pair_bias(st, device_tensor(z, dtype), P.single_attention_to_openfold3(w), no_heads=16,
                                        mask=device_tensor(m, dtype), residual=st)
    torch.cuda.synchronize()
    want = prep(s, dtype) + O.openfold3_attention_pair_bias(prep(s, dtype), prep(z, dtype),
                                                            of3_apb_fields(prep_tree(w, dtype)), no_heads=16, mask=m)
    assert_parity(to_np(got), want, dtype, "openfold3 apb")


def test_single_attention_fp32_over_bf16_pair():
    """Boltz-2's precision split (``B2K/pairformer.py:182-199``): a float32 s
    and float32 weights over a bfloat16 z. The bias is computed in float32
    from z's bf16 values, so the bar is the fp32 one against the oracle on
    those values."""
    n, n_real = 60, 52
    say(f"single attention fp32 s over bf16 z n={n}")
    s = syn.single_input(n, 384, seed=67, batch=1)
    z = prep(syn.pair_input(n, 128, seed=68, batch=1), torch.bfloat16)
    m = syn.token_mask(n, n_real)[None]
    w = syn.single_attention_weights(seed=69)
    att, pre = P.single_attention_to_boltz2(w)
    packed = P.pack_single_attention_boltz2(att, torch.float32, "cuda", pre_norm=pre)
    st = device_tensor(s, torch.float32)
    got = kernels.single_attention(st, device_tensor(z, torch.bfloat16), device_tensor(m, torch.float32), packed,
                                   residual=st)
    torch.cuda.synchronize()
    s_ln = O.layer_norm(s, w["pre_norm_s"]["weight"], w["pre_norm_s"]["bias"])
    want = s + O.boltz2_attention_pair_bias(w, s_ln, z, m)
    assert got.dtype == torch.float32
    assert_parity(to_np(got), want, torch.float32, "fp32 single attention over bf16 z")


# ------------------------------------------------------------- output masks


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("c,c_h,heads", [(128, 128, 4), (64, 128, 4), (64, 64, 2)])
def test_out_mask_gates_every_pair_kernel(dt, c, c_h, heads):
    """``out_mask`` multiplies each written position by ``out_mask != 0``,
    residual included: the gated call equals the ungated one with the masked
    positions zeroed, bit for bit (fused kernels at c=128, their narrow forms
    at c=64 with c_h=128 and 4 heads, the general-width paths at c_h=64 and
    2 heads)."""
    dtype = DTYPES[dt]
    n = 33
    say(f"out_mask pair kernels c={c} c_h={c_h} heads={heads} n={n} {dt}")
    z = device_tensor(syn.pair_input(n, c, seed=70, batch=1), dtype)
    pm = device_tensor(_holey_pair_mask(n, 29), dtype)
    keep = (pm != 0)[..., None]
    tm = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(c, c_h, seed=71)), dtype, "cuda")
    ta = P.pack_triattn_protenix(P.triattn_to_protenix(syn.triattn_weights(c, heads, 32, seed=72)), dtype, "cuda")
    tr = P.pack_transition_torch(P.transition_to_protenix(syn.transition_weights(c, seed=73)), dtype, "cuda")
    cases = [
        ("trimul out", lambda **k: kernels.trimul(z, pm, tm, "outgoing", residual=z, **k)),
        ("trimul in", lambda **k: kernels.trimul(z, pm, tm, "incoming", residual=z, **k)),
        ("triattn start", lambda **k: kernels.triattn(z, pm, ta, starting=True, residual=z, **k)),
        ("triattn end", lambda **k: kernels.triattn(z, pm, ta, starting=False, residual=z, **k)),
        ("transition", lambda **k: kernels.transition(z, tr, residual=z, **k)),
    ]
    for name, f in cases:
        plain = f()
        gated = f(out_mask=pm)
        torch.cuda.synchronize()
        assert torch.equal(gated, torch.where(keep, plain, torch.zeros_like(plain))), name
        assert not gated[0, 1, 3].any() and gated[0, 2, 4].abs().sum() > 0, name


def test_out_mask_gates_single_track():
    dtype = torch.bfloat16
    n = 45
    say(f"out_mask single track n={n}")
    s = device_tensor(syn.single_input(n, 384, seed=74, batch=1), dtype)
    z = device_tensor(syn.pair_input(n, 128, seed=75, batch=1), dtype)
    valid = device_tensor(syn.token_mask(n, 40)[None], dtype)
    w = syn.single_attention_weights(seed=76)
    att = P.pack_single_attention_protenix(P.single_attention_to_protenix(w), dtype, "cuda")
    tr = P.pack_transition_torch(P.transition_to_protenix(syn.transition_weights(384, seed=77)), dtype, "cuda")
    keep = (valid != 0)[..., None]
    plain = kernels.single_attention(s, z, valid, att, residual=s)
    gated = kernels.single_attention(s, z, valid, att, residual=s, out_mask=valid)
    tp = kernels.transition(s, tr, residual=s)
    tg = kernels.transition(s, tr, residual=s, out_mask=valid)
    torch.cuda.synchronize()
    assert torch.equal(gated, torch.where(keep, plain, torch.zeros_like(plain)))
    assert torch.equal(tg, torch.where(keep, tp, torch.zeros_like(tp)))


# ------------------------------------------------------------ Protenix blocks


def _px_oracle_block(w, s, z, pm, dtype):
    return O.protenix_pairformer_block(None if s is None else prep(s, dtype), prep(z, dtype), pm,
                                       px_block_fields(prep_tree(w, dtype)))


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("mask", ["padded", "holey", "none"])
def test_protenix_pairformer_block(dt, mask):
    dtype = DTYPES[dt]
    n, n_real = 40, 35
    say(f"protenix pairformer_block n={n} mask={mask} {dt}")
    w = syn.pairformer_layer_weights(seed=80)
    s = syn.single_input(n, 384, seed=81, batch=1)
    z = syn.pair_input(n, 128, seed=82, batch=1)
    pm = None
    if mask != "none":
        pm = syn.pair_mask(n, n_real)[None] if mask == "padded" else _holey_pair_mask(n, n_real)
        # adversarial padded tokens (``T/models/protenix/test_pairformer.py:91-132``)
        s[:, n_real:] = 1e3
        z[:, n_real:] = -1e3
        z[:, :, n_real:] = 1e3
    gs, gz = protenix.pairformer_block(device_tensor(s, dtype), device_tensor(z, dtype),
                                       None if pm is None else device_tensor(pm, dtype),
                                       P.pairformer_block_to_protenix(w))
    torch.cuda.synchronize()
    ws, wz = _px_oracle_block(w, s, z, pm, dtype)
    v = slice(0, n if pm is None else n_real)
    assert_parity(to_np(gz)[:, v, v], wz[:, v, v], dtype, "protenix block z")
    assert_parity(to_np(gs)[:, v], ws[:, v], dtype, "protenix block s")
    if pm is not None:
        gzn, gsn = to_np(gz), to_np(gs)
        assert not gzn[:, n_real:].any() and not gzn[:, :, n_real:].any() and not gsn[:, n_real:].any()
        if mask == "holey":
            assert not gzn[0, 1, 3].any()


def test_protenix_pairformer_block_without_single_track():
    """A block with no ``attention_pair_bias`` (the MSA and template stacks'
    form) updates z only and returns s gated by the pair mask's diagonal."""
    dtype = torch.bfloat16
    n, n_real = 36, 30
    say(f"protenix pair-only block n={n}")
    w = syn.pairformer_layer_weights(seed=83)
    z = syn.pair_input(n, 128, seed=84, batch=1)
    s = syn.single_input(n, 384, seed=85, batch=1)
    pm = syn.pair_mask(n, n_real)[None]
    p = P.pairformer_block_to_protenix(w)._replace(attention_pair_bias=None, single_transition=None)
    gs, gz = protenix.pairformer_block(device_tensor(s, dtype), device_tensor(z, dtype), device_tensor(pm, dtype), p)
    torch.cuda.synchronize()
    fields = px_block_fields(prep_tree(w, dtype))
    fields["attention_pair_bias"] = None
    ws, wz = O.protenix_pairformer_block(prep(s, dtype), prep(z, dtype), pm, fields)
    assert_parity(to_np(gz), wz, dtype, "pair-only block z")
    np.testing.assert_array_equal(to_np(gs), ws)


def test_protenix_pairformer_stack_two_blocks():
    """Two blocks: the stack equals the oracle block applied twice; scanned
    (stacked weights) and unrolled runs give identical bits."""
    dtype = torch.bfloat16
    n, n_real = 36, 33
    say(f"protenix pairformer_stack 2 blocks n={n}")
    ws_ = [syn.pairformer_layer_weights(seed=90), syn.pairformer_layer_weights(seed=100)]
    s = syn.single_input(n, 384, seed=91, batch=1)
    z = syn.pair_input(n, 128, seed=92, batch=1)
    pm = syn.pair_mask(n, n_real)[None]
    params = protenix.PairformerStackParams(blocks=tuple(P.pairformer_block_to_protenix(w) for w in ws_))
    args = (device_tensor(s, dtype), device_tensor(z, dtype), device_tensor(pm, dtype))
    gs, gz = protenix.pairformer_stack(*args, params, use_scan=True)
    us, uz = protenix.pairformer_stack(*args, params, use_scan=False)
    stacked = protenix.stack_pairformer_block_params(params.blocks, dtype, "cuda")
    ss, sz = protenix.pairformer_stack(*args, stacked)
    torch.cuda.synchronize()
    assert isinstance(stacked, StackedLayers) and len(stacked) == 2
    assert torch.equal(gs, us) and torch.equal(gz, uz) and torch.equal(gs, ss) and torch.equal(gz, sz)
    es, ez = prep(s, dtype), prep(z, dtype)
    for w in ws_:
        es, ez = O.protenix_pairformer_block(es, ez, pm, px_block_fields(prep_tree(w, dtype)))
    v = slice(0, n_real)
    assert_parity(to_np(gz)[:, v, v], ez[:, v, v], dtype, "protenix stack z")
    assert_parity(to_np(gs)[:, v], es[:, v], dtype, "protenix stack s")


# ----------------------------------------------------------- OpenFold3 blocks


@pytest.mark.parametrize("dt,mask_transition", [("fp32", True), ("bf16", True), ("bf16", False)])
def test_openfold3_pairformer_block(dt, mask_transition):
    dtype = DTYPES[dt]
    n, n_real = 38, 33
    say(f"openfold3 pairformer_block n={n} mask_transition={mask_transition} {dt}")
    w = syn.pairformer_layer_weights(seed=110)
    s = syn.single_input(n, 384, seed=111, batch=1)
    z = syn.pair_input(n, 128, seed=112, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    gs, gz = openfold3.pairformer_block(device_tensor(s, dtype), device_tensor(z, dtype),
                                        P.pairformer_block_to_openfold3(w), single_mask=device_tensor(tm, dtype),
                                        pair_mask=device_tensor(pm, dtype), no_heads_pair=4, no_heads_pair_bias=16,
                                        mask_transition=mask_transition)
    torch.cuda.synchronize()
    ws, wz = O.openfold3_pairformer_block(prep(s, dtype), prep(z, dtype), of3_block_fields(prep_tree(w, dtype)),
                                          single_mask=tm, pair_mask=pm, no_heads_pair=4, no_heads_pair_bias=16,
                                          mask_transition=mask_transition)
    v = slice(0, n_real)
    assert_parity(to_np(gz)[:, v, v], wz[:, v, v], dtype, "openfold3 block z")
    assert_parity(to_np(gs)[:, v], ws[:, v], dtype, "openfold3 block s")
    with pytest.raises(ValueError, match="no_heads_pair_bias"):
        openfold3.pairformer_block(device_tensor(s, dtype), device_tensor(z, dtype),
                                   P.pairformer_block_to_openfold3(w), single_mask=device_tensor(tm, dtype),
                                   pair_mask=device_tensor(pm, dtype), no_heads_pair=4, no_heads_pair_bias=8)


def test_openfold3_pairformer_stack():
    dtype = torch.bfloat16
    n, n_real = 34, 30
    say(f"openfold3 pairformer_stack 2 blocks n={n}")
    ws_ = [syn.pairformer_layer_weights(seed=120), syn.pairformer_layer_weights(seed=130)]
    s = syn.single_input(n, 384, seed=121, batch=1)
    z = syn.pair_input(n, 128, seed=122, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    params = openfold3.PairformerStackParams(blocks=tuple(P.pairformer_block_to_openfold3(w) for w in ws_))
    kw = dict(single_mask=device_tensor(tm, dtype), pair_mask=device_tensor(pm, dtype), no_heads_pair=4,
              no_heads_pair_bias=16)
    gs, gz = openfold3.pairformer_stack(device_tensor(s, dtype), device_tensor(z, dtype), params, **kw)
    us, uz = openfold3.pairformer_stack(device_tensor(s, dtype), device_tensor(z, dtype), params, scan_blocks=False,
                                        **kw)
    torch.cuda.synchronize()
    assert torch.equal(gs, us) and torch.equal(gz, uz)
    es, ez = prep(s, dtype), prep(z, dtype)
    for w in ws_:
        es, ez = O.openfold3_pairformer_block(es, ez, of3_block_fields(prep_tree(w, dtype)), single_mask=tm,
                                              pair_mask=pm, no_heads_pair=4, no_heads_pair_bias=16)
    v = slice(0, n_real)
    assert_parity(to_np(gz)[:, v, v], ez[:, v, v], dtype, "openfold3 stack z")
    assert_parity(to_np(gs)[:, v], es[:, v], dtype, "openfold3 stack s")


# ------------------------------------------- Boltz-2 layer with an fp32 s track


def test_boltz2_layer_fp32_single_track():
    """The Boltz-2 layer as the reference runs it in bf16: the pair track in
    bf16, s and the single-track weights in fp32 (``B2K/pairformer.py:182-199``).
    The pair track meets the bf16 bar; the s track carries the pair track's
    bf16 error through the bias, so it meets the bf16 bar too, and it is
    checked to be float32 and closer to the oracle than the all-bf16 run."""
    n, n_real = 44, 40
    say(f"boltz2 layer fp32 single track n={n}")
    w = syn.pairformer_layer_weights(seed=140)
    s = syn.single_input(n, 384, seed=141, batch=1)
    z = syn.pair_input(n, 128, seed=142, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    bf = torch.bfloat16
    mixed = PairformerLayerWeights.from_fields(w, bf, "cuda", single_dtype=torch.float32)
    gs, gz = mixed.forward(device_tensor(s, torch.float32), device_tensor(z, bf), device_tensor(tm, torch.float32),
                           device_tensor(pm, bf))
    flat = PairformerLayerWeights.from_fields(w, bf, "cuda")
    fs, fz = flat.forward(device_tensor(s, bf), device_tensor(z, bf), device_tensor(tm, bf), device_tensor(pm, bf))
    bs, bz = boltz2.pairformer_layer_forward(P.pairformer_layer_to_boltz2(w), device_tensor(s, torch.float32),
                                             device_tensor(z, bf), device_tensor(tm, torch.float32),
                                             device_tensor(pm, bf))
    torch.cuda.synchronize()
    assert gs.dtype == torch.float32 and gz.dtype == bf
    assert torch.equal(bs, gs) and torch.equal(bz, gz)
    assert torch.equal(gz, fz)  # the pair track does not depend on the single track
    # oracle: bf16-valued pair-track weights and inputs, fp32 single-track weights
    wr = dict(w)
    for k in ("tri_mul_out", "tri_mul_in", "tri_att_start", "tri_att_end", "transition_z"):
        wr[k] = prep_tree(w[k], bf)
    ws, wz = O.boltz2_pairformer_layer(wr, s, prep(z, bf), tm, pm)
    v = slice(0, n_real)
    assert_parity(to_np(gz)[:, v, v], wz[:, v, v], bf, "mixed layer z")
    err_mixed = assert_parity(to_np(gs)[:, v], ws[:, v], bf, "mixed layer s")
    err_flat = assert_parity(to_np(fs)[:, v], ws[:, v], bf, "bf16 layer s")
    assert err_mixed < err_flat, (err_mixed, err_flat)


def test_boltz2_fp32_single_track_attention_against_fp32_bar():
    """Given the layer's own bf16 z, the fp32 single-track attention and
    transition meet the fp32 bar (max-abs 1e-4) against the oracle."""
    n, n_real = 44, 40
    say(f"boltz2 fp32 single track on a given z n={n}")
    w = syn.pairformer_layer_weights(seed=150)
    s = syn.single_input(n, 384, seed=151, batch=1)
    z = prep(syn.pair_input(n, 128, seed=152, batch=1), torch.bfloat16)
    tm = syn.token_mask(n, n_real)[None]
    layer = PairformerLayerWeights.from_fields(w, torch.bfloat16, "cuda", single_dtype=torch.float32)
    st = device_tensor(s, torch.float32)
    got = kernels.single_attention(st, device_tensor(z, torch.bfloat16), device_tensor(tm, torch.float32),
                                   layer.attention, residual=st)
    got = kernels.transition(got, layer.transition_s, residual=got)
    torch.cuda.synchronize()
    a = w["attention"]
    s_ln = O.layer_norm(s, a["pre_norm_s"]["weight"], a["pre_norm_s"]["bias"])
    want = s + O.boltz2_attention_pair_bias(a, s_ln, z, tm)
    want = want + O.transition(want, w["transition_s"])
    err = max_abs(to_np(got), want)
    assert err <= FP32_MAX_ABS, err


@pytest.mark.parametrize("n,heads,expansion", [(64, 16, 4), (37, 16, 4), (24, 24, 4), (24, 16, 2)])
def test_transition_fp32_pair_bias_over_bf16(n, heads, expansion):
    """A bf16 pair transition preparing the bias of an fp32 attention (the
    Boltz-2 precision split): the bias is LN_z(out) w_z^T of the transition's
    own bf16 output to the fp32 bar, zero on the padded border, and the
    attention fed it agrees with the one that reads z itself (fused epilogue
    at 16 heads and a 4x width; the separate pass otherwise)."""
    say(f"transition fp32 pair bias over bf16 n={n} heads={heads} x{expansion}")
    bf = torch.bfloat16
    z = syn.pair_input(n, 128, seed=160, batch=1)
    s = syn.single_input(n, 384, seed=161, batch=1)
    mask = syn.token_mask(n, n - 2)[None]
    tr = syn.transition_weights(128, expansion, seed=162)
    tw = P.pack_transition_torch(P.transition_to_protenix(tr), bf, "cuda")
    w = syn.single_attention_weights(heads=heads, seed=163)
    att, pre = P.single_attention_to_boltz2(w)
    att32 = P.pack_single_attention_boltz2(att, torch.float32, "cuda", pre_norm=pre)
    zt = device_tensor(z, bf)
    plain = kernels.transition(zt, tw, residual=zt)
    out, pb = kernels.transition(zt, tw, residual=zt, pair_bias_for=att32)
    torch.cuda.synchronize()
    assert torch.equal(out, plain) and pb.dtype == torch.float32
    np_ = (n + 63) // 64 * 64
    pbn = to_np(pb)
    assert not pbn[:, :, n:, :].any() and not pbn[:, :, :, n:].any()
    ln = O.layer_norm(to_np(out), w["proj_z_norm"]["weight"], w["proj_z_norm"]["bias"])
    want = np.transpose(O.linear_torch(ln, {"weight": w["proj_z"]["weight"]}), (0, 3, 1, 2)) * np.log2(np.e)
    err = max_abs(pbn[:, :, :n, :n], want)
    assert err <= FP32_MAX_ABS, f"fp32 pair bias max-abs {err:.2e}"
    st, mt = device_tensor(s, torch.float32), device_tensor(mask, torch.float32)
    ref = kernels.single_attention(st, out, mt, att32, residual=st)
    got = kernels.single_attention(st, None, mt, att32, residual=st, pair_bias=pb)
    torch.cuda.synchronize()
    err = max_abs(to_np(got), to_np(ref))
    assert err <= FP32_MAX_ABS, f"attention with the prepared fp32 bias: max-abs {err:.2e}"
