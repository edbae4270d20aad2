"""GPU parity of the rest of the Pairformer block (pair/single transition,
single attention with pair bias) and of one full layer, against the CPU
oracle on the same values (fp32: max-abs <= 1e-4; bf16: relative <= 2e-2)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from foldjax_amd import boltz2, kernels, openfold3, protenix
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn
from foldjax_amd.pairformer import PairformerLayerWeights
from oracle import triangle as O
from tests.gpu_util import assert_parity, device_tensor, prep, prep_tree, say, spike_rows, to_np

pytestmark = pytest.mark.gpu

DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16}


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("c,rows", [(128, 1), (128, 200), (384, 70)])
def test_transition_parity(dt, c, rows):
    dtype = DTYPES[dt]
    say(f"transition c={c} rows={rows} {dt}")
    rng = np.random.default_rng(c + rows)
    x = rng.standard_normal((rows, c)).astype(np.float32)
    w = syn.transition_weights(c, seed=rows)
    got = protenix.transition(device_tensor(x, dtype), _protenix_transition(w), residual=device_tensor(x, dtype))
    torch.cuda.synchronize()
    xr = prep(x, dtype)
    want = xr + O.transition(xr, prep_tree(w, dtype))
    assert_parity(to_np(got), want, dtype, f"transition c={c}")


def test_transition_spike_rows_bf16():
    """Rows whose mean dwarfs their spread, where the LayerNorm's one-pass
    statistics E[x^2] - mean^2 cancel most (the bf16 LayerNorm takes them on
    dot2 instructions and switches to the two-pass variance past a ratio of
    64): each such row's update stays at the bf16 bar on its own."""
    dtype = torch.bfloat16
    say("transition spike rows bf16")
    rng = np.random.default_rng(11)
    x = spike_rows(rng, 96)
    w = syn.transition_weights(128, seed=11)
    got = protenix.transition(device_tensor(x, dtype), _protenix_transition(w))
    torch.cuda.synchronize()
    want = O.transition(prep(x, dtype), prep_tree(w, dtype))
    g = to_np(got)
    for r in range(0, 96, 2):
        assert_parity(g[r], want[r], dtype, f"transition spike row {r}")
    assert_parity(g, want, dtype, "transition spike rows")


def _protenix_transition(w):
    return {"layer_norm": w["layer_norm"], "linear_a": w["linear_a"], "linear_b": w["linear_b"],
            "linear_out": w["linear_out"]}


def test_transition_ports_agree_and_mask():
    say("transition ports n=20 bf16")
    dtype = torch.bfloat16
    z = device_tensor(syn.pair_input(20, 128, seed=3), dtype)
    w = syn.transition_weights(128, seed=4)
    a = protenix.transition(z, _protenix_transition(w))
    b = boltz2.transition_forward(P.transition_to_boltz2(w), z)
    of3 = {"layer_norm": w["layer_norm"], "swiglu": {"linear_a": w["linear_a"], "linear_b": w["linear_b"]},
           "linear_out": w["linear_out"]}
    c = openfold3.swiglu_transition(z, of3)
    assert torch.equal(a, b) and torch.equal(a, c)
    m = device_tensor(syn.pair_mask(20, 15), dtype)
    cm = openfold3.swiglu_transition(z, of3, mask=m)
    assert torch.equal(cm, a * m[..., None])


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("n,n_real", [(37, 37), (100, 90)])
def test_single_attention_parity(dt, n, n_real):
    dtype = DTYPES[dt]
    say(f"single attention n={n} {dt}")
    s = syn.single_input(n, 384, seed=5, batch=1)
    z = syn.pair_input(n, 128, seed=6, batch=1)
    mask = syn.token_mask(n, n_real)[None]
    w = syn.single_attention_weights(seed=7)
    att, pre = P.single_attention_to_boltz2(w)
    st = device_tensor(s, dtype)
    s_ln = O.layer_norm(prep(s, dtype), prep(w["pre_norm_s"]["weight"], dtype), prep(w["pre_norm_s"]["bias"], dtype))
    packed = P.pack_single_attention_boltz2(att, dtype, "cuda", pre_norm=pre)
    got = kernels.single_attention(st, device_tensor(z, dtype), device_tensor(mask, dtype), packed, residual=st)
    torch.cuda.synchronize()
    want = prep(s, dtype) + O.boltz2_attention_pair_bias(prep_tree(w, dtype), s_ln, prep(z, dtype), mask)
    assert_parity(to_np(got)[:, :n_real], want[:, :n_real], dtype, "single attention")
    # the mirror (already-normalised s, update only) agrees with the fused call
    upd = boltz2.attention_pair_bias_forward(att, device_tensor(s_ln, dtype), device_tensor(z, dtype),
                                             device_tensor(mask, dtype))
    torch.cuda.synchronize()
    want_u = O.boltz2_attention_pair_bias(prep_tree(w, dtype), prep(s_ln, dtype), prep(z, dtype), mask)
    assert_parity(to_np(upd)[:, :n_real], want_u[:, :n_real], dtype, "single attention update")


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("batch,n,heads,expansion", [
    (1, 64, 16, 4),  # fused into the transition epilogue, no padding
    (1, 37, 16, 4),  # fused, n % 4 != 0, padded border
    (2, 40, 12, 4),  # fused, two batch entries, padded border
    (1, 20, 24, 4),  # more than 16 heads: a separate pass after the fused transition
    (1, 24, 16, 2),  # a 2x hidden width: general transition path, then the pass
])
def test_transition_pair_bias_output(dt, batch, n, heads, expansion):
    """The pair transition's pair-bias output: its own output unchanged, the
    prepared bias equal to log2(e) LN_z(out) w_z^T of that output inside
    [n, n] and zero on the padded border, and the single attention fed the
    prepared bias agreeing with the one that builds its own from z."""
    dtype = DTYPES[dt]
    say(f"transition pair-bias output batch={batch} n={n} heads={heads} x{expansion} {dt}")
    z = syn.pair_input(n, 128, seed=41, batch=batch)
    s = syn.single_input(n, 384, seed=42, batch=batch)
    mask = np.stack([syn.token_mask(n, n - 3 * b) for b in range(batch)])
    tr = syn.transition_weights(128, expansion, seed=44)
    tw = P.pack_transition_torch({k: tr[k] for k in ("layer_norm", "linear_a", "linear_b", "linear_out")}, dtype, "cuda")
    w = syn.single_attention_weights(heads=heads, seed=43)
    att, pre = P.single_attention_to_boltz2(w)
    packed = P.pack_single_attention_boltz2(att, dtype, "cuda", pre_norm=pre)
    zt = device_tensor(z, dtype)
    plain = kernels.transition(zt, tw, residual=zt)
    out, pb = kernels.transition(zt, tw, residual=zt, pair_bias_for=packed)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    np_ = (n + 63) // 64 * 64
    assert tuple(pb.shape) == (batch, heads, np_, np_)
    pbn = to_np(pb)
    assert not pbn[:, :, n:, :].any() and not pbn[:, :, :, n:].any()
    o = to_np(out)
    ln = O.layer_norm(o, prep(w["proj_z_norm"]["weight"], dtype), prep(w["proj_z_norm"]["bias"], dtype))
    want = np.transpose(O.linear_torch(ln, {"weight": prep(w["proj_z"]["weight"], dtype)}), (0, 3, 1, 2))
    assert_parity(pbn[:, :, :n, :n], want * np.log2(np.e), dtype, "prepared pair bias")
    st, mt = device_tensor(s, dtype), device_tensor(mask, dtype)
    ref = kernels.single_attention(st, out, mt, packed, residual=st)
    got = kernels.single_attention(st, None, mt, packed, residual=st, pair_bias=pb)
    torch.cuda.synchronize()
    assert_parity(to_np(got), to_np(ref), dtype, "single attention with the prepared bias")


def test_pair_bias_argument_errors():
    """Misuse of the prepared pair bias is refused on the host: a transition
    input that is not a pair tensor, a bias of the wrong shape or dtype, and
    a single attention given neither z nor a prepared bias."""
    dtype = torch.bfloat16
    n = 24
    tr = syn.transition_weights(128, 4, seed=44)
    tw = P.pack_transition_torch({k: tr[k] for k in ("layer_norm", "linear_a", "linear_b", "linear_out")}, dtype, "cuda")
    w = syn.single_attention_weights(heads=16, seed=43)
    att, pre = P.single_attention_to_boltz2(w)
    packed = P.pack_single_attention_boltz2(att, dtype, "cuda", pre_norm=pre)
    rows = device_tensor(syn.pair_input(n, 128, seed=1)[0], dtype)  # [n, 128]: not a pair tensor
    with pytest.raises(ValueError, match="pair tensor"):
        kernels.transition(rows, tw, pair_bias_for=packed)
    z = device_tensor(syn.pair_input(n, 128, seed=1, batch=1), dtype)
    s = device_tensor(syn.single_input(n, 384, seed=2, batch=1), dtype)
    _, pb = kernels.transition(z, tw, residual=z, pair_bias_for=packed)
    with pytest.raises(ValueError, match="prepared"):
        kernels.single_attention(s, None, None, packed, pair_bias=pb[:, :8].contiguous())
    with pytest.raises(ValueError, match="prepared"):
        kernels.single_attention(s, None, None, packed, pair_bias=pb.float())
    with pytest.raises(ValueError, match="needs z or a prepared pair_bias"):
        kernels.single_attention(s, None, None, packed)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_pairformer_layer_parity(dt):
    dtype = DTYPES[dt]
    n, n_real = 48, 44
    say(f"pairformer layer n={n} {dt}")
    w = syn.pairformer_layer_weights(seed=9)
    s = syn.single_input(n, 384, seed=1, batch=1)
    z = syn.pair_input(n, 128, seed=0, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    layer = PairformerLayerWeights.from_fields(w, dtype, "cuda")
    gs, gz = layer.forward(device_tensor(s, dtype), device_tensor(z, dtype), device_tensor(tm, dtype),
                           device_tensor(pm, dtype))
    torch.cuda.synchronize()
    ws, wz = O.boltz2_pairformer_layer(prep_tree(w, dtype), prep(s, dtype), prep(z, dtype), tm, pm)
    v = slice(0, n_real)
    assert_parity(to_np(gz)[:, v, v], wz[:, v, v], dtype, "layer z")
    assert_parity(to_np(gs)[:, v], ws[:, v], dtype, "layer s")
    # the Boltz-2 mirror with the Boltz-2 parameter dict runs the same kernels
    ms, mz = boltz2.pairformer_layer_forward(P.pairformer_layer_to_boltz2(w), device_tensor(s, dtype),
                                             device_tensor(z, dtype), device_tensor(tm, dtype),
                                             device_tensor(pm, dtype))
    assert torch.equal(ms, gs) and torch.equal(mz, gz)


@pytest.mark.gpu
def test_pairformer_module_two_layers():
    """``pairformer_module_forward`` over two layers equals the oracle layer
    applied twice (bf16), and a pre-packed stack gives identical bits."""
    dtype = DTYPES["bf16"]
    n, n_real = 40, 37
    say(f"pairformer module 2 layers n={n} bf16")
    ws_ = [syn.pairformer_layer_weights(seed=20), syn.pairformer_layer_weights(seed=40)]
    s = syn.single_input(n, 384, seed=1, batch=1)
    z = syn.pair_input(n, 128, seed=0, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    params = {"layers": [P.pairformer_layer_to_boltz2(w) for w in ws_]}
    args = (device_tensor(s, dtype), device_tensor(z, dtype), device_tensor(tm, dtype), device_tensor(pm, dtype))
    gs, gz = boltz2.pairformer_module_forward(params, *args)
    torch.cuda.synchronize()
    es, ez = prep(s, dtype), prep(z, dtype)
    for w in ws_:
        es, ez = O.boltz2_pairformer_layer(prep_tree(w, dtype), es, ez, tm, pm)
    v = slice(0, n_real)
    assert_parity(to_np(gz)[:, v, v], ez[:, v, v], dtype, "module z")
    assert_parity(to_np(gs)[:, v], es[:, v], dtype, "module s")
    packed = {"layers": [PairformerLayerWeights.from_fields(w, dtype, "cuda") for w in ws_]}
    ps, pz = boltz2.pairformer_module_forward(packed, *args, use_scan=False)
    assert torch.equal(ps, gs) and torch.equal(pz, gz)


def test_pairformer_no_seq_layer():
    """The MSA module's pair block (``boltz2.pairformer_no_seq_layer_forward``)
    against the oracle (bf16), and the pair half of a full layer gives the
    same bits."""
    dtype = DTYPES["bf16"]
    n, n_real = 40, 35
    say(f"pairformer no-seq layer n={n} bf16")
    w = syn.pairformer_layer_weights(seed=31)
    z = syn.pair_input(n, 128, seed=2, batch=1)
    pm = syn.pair_mask(n, n_real)[None]
    bp = P.pairformer_layer_to_boltz2(w)
    params = {k: bp[k] for k in ("tri_mul_out", "tri_mul_in", "tri_att_start", "tri_att_end", "transition_z")}
    got = boltz2.pairformer_no_seq_layer_forward(params, device_tensor(z, dtype), device_tensor(pm, dtype))
    torch.cuda.synchronize()
    want = O.boltz2_pairformer_no_seq_layer(prep_tree(w, dtype), prep(z, dtype), pm)
    v = slice(0, n_real)
    assert_parity(to_np(got)[:, v, v], want[:, v, v], dtype, "no-seq layer z")
    s = syn.single_input(n, 384, seed=3, batch=1)
    tm = syn.token_mask(n, n_real)[None]
    _, gz = boltz2.pairformer_layer_forward(bp, device_tensor(s, dtype), device_tensor(z, dtype),
                                            device_tensor(tm, dtype), device_tensor(pm, dtype))
    assert torch.equal(gz, got)


def _of3_pair_block_oracle(z, p, pm, *, mask_transition, tri_mul_first):
    """The reference's ``pair_block`` composition on the oracle, with the
    ending node as a starting module between two transposes (as upstream)."""
    def mul_pair(z):
        z = z + O.openfold3_triangle_multiplication(z, p["tri_mul_out"], outgoing=True, mask=pm)
        return z + O.openfold3_triangle_multiplication(z, p["tri_mul_in"], outgoing=False, mask=pm)

    def att_pair(z):
        z = z + O.openfold3_triangle_attention(z, p["tri_att_start"], no_heads=4, mask=pm)
        zt = np.swapaxes(z, -2, -3)
        zt = zt + O.openfold3_triangle_attention(zt, p["tri_att_end"], no_heads=4, mask=np.swapaxes(pm, -1, -2))
        return np.swapaxes(zt, -2, -3)

    z = att_pair(mul_pair(z)) if tri_mul_first else mul_pair(att_pair(z))
    return z + O.transition(z, p["pair_transition"], mask=pm if mask_transition else None)


@pytest.mark.parametrize("dt,mask_transition,tri_mul_first", [("fp32", True, True), ("bf16", True, True),
                                                              ("fp32", False, False)])
def test_openfold3_pair_block(dt, mask_transition, tri_mul_first):
    dtype = DTYPES[dt]
    n, n_real = 36, 31
    say(f"openfold3 pair_block n={n} {dt} mask_transition={mask_transition} tri_mul_first={tri_mul_first}")
    z = syn.pair_input(n, 128, seed=11, batch=1)
    pm = syn.pair_mask(n, n_real)[None]
    tw = syn.transition_weights(128, seed=16)
    fields = {"tri_mul_out": syn.trimul_weights(seed=12), "tri_mul_in": syn.trimul_weights(seed=13),
              "tri_att_start": syn.triattn_weights(seed=14), "tri_att_end": syn.triattn_weights(seed=15)}
    of3 = {k: (P.trimul_to_openfold3(v) if k.startswith("tri_mul") else P.triattn_to_openfold3(v))
           for k, v in fields.items()}
    of3["pair_transition"] = {"layer_norm": tw["layer_norm"],
                              "swiglu": {"linear_a": tw["linear_a"], "linear_b": tw["linear_b"]},
                              "linear_out": tw["linear_out"]}
    params = openfold3.PairBlockParams(**of3)
    got = openfold3.pair_block(device_tensor(z, dtype), params, pair_mask=device_tensor(pm, dtype), no_heads_pair=4,
                               mask_transition=mask_transition, tri_mul_first=tri_mul_first)
    torch.cuda.synchronize()
    ref = {k: prep_tree(v, dtype) for k, v in fields.items()}
    for k in ("tri_att_start", "tri_att_end"):  # OpenFold3 field names of the oracle
        ref[k] = {"layer_norm": ref[k]["layer_norm"], "linear_z": ref[k]["linear"], "mha": ref[k]["attention"]}
    ref["pair_transition"] = prep_tree(tw, dtype)
    want = _of3_pair_block_oracle(prep(z, dtype), ref, pm, mask_transition=mask_transition,
                                  tri_mul_first=tri_mul_first)
    v = slice(0, n_real)
    assert_parity(to_np(got)[:, v, v], want[:, v, v], dtype, "openfold3 pair_block")

