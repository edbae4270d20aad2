"""Host-side behaviour of the port mirrors that needs no GPU: selector values
and error messages (``T/models/boltz2/test_triangle_precision.py:30-65``,
``T/models/protenix/test_triangle_cueq.py:76-152``,
``T/models/openfold3/test_triangle_attention_cueq.py:70-87``), parameter
packing layouts, and the refusal of host tensors."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from foldjax_amd import boltz2, kernels, openfold3, protenix
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn


def _z(n=4):
    return torch.zeros(n, n, 128)


def test_boltz2_trimul_selector(monkeypatch):
    tm = P.trimul_to_boltz2(syn.trimul_weights())
    monkeypatch.setenv("BOLTZ_JAX_TRIANGLE_MULTIPLICATION_BACKEND", "nope")
    with pytest.raises(ValueError, match="Unsupported triangle multiplication backend: 'nope'"):
        boltz2.triangle_multiplication_forward(tm, _z(), None, "outgoing")
    monkeypatch.setenv("BOLTZ_JAX_TRIANGLE_MULTIPLICATION_BACKEND", "cueq")
    with pytest.raises(RuntimeError, match="provides 'hip'"):
        boltz2.triangle_multiplication_forward(tm, _z(), None, "outgoing")
    monkeypatch.setenv("BOLTZ_JAX_TRIANGLE_MULTIPLICATION_BACKEND", "hip")
    with pytest.raises(ValueError, match="Unsupported contraction_precision"):
        boltz2.triangle_multiplication_forward(tm, _z(), None, "outgoing", contraction_precision="fp8")
    with pytest.raises(ValueError, match="device tensors"):
        boltz2.triangle_multiplication_forward(tm, _z(), None, "outgoing")


def test_boltz2_attention_selector():
    ta = P.triattn_to_boltz2(syn.triattn_weights())
    with pytest.raises(ValueError, match="Unsupported triangle_backend"):
        boltz2.triangle_attention_forward(ta, _z(), triangle_backend="mystery")
    for b in ("xla", "pallas", "tokamax", "cueq"):
        with pytest.raises(RuntimeError):
            boltz2.triangle_attention_forward(ta, _z(), triangle_backend=b)
    with pytest.raises(ValueError, match="Unsupported matmul_precision"):
        boltz2.triangle_attention_forward(ta, _z(), matmul_precision="bogus")


def test_protenix_selectors(monkeypatch):
    tm = P.trimul_to_protenix(syn.trimul_weights())
    ta = P.triattn_to_protenix(syn.triattn_weights())
    monkeypatch.setenv("PROTENIX_TRIANGLE_BACKEND", "SomeThing")
    with pytest.raises(ValueError, match="unsupported triangle attention backend: 'something'"):
        protenix.triangle_attention(_z(), None, ta, num_heads=4)
    monkeypatch.setenv("PROTENIX_TRIANGLE_BACKEND", "CUEQ_JIT")
    with pytest.raises(RuntimeError):
        protenix.triangle_attention(_z(), None, ta, num_heads=4)
    monkeypatch.setenv("PROTENIX_TRIANGLE_MULTIPLICATION_BACKEND", "xyz")
    with pytest.raises(ValueError, match="unsupported triangle multiplication backend"):
        protenix.triangle_multiplication(_z(), None, tm, "outgoing")
    monkeypatch.delenv("PROTENIX_TRIANGLE_BACKEND")
    with pytest.raises(ValueError, match="device tensors"):
        protenix.triangle_attention(_z(), None, ta, num_heads=4)


def test_openfold3_selector(monkeypatch):
    ta = P.triattn_to_openfold3(syn.triattn_weights())
    monkeypatch.setenv("OPENFOLD3_TRIANGLE_BACKEND", "XLA")
    with pytest.raises(RuntimeError):
        openfold3.triangle_attention(_z(), ta, no_heads=4)
    with pytest.raises(ValueError, match="unsupported triangle attention backend"):
        openfold3.triangle_attention(_z(), ta, no_heads=4, backend="magic")


def test_projection_biases_are_rejected():
    w = syn.trimul_weights()
    w["linear_a_p"]["bias"] = np.zeros(128, np.float32)
    with pytest.raises(ValueError, match="bias-free"):
        P.pack_trimul_torch(P.trimul_to_protenix(w), torch.float32, "cpu")


def test_packing_layouts_agree_across_ports():
    tm = syn.trimul_weights(seed=3)
    a = P.pack_trimul_torch(P.trimul_to_protenix(tm), torch.float32, "cpu")
    b = P.pack_trimul_torch(P.trimul_to_openfold3(tm), torch.float32, "cpu")
    c = P.pack_trimul_boltz2(P.trimul_to_boltz2(tm), torch.float32, "cpu")
    for f in ("p_in_weight", "g_in_weight", "p_out_weight", "g_out_weight", "norm_out_bias"):
        assert torch.equal(getattr(a, f), getattr(b, f)) and torch.equal(getattr(a, f), getattr(c, f))
    # a rows first, as the cuEq call expects (B2T/triangle_cueq.py:94-95)
    assert torch.equal(a.p_in_weight[:128], torch.from_numpy(tm["linear_a_p"]["weight"]))
    ta = syn.triattn_weights(seed=4)
    x = P.pack_triattn_protenix(P.triattn_to_protenix(ta), torch.float32, "cpu")
    y = P.pack_triattn_openfold3(P.triattn_to_openfold3(ta), torch.float32, "cpu")
    z = P.pack_triattn_boltz2(P.triattn_to_boltz2(ta), torch.float32, "cpu")
    for f in ("bias_weight", "q_weight", "k_weight", "v_weight", "g_weight", "o_weight"):
        assert torch.equal(getattr(x, f), getattr(y, f)) and torch.equal(getattr(x, f), getattr(z, f))
    assert x.heads == 4


def test_kernels_reject_host_tensors_and_bad_dtypes():
    w = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights()), torch.float32, "cpu")
    with pytest.raises(ValueError, match="device tensors"):
        kernels.trimul(_z(), None, w, "outgoing")
    with pytest.raises(ValueError):
        kernels._code(torch.float16)


def test_bf16_round_matches_torch():
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 100
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(syn.bf16_round(x), want)


def _meta(t: torch.Tensor) -> torch.Tensor:
    """The same shape on another device (``meta``): a stand-in for an operand
    left on the wrong device, which must be refused before any launch."""
    return torch.empty(t.shape, dtype=t.dtype, device="meta")


def test_kernels_refuse_operands_on_another_device():
    z = _z(8)
    tm = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights()), torch.float32, "cpu")
    ta = P.pack_triattn_protenix(P.triattn_to_protenix(syn.triattn_weights()), torch.float32, "cpu")
    tr = P.pack_transition_torch(syn.transition_weights(), torch.float32, "cpu")
    m = torch.ones(8, 8)
    with pytest.raises(ValueError, match="mask is on meta"):
        kernels.trimul(z, _meta(m), tm, "outgoing")
    with pytest.raises(ValueError, match="residual is on meta"):
        kernels.trimul(z, m, tm, "outgoing", residual=_meta(z))
    with pytest.raises(ValueError, match="mask is on meta"):
        kernels.triattn(z, _meta(m), ta)
    with pytest.raises(ValueError, match="residual is on meta"):
        kernels.triattn(z, m, ta, residual=_meta(z))
    q = torch.zeros(1, 8, 4, 8, 32)
    tb = torch.zeros(1, 1, 4, 8, 8)
    for name, args in (("k", (q, _meta(q), q, tb, None)), ("v", (q, q, _meta(q), tb, None)),
                       ("tri_bias", (q, q, q, _meta(tb), None)),
                       ("mask_bias", (q, q, q, tb, _meta(torch.zeros(1, 8, 1, 1, 8))))):
        with pytest.raises(ValueError, match=f"{name} is on meta"):
            kernels.triattn_core(*args, scale=1.0)
    with pytest.raises(ValueError, match="row_mask is on meta"):
        kernels.transition(z, tr, row_mask=_meta(m))


def test_kernels_refuse_mismatched_shapes():
    z = _z(8)
    m = torch.ones(8, 8)
    w64 = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(64, 128)), torch.float32, "cpu")
    with pytest.raises(ValueError, match="tri-mul weight norm_in_weight must have shape"):
        kernels.trimul(z, m, w64, "outgoing")  # packed for c_z = 64, called with 128
    tm = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights()), torch.float32, "cpu")
    with pytest.raises(ValueError, match="residual must have shape"):
        kernels.trimul(z, m, tm, "outgoing", residual=_z(4))
    ta64 = P.pack_triattn_protenix(P.triattn_to_protenix(syn.triattn_weights(64, 4, 16)), torch.float32, "cpu")
    with pytest.raises(ValueError, match="tri-attn weight"):
        kernels.triattn(z, m, ta64)
    q = torch.zeros(1, 8, 4, 8, 32)
    with pytest.raises(ValueError, match="q, k, v must share"):
        kernels.triattn_core(q, torch.zeros(1, 8, 4, 9, 32), q, torch.zeros(1, 1, 4, 8, 8), None, scale=1.0)
    with pytest.raises(ValueError, match="tri_bias must be"):
        kernels.triattn_core(q, q, q, torch.zeros(1, 1, 4, 8, 9), None, scale=1.0)
    with pytest.raises(ValueError, match="mask_bias must be"):
        kernels.triattn_core(q, q, q, torch.zeros(1, 1, 4, 8, 8), torch.zeros(1, 8, 1, 1, 7), scale=1.0)
    tr = P.pack_transition_torch({"layer_norm": {"weight": np.ones(96), "bias": np.zeros(96)},
                                  "linear_a": {"weight": np.zeros((384, 96))}, "linear_b": {"weight": np.zeros((384, 96))},
                                  "linear_out": {"weight": np.zeros((96, 384))}}, torch.float32, "cpu")
    with pytest.raises(ValueError, match="transition weight norm_weight must have shape"):
        kernels.transition(z, tr)
    sa = P.pack_single_attention_boltz2(P.single_attention_to_boltz2(syn.single_attention_weights())[0],
                                        torch.float32, "cpu")
    with pytest.raises(ValueError, match="single attention weight q_weight must have shape"):
        kernels.single_attention(torch.zeros(1, 8, 256), torch.zeros(1, 8, 8, 128), None, sa)
    with pytest.raises(ValueError, match="residual must have shape"):
        kernels.single_attention(torch.zeros(1, 8, 384), torch.zeros(1, 8, 8, 128), None, sa,
                                 residual=torch.zeros(1, 7, 384))


def test_port_single_attention_and_block_arguments_are_validated():
    """Selector values, the diffusion-only forms and missing pieces are
    refused on the host, with the reference's messages where it has them."""
    z = _z(8)
    s = torch.zeros(1, 8, 384)
    w = syn.single_attention_weights(seed=3)
    px = P.single_attention_to_protenix(w)
    with pytest.raises(ValueError, match="unsupported attention backend"):
        protenix.attention_pair_bias(s, None, z, px, num_heads=16, attention_backend="flash")
    with pytest.raises(ValueError, match="z_is_normalized"):
        protenix.attention_pair_bias(s, None, z, px, num_heads=16, z_is_normalized=True)
    with pytest.raises(ValueError, match="trunk form"):
        P.pack_single_attention_protenix(px._replace(has_s=True), torch.float32, "cpu")
    with pytest.raises(ValueError, match="gated attention"):
        P.pack_single_attention_openfold3(P.single_attention_to_openfold3(w)._replace(
            mha=px.attention._replace(linear_g=None)), torch.float32, "cpu")
    with pytest.raises(ValueError, match="num_heads=8"):
        protenix.attention_pair_bias(s, None, z, px, num_heads=8)
    with pytest.raises(ValueError, match="PairformerStack requires at least one block"):
        protenix.pairformer_stack(s, z, None, protenix.PairformerStackParams(blocks=()))
    with pytest.raises(ValueError, match="unsupported triangle attention backend"):
        protenix.pairformer_block(s, z, None, P.pairformer_block_to_protenix(syn.pairformer_layer_weights()),
                                  triangle_attention_backend="pallas")


def test_single_attention_extra_bias_and_out_mask_shapes():
    """An extra bias must be 4-D over [N, N] and broadcast to [B, H, N, N];
    an output mask must broadcast to [B, N]. Both are refused before any
    launch (here on host tensors, which the device check then refuses)."""
    w = P.pack_single_attention_boltz2(*P.single_attention_to_boltz2(syn.single_attention_weights(seed=3))[:1],
                                       torch.float32, "cpu")
    s = torch.zeros(1, 8, 384)
    z = _z(8)
    with pytest.raises(ValueError, match="extra_bias must be a 4-D tensor"):
        kernels.single_attention(s, z, None, w, extra_bias=torch.zeros(8, 8))
    with pytest.raises(ValueError, match="does not broadcast"):
        kernels.single_attention(s, z, None, w, extra_bias=torch.zeros(1, 3, 8, 8))
    with pytest.raises(ValueError, match="out_mask of shape"):
        kernels.single_attention(s, z, None, w, out_mask=torch.ones(1, 7))


def test_stacked_layers_share_one_buffer_per_weight_kind():
    from foldjax_amd.pairformer import PairformerLayerWeights
    from foldjax_amd.stacking import StackedLayers, stackable, stacked_or_stack

    ls = [PairformerLayerWeights.random(torch.float32, "cpu", seed=i) for i in (1, 9)]
    st = stacked_or_stack(ls)
    assert stacked_or_stack(st) is st and len(st) == 2 and stackable(ls)
    buf = st.stacked["triangle"]["tri_mul_out"]["p_in_weight"]
    assert tuple(buf.shape) == (2, 256, 128)
    for i, layer in enumerate(st):
        v = layer.triangle.tri_mul_out.p_in_weight
        assert torch.equal(v, ls[i].triangle.tri_mul_out.p_in_weight)
        assert v.data_ptr() == buf[i].data_ptr() and v.is_contiguous()
    other = PairformerLayerWeights.from_fields(syn.pairformer_layer_weights(heads_single=8), torch.float32, "cpu")
    assert not stackable([ls[0], other])
    with pytest.raises(ValueError):
        StackedLayers([ls[0], other])
    with pytest.raises(ValueError, match="empty"):
        stacked_or_stack([])


def test_stacking_keeps_single_attention_projections_back_to_back():
    """A packed single attention keeps q|k|v|g in one buffer, so the library
    runs one projection GEMM (``fjx_single_attention_fwd``); the stacked
    layers' views keep that layout: each layer's four weights are consecutive
    slices of one [4 c_s, c_s] row of a [L, 4 c_s, c_s] buffer."""
    from foldjax_amd.pairformer import PairformerLayerWeights
    from foldjax_amd.stacking import stacked_or_stack

    ls = [PairformerLayerWeights.random(torch.float32, "cpu", seed=i) for i in (3, 4, 5)]
    c = int(ls[0].attention.q_weight.shape[0])
    step = c * c * ls[0].attention.q_weight.element_size()

    def back_to_back(a):
        ptrs = [getattr(a, k).data_ptr() for k in ("q_weight", "k_weight", "v_weight", "g_weight")]
        return all(p1 - p0 == step for p0, p1 in zip(ptrs, ptrs[1:]))

    assert all(back_to_back(layer.attention) for layer in ls)
    st = stacked_or_stack(ls)
    buf = st.stacked["attention"]["q_weight|k_weight|v_weight|g_weight"]
    assert tuple(buf.shape) == (3, 4 * c, c)
    for i, layer in enumerate(st):
        a = layer.attention
        assert back_to_back(a) and a.q_weight.data_ptr() == buf[i].data_ptr()
        for k in ("q_weight", "k_weight", "v_weight", "g_weight", "o_weight"):
            assert torch.equal(getattr(a, k), getattr(ls[i].attention, k))


def test_neutral_triangle_kernel_knob():
    """``triangle_kernel`` (``src/foldjax/execution.py:43``) gains "hip";
    "auto" maps to it explicitly on every port, the reference's values keep
    their native spellings, and errors follow ``execution.translate``."""
    from foldjax_amd import execution as E

    for model, native in (("boltz2", "triangle_backend"), ("protenix", "trunk_triangle_attention_backend"),
                          ("openfold3", "triangle_kernel")):
        assert E.translate({"triangle_kernel": "auto"}, model) == {native: "hip"}
        assert E.triangle_kernel(model) == "hip" and E.triangle_kernel(model, "hip") == "hip"
    assert E.triangle_kernel("protenix", "cueq") == "cueq_jit"
    assert E.triangle_kernel("protenix", "xla") == "xla_jit"
    assert E.triangle_kernel("boltz2", "xla") == "xla"
    with pytest.raises(ValueError, match="must be one of"):
        E.translate({"triangle_kernel": "pallas"}, "boltz2")
    with pytest.raises(ValueError, match="were both set"):
        E.translate({"triangle_kernel": "auto", "triangle_backend": "xla"}, "boltz2")
    with pytest.raises(ValueError, match="unknown model"):
        E.translate({"triangle_kernel": "auto"}, "af2")
    assert E.normalize({"triangle_backend": "hip"}, native=set()) == {"triangle_kernel": "hip"}
    assert E.normalize({"triangle_backend": "hip"}, native={"triangle_backend"}) == {"triangle_backend": "hip"}
    # the translated value is accepted by the port's own selector
    assert boltz2.resolve_matmul_precision("highest")
    with pytest.raises(RuntimeError, match="JAX backend"):
        protenix.triangle_attention(_z(8), None, P.triattn_to_protenix(syn.triattn_weights()), num_heads=4,
                                    attention_backend=E.triangle_kernel("protenix", "xla"))
