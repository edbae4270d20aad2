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
