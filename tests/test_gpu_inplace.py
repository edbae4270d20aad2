"""In-place updates: every pair-track entry point writes into a caller's
``out`` that may be its input ``x`` and its residual at once, as the block and
stack forwards now do (one pair tensor per block; with donation none,
``B2K/pairformer.py:74-96``). Each in-place result must equal the
out-of-place one bit for bit: the kernels read every input of an output
position before writing it, and only the workgroup that writes a position
reads it. Covered: the fused c = 128 kernels (LDS-DMA contraction and
128-query attention at N = 256), the narrow c_z = 64 forms, the general-width
paths (c_z = 48), the transition with its fused pair-bias epilogue, and whole
block and stack forwards with and without donation."""

from __future__ import annotations

import pytest
import torch

from foldjax_amd import boltz2, kernels
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn
from foldjax_amd.pairformer import PairformerLayerWeights
from tests.gpu_util import device_tensor, say

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _pair(n, c, seed, dtype=BF16):
    return device_tensor(syn.pair_input(n, c, seed=seed, batch=1), dtype)


@pytest.mark.parametrize("c_z", [128, 64, 48])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_in_place(c_z, direction):
    n = 256 if c_z != 48 else 136
    say(f"in-place trimul c_z={c_z} n={n} {direction}")
    w = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(c_z, 128, seed=40)), BF16, "cuda")
    m = device_tensor(syn.pair_mask(n, n - 9)[None], BF16)
    z = _pair(n, c_z, 41)
    om = device_tensor(syn.pair_mask(n, n - 5)[None], BF16)
    want = kernels.trimul(z, m, w, direction, residual=z, out_mask=om)
    buf = z.clone()
    got = kernels.trimul(buf, m, w, direction, residual=buf, out_mask=om, out=buf)
    torch.cuda.synchronize()
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(got, want)


@pytest.mark.parametrize("c_z", [128, 64, 48])
@pytest.mark.parametrize("starting", [True, False])
def test_triattn_in_place(c_z, starting):
    n = 256 if c_z != 48 else 136
    heads = 4 if c_z != 48 else 2
    say(f"in-place triattn c_z={c_z} n={n} starting={starting}")
    w = P.pack_triattn_protenix(P.triattn_to_protenix(syn.triattn_weights(c_z, heads, 32, seed=42)), BF16, "cuda")
    m = device_tensor(syn.pair_mask(n, n - 9)[None], BF16)
    z = _pair(n, c_z, 43)
    want = kernels.triattn(z, m, w, starting=starting, residual=z)
    buf = z.clone()
    got = kernels.triattn(buf, m, w, starting=starting, residual=buf, out=buf)
    torch.cuda.synchronize()
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(got, want)


@pytest.mark.parametrize("c", [128, 64, 48, 384])
def test_transition_in_place(c):
    n = 128 if c != 384 else 24
    say(f"in-place transition c={c} n={n}")
    w = P.pack_transition_torch(P.transition_to_protenix(syn.transition_weights(c, seed=44)), BF16, "cuda")
    z = _pair(n, c, 45)
    rm = device_tensor(syn.pair_mask(n, n - 3)[None], BF16)
    want = kernels.transition(z, w, residual=z, row_mask=rm)
    buf = z.clone()
    got = kernels.transition(buf, w, residual=buf, row_mask=rm, out=buf)
    torch.cuda.synchronize()
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(got, want)


@pytest.mark.parametrize("single_dtype", [BF16, torch.float32])
def test_transition_pair_bias_in_place(single_dtype):
    n = 192
    say(f"in-place transition with the pair bias n={n} single {single_dtype}")
    w = P.pack_transition_torch(P.transition_to_protenix(syn.transition_weights(128, seed=46)), BF16, "cuda")
    att, pre = P.single_attention_to_boltz2(syn.single_attention_weights(heads=16, seed=47))
    aw = P.pack_single_attention_boltz2(att, single_dtype, "cuda", pre_norm=pre)
    z = _pair(n, 128, 48)
    want, want_pb = kernels.transition(z, w, residual=z, pair_bias_for=aw)
    buf = z.clone()
    got, got_pb = kernels.transition(buf, w, residual=buf, pair_bias_for=aw, out=buf)
    torch.cuda.synchronize()
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(got, want) and torch.equal(got_pb, want_pb)


def test_out_argument_checks():
    z = _pair(16, 128, 49)
    w = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(128, 128, seed=50)), BF16, "cuda")
    with pytest.raises(ValueError, match="out must be"):
        kernels.trimul(z, None, w, "outgoing", out=torch.empty((1, 16, 16, 64), device="cuda", dtype=BF16))
    with pytest.raises(ValueError, match="out must be contiguous"):
        kernels.trimul(z, None, w, "outgoing", out=torch.empty((1, 16, 128, 16), device="cuda", dtype=BF16)
                       .transpose(2, 3))


@pytest.mark.parametrize("single_dtype", [BF16, torch.float32])
def test_block_forward_donated(single_dtype):
    """A block forward that writes one new pair tensor (no donation) and one
    that overwrites its donated inputs give the same s and z as separate
    out-of-place sublayer calls; without donation the inputs are unchanged."""
    n, n_real = 200, 190
    say(f"block forward in place / donated n={n} single {single_dtype}")
    layer = PairformerLayerWeights.random(BF16, "cuda", seed=51, single_dtype=single_dtype)
    z0 = _pair(n, 128, 52)
    s0 = device_tensor(syn.single_input(n, 384, seed=53, batch=1), single_dtype)
    tm = device_tensor(syn.token_mask(n, n_real)[None], single_dtype)
    pm = device_tensor(syn.pair_mask(n, n_real)[None], BF16)
    tri = layer.triangle
    z = kernels.trimul(z0, pm, tri.tri_mul_out, "outgoing", residual=z0)
    z = kernels.trimul(z, pm, tri.tri_mul_in, "incoming", residual=z)
    z = kernels.triattn(z, pm, tri.tri_att_start, starting=True, residual=z)
    z = kernels.triattn(z, pm, tri.tri_att_end, starting=False, residual=z)
    z, pb = kernels.transition(z, layer.transition_z, residual=z, pair_bias_for=layer.attention)
    s = kernels.single_attention(s0, None, tm, layer.attention, residual=s0, pair_bias=pb)
    s = kernels.transition(s, layer.transition_s, residual=s)
    z_keep, s_keep = z0.clone(), s0.clone()
    fs, fz = layer.forward(s0, z0, tm, pm)
    torch.cuda.synchronize()
    assert torch.equal(fz, z) and torch.equal(fs, s)
    assert torch.equal(z0, z_keep) and torch.equal(s0, s_keep), "a forward without donation changed its inputs"
    zd, sd = z0.clone(), s0.clone()
    ds, dz = layer.forward(sd, zd, tm, pm, donate=True)
    torch.cuda.synchronize()
    assert dz.data_ptr() == zd.data_ptr() and ds.data_ptr() == sd.data_ptr()
    assert torch.equal(dz, z) and torch.equal(ds, s)


def test_stack_carry_donation():
    """The Boltz-2 module forward donates the carry from its second layer on:
    equal, bit for bit, to the layers applied one by one without donation,
    and the caller's s and z are left unchanged."""
    n, n_real = 136, 130
    say(f"stack carry donation n={n}")
    layers = [PairformerLayerWeights.random(BF16, "cuda", seed=60 + 3 * i) for i in range(3)]
    z0 = _pair(n, 128, 61)
    s0 = device_tensor(syn.single_input(n, 384, seed=62, batch=1), BF16)
    tm = device_tensor(syn.token_mask(n, n_real)[None], BF16)
    pm = device_tensor(syn.pair_mask(n, n_real)[None], BF16)
    z_keep, s_keep = z0.clone(), s0.clone()
    s, z = s0, z0
    for lay in layers:
        s, z = lay.forward(s, z, tm, pm)
    gs, gz = boltz2.pairformer_module_forward({"layers": layers}, s0, z0, tm, pm, use_scan=False)
    torch.cuda.synchronize()
    assert torch.equal(gz, z) and torch.equal(gs, s)
    assert torch.equal(z0, z_keep) and torch.equal(s0, s_keep)
