"""GPU parity at pair widths other than 128, against the CPU oracle on the
same values (fp32: max-abs <= 1e-4; bf16: relative <= 2e-2):

- the narrow forms of the fused kernels, c_z in {32, 64, 96} with c_h = 128
  (tri-mul), 4 heads of 32 (tri-attn) and a 4x transition -- the Protenix
  template stack is c_z = 64 with c_h = 128 (``PXT/triangle.py:131-137``);
- the general-width paths for every other shape: c_z = 48 (not a multiple of
  32), c_h = 64 or 2 heads with c_z = 64, a c = 384 track (OpenDDE's
  c_z = c_h = 384) and transitions of other widths and expansions."""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from foldjax_amd import kernels, protenix
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn
from oracle import triangle as O
from tests.gpu_util import assert_parity, device_tensor, mask_case, prep, prep_tree, say, to_np

pytestmark = pytest.mark.gpu

DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16}


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("c_z,c_h,n,mask_kind", [(64, 128, 33, "tail"), (64, 128, 70, "random"),
                                                 (32, 128, 40, "random"), (96, 128, 17, "row0"),
                                                 (48, 128, 20, "random"), (64, 64, 24, "tail"),
                                                 (384, 384, 20, "random")])
def test_trimul_widths(dt, direction, c_z, c_h, n, mask_kind):
    dtype = DTYPES[dt]
    say(f"trimul widths c_z={c_z} c_h={c_h} n={n} {dt} {direction}")
    z = syn.pair_input(n, c_z, seed=5)
    m = mask_case(mask_kind, n)
    w = syn.trimul_weights(c_z, c_h, seed=6)
    got = protenix.triangle_multiplication(device_tensor(z, dtype), device_tensor(m, dtype),
                                           P.trimul_to_protenix(w), direction)
    torch.cuda.synchronize()
    want = O.protenix_triangle_multiplication(prep(z, dtype), prep(m, dtype), prep_tree(w, dtype), direction)
    assert got.shape == (n, n, c_z)
    assert_parity(to_np(got), want, dtype, f"trimul c_z={c_z} c_h={c_h} {direction}")


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("c_z,heads,n", [(64, 4, 33), (32, 4, 40), (96, 4, 70), (64, 2, 70), (48, 4, 20),
                                         (384, 8, 20)])
def test_triattn_widths(dt, starting, c_z, heads, n):
    dtype = DTYPES[dt]
    say(f"triattn widths c_z={c_z} heads={heads} n={n} {dt} starting={starting}")
    z = syn.pair_input(n, c_z, seed=7)
    m = mask_case("tail", n)
    w = syn.triattn_weights(c_z, heads, 32, seed=8)
    got = protenix.triangle_attention(device_tensor(z, dtype), device_tensor(m, dtype), P.triattn_to_protenix(w),
                                      num_heads=heads, starting=starting)
    torch.cuda.synchronize()
    want = O.protenix_triangle_attention(prep(z, dtype), prep(m, dtype), prep_tree(w, dtype), num_heads=heads,
                                         starting=starting)
    mv = m if starting else m.T
    rows = mv.max(axis=1) > 0
    g, w_ = (to_np(got)[rows], want[rows]) if starting else (to_np(got)[:, rows], want[:, rows])
    assert_parity(g, w_, dtype, f"triattn c_z={c_z} heads={heads} starting={starting}")


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("c,expansion,rows,masked", [(64, 4, 300, False), (32, 4, 100, True), (96, 4, 77, False),
                                                     (64, 2, 77, True), (48, 4, 50, False), (256, 4, 130, True)])
def test_transition_widths(dt, c, expansion, rows, masked):
    dtype = DTYPES[dt]
    say(f"transition widths c={c} x{expansion} rows={rows} {dt} masked={masked}")
    rng = np.random.default_rng(c + rows)
    x = rng.standard_normal((rows, c)).astype(np.float32)
    w = syn.transition_weights(c, expansion, seed=9)
    rm = (rng.random(rows) > 0.3).astype(np.float32) if masked else None
    tw = P.pack_transition_torch({k: w[k] for k in ("layer_norm", "linear_a", "linear_b", "linear_out")}, dtype, "cuda")
    xt = device_tensor(x, dtype)
    got = kernels.transition(xt, tw, row_mask=None if rm is None else device_tensor(rm, dtype), residual=xt)
    torch.cuda.synchronize()
    xr = prep(x, dtype)
    want = xr + O.transition(xr, prep_tree(w, dtype), mask=rm)
    assert_parity(to_np(got), want, dtype, f"transition c={c} x{expansion}")


def test_template_stack_pair_block_bf16():
    """One pair block at the template stack's widths (c_z = 64, c_h = 128,
    4 heads of 32, transition x4) through the narrow fused kernels, each
    residual added by the kernels, against the oracle composition."""
    dtype = DTYPES["bf16"]
    n, n_real, c_z = 40, 36, 64
    say(f"template pair block c_z={c_z} n={n} bf16")
    z = syn.pair_input(n, c_z, seed=12)
    pm = syn.pair_mask(n, n_real)
    tm = [syn.trimul_weights(c_z, 128, seed=13 + i) for i in range(2)]
    ta = [syn.triattn_weights(c_z, 4, 32, seed=15 + i) for i in range(2)]
    tr = syn.transition_weights(c_z, 4, seed=17)
    zt, mt = device_tensor(z, dtype), device_tensor(pm, dtype)
    zt = protenix.triangle_multiplication(zt, mt, P.trimul_to_protenix(tm[0]), "outgoing", residual=zt)
    zt = protenix.triangle_multiplication(zt, mt, P.trimul_to_protenix(tm[1]), "incoming", residual=zt)
    zt = protenix.triangle_attention(zt, mt, P.triattn_to_protenix(ta[0]), num_heads=4, starting=True, residual=zt)
    zt = protenix.triangle_attention(zt, mt, P.triattn_to_protenix(ta[1]), num_heads=4, starting=False, residual=zt)
    zt = protenix.transition(zt, {k: tr[k] for k in ("layer_norm", "linear_a", "linear_b", "linear_out")}, residual=zt)
    torch.cuda.synchronize()
    ze = prep(z, dtype)
    ze = ze + O.protenix_triangle_multiplication(ze, pm, prep_tree(tm[0], dtype), "outgoing")
    ze = ze + O.protenix_triangle_multiplication(ze, pm, prep_tree(tm[1], dtype), "incoming")
    ze = ze + O.protenix_triangle_attention(ze, pm, prep_tree(ta[0], dtype), num_heads=4, starting=True)
    ze = ze + O.protenix_triangle_attention(ze, pm, prep_tree(ta[1], dtype), num_heads=4, starting=False)
    ze = ze + O.transition(ze, prep_tree(tr, dtype))
    v = slice(0, n_real)
    assert_parity(to_np(zt)[v, v], ze[v, v], dtype, "template pair block")


@pytest.mark.parametrize("c_z,c_h", [(128, 128), (64, 128)])
@pytest.mark.parametrize("n", [1, 2])
def test_tiny_n_fused_and_general(c_z, c_h, n):
    """One and two tokens on the fused (c = 128) and the general paths: tri-mul
    both directions, tri-attn both nodes, bf16, against the oracle."""
    dtype = DTYPES["bf16"]
    say(f"tiny n={n} c_z={c_z} c_h={c_h}")
    z = syn.pair_input(n, c_z, seed=21)
    m = np.ones((n, n), np.float32)
    w = syn.trimul_weights(c_z, c_h, seed=22)
    wa = syn.triattn_weights(c_z, 4, 32, seed=23)
    for direction in ("outgoing", "incoming"):
        got = protenix.triangle_multiplication(device_tensor(z, dtype), device_tensor(m, dtype),
                                               P.trimul_to_protenix(w), direction)
        want = O.protenix_triangle_multiplication(prep(z, dtype), m, prep_tree(w, dtype), direction)
        assert_parity(to_np(got), want, dtype, f"tiny trimul {direction}")
    for starting in (True, False):
        got = protenix.triangle_attention(device_tensor(z, dtype), device_tensor(m, dtype), P.triattn_to_protenix(wa),
                                          num_heads=4, starting=starting)
        want = O.protenix_triangle_attention(prep(z, dtype), m, prep_tree(wa, dtype), num_heads=4, starting=starting)
        assert_parity(to_np(got), want, dtype, f"tiny triattn starting={starting}")


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("c_z", [64, 96])
def test_narrow_separate_residual_and_out_mask(dt, c_z):
    """The narrow kernels with a residual that is not x (the epilogues' global
    residual read) and an output mask: out = (residual + update) * (mask != 0),
    tri-mul both directions and tri-attn both nodes, against the oracle."""
    dtype = DTYPES[dt]
    n = 37
    say(f"narrow residual/out_mask c_z={c_z} n={n} {dt}")
    z = syn.pair_input(n, c_z, seed=31)
    r = syn.pair_input(n, c_z, seed=32)
    m = mask_case("random", n)
    om = mask_case("tail", n)
    wm = syn.trimul_weights(c_z, 128, seed=33)
    wa = syn.triattn_weights(c_z, 4, 32, seed=34)
    tm = P.pack_trimul_torch(P.trimul_to_protenix(wm), dtype, "cuda")
    ta = P.pack_triattn_protenix(P.triattn_to_protenix(wa), dtype, "cuda")
    zt, rt, mt, omt = (device_tensor(a, dtype) for a in (z, r, m, om))
    zr, rr, mr = prep(z, dtype), prep(r, dtype), prep(m, dtype)
    keep = (prep(om, dtype) != 0)[..., None]
    for direction in ("outgoing", "incoming"):
        got = kernels.trimul(zt, mt, tm, direction, residual=rt, out_mask=omt)
        torch.cuda.synchronize()
        want = (rr + O.protenix_triangle_multiplication(zr, mr, prep_tree(wm, dtype), direction)) * keep
        assert_parity(to_np(got), want, dtype, f"narrow trimul {direction} residual")
    for starting in (True, False):
        got = kernels.triattn(zt, mt, ta, starting=starting, residual=rt, out_mask=omt)
        torch.cuda.synchronize()
        want = (rr + O.protenix_triangle_attention(zr, mr, prep_tree(wa, dtype), num_heads=4,
                                                   starting=starting)) * keep
        mv = m if starting else m.T
        rows = mv.max(axis=1) > 0
        g, w_ = (to_np(got)[rows], want[rows]) if starting else (to_np(got)[:, rows], want[:, rows])
        assert_parity(g, w_, dtype, f"narrow triattn starting={starting} residual")


def test_single_projection_dma_gemm_row_tail_caller_operand_bf16():
    """The q|k|v|g projection of a single attention without a pre-norm reads
    the caller's s as the LDS-DMA GEMM's A operand (72 tiles of 256 x 256 at
    n = 2839). n % 256 = 23, so in the last row tile 9 of the first 32-row
    group's rows and every row of the other groups lie past s: each DMA
    instruction's row is tested against M through the buffer range check,
    and such rows read zero instead of the memory that follows s. Here s is a
    tensor of exactly n rows; the attention rows, the last ones included,
    match the oracle (a row read from past s would only reach output rows that
    are not stored, so the test pins the tail's results, not the absence of
    the read, which the range check guarantees)."""
    n, n_real, dtype = 2839, 2830, torch.bfloat16
    say(f"single attention no pre-norm, dma gemm row tail n={n}")
    w = syn.single_attention_weights(heads=16, seed=71)
    att, _ = P.single_attention_to_boltz2(w)
    aw = P.pack_single_attention_boltz2(att, dtype, "cuda", pre_norm=None)
    s_np = syn.single_input(n, 384, seed=72)
    s = torch.empty((n, 384), device="cuda", dtype=dtype)
    s.copy_(torch.from_numpy(s_np))
    g = torch.Generator(device="cuda")
    g.manual_seed(73)
    z = torch.randn((1, n, n, 128), generator=g, device="cuda", dtype=torch.float32).to(dtype)
    tm = syn.token_mask(n, n_real)
    got = kernels.single_attention(s[None], z, device_tensor(tm[None], dtype), aw)
    torch.cuda.synchronize()
    queries = [0, 1, 2560, 2815, 2816, n - 9, n - 1]
    zl = lambda i: z[0, i].float().cpu().numpy().astype(np.float64)  # noqa: E731

    class Rows:
        def __getitem__(self, i):
            return zl(int(i))

    wq = prep_tree(w, dtype)
    want = O.boltz2_attention_pair_bias_at({k: wq[k] for k in wq if k != "pre_norm_s"}, prep(s_np, dtype), Rows(),
                                            tm, queries)
    assert_parity(to_np(got[0])[queries], want, dtype, "single attention rows past the last full tile")


@pytest.mark.parametrize("c,rows,masked", [(384, 8300, True), (264, 8300, False), (384, 8215, False)])
def test_transition_wide_rows_dma_gemm_bf16(c, rows, masked):
    """Wide transitions over enough rows that their GEMMs run on the LDS-DMA
    kernel (64 or more 256 x 256 tiles): c = 384 (K = 384 and 1536, even
    stage counts) and c = 264 (K = 264 and 1056: odd stage counts, a k tail
    of 8 and 32, and an output width that ends 8 columns into a tile)."""
    dtype = DTYPES["bf16"]
    say(f"transition dma gemm c={c} rows={rows} masked={masked}")
    rng = np.random.default_rng(c + 7)
    x = rng.standard_normal((rows, c)).astype(np.float32)
    w = syn.transition_weights(c, 4, seed=19)
    rm = (rng.random(rows) > 0.3).astype(np.float32) if masked else None
    tw = P.pack_transition_torch({k: w[k] for k in ("layer_norm", "linear_a", "linear_b", "linear_out")}, dtype, "cuda")
    xt = device_tensor(x, dtype)
    got = kernels.transition(xt, tw, row_mask=None if rm is None else device_tensor(rm, dtype), residual=xt)
    torch.cuda.synchronize()
    xr = prep(x, dtype)
    want = xr + O.transition(xr, prep_tree(w, dtype), mask=rm)
    assert_parity(to_np(got), want, dtype, f"transition c={c} rows={rows}")


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_wide_dma_gemm_bf16(direction):
    """c_z = c_h = 384 at n = 96: the projections (9216 rows) run on the
    LDS-DMA GEMM, against the oracle."""
    dtype = DTYPES["bf16"]
    n, c = 96, 384
    say(f"trimul dma gemm c={c} n={n} {direction}")
    z = syn.pair_input(n, c, seed=41)
    m = mask_case("tail", n)
    w = syn.trimul_weights(c, c, seed=42)
    got = protenix.triangle_multiplication(device_tensor(z, dtype), device_tensor(m, dtype),
                                           P.trimul_to_protenix(w), direction)
    torch.cuda.synchronize()
    want = O.protenix_triangle_multiplication(prep(z, dtype), prep(m, dtype), prep_tree(w, dtype), direction)
    assert_parity(to_np(got), want, dtype, f"trimul c={c} n={n} {direction}")


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_wide_dma_gemm_bf16(starting):
    """c_z = 384 with 8 heads of 32 at n = 96: the q/k/v/g and output
    projections run on the LDS-DMA GEMM, against the oracle."""
    dtype = DTYPES["bf16"]
    n, c, heads = 96, 384, 8
    say(f"triattn dma gemm c={c} heads={heads} n={n} starting={starting}")
    z = syn.pair_input(n, c, seed=43)
    m = mask_case("tail", n)
    w = syn.triattn_weights(c, heads, 32, seed=44)
    got = protenix.triangle_attention(device_tensor(z, dtype), device_tensor(m, dtype), P.triattn_to_protenix(w),
                                      num_heads=heads, starting=starting)
    torch.cuda.synchronize()
    want = O.protenix_triangle_attention(prep(z, dtype), prep(m, dtype), prep_tree(w, dtype), num_heads=heads,
                                         starting=starting)
    mv = m if starting else m.T
    rows = mv.max(axis=1) > 0
    g, w_ = (to_np(got)[rows], want[rows]) if starting else (to_np(got)[:, rows], want[:, rows])
    assert_parity(g, w_, dtype, f"triattn c={c} n={n} starting={starting}")


@pytest.mark.parametrize("c_z,heads,n", [(128, 4, 40), (64, 4, 33), (384, 8, 20), (384, 8, 96)])
@pytest.mark.parametrize("starting", [True, False])
def test_ungated_triattn_is_twice_the_zero_gate(c_z, heads, n, starting):
    """An ungated module (g_weight None) on the fused, narrow and general
    paths, pinned to the oracle: with W_g = 0 the gate is sigmoid(0) = 1/2 at
    every position, so the ungated update is exactly twice the oracle's update
    with a zero gate weight (bf16; the halving is exact)."""
    dtype = DTYPES["bf16"]
    say(f"ungated triattn c_z={c_z} heads={heads} n={n} starting={starting}")
    z = syn.pair_input(n, c_z, seed=51)
    m = mask_case("tail", n)
    w = syn.triattn_weights(c_z, heads, 32, seed=52)
    w["attention"]["linear_g"]["weight"] = np.zeros_like(w["attention"]["linear_g"]["weight"])
    packed = dataclasses.replace(P.pack_triattn_protenix(P.triattn_to_protenix(w), dtype, "cuda"), g_weight=None)
    got = kernels.triattn(device_tensor(z, dtype), device_tensor(m, dtype), packed, starting=starting)
    torch.cuda.synchronize()
    want = 2.0 * O.protenix_triangle_attention(prep(z, dtype), prep(m, dtype), prep_tree(w, dtype), num_heads=heads,
                                               starting=starting)
    mv = m if starting else m.T
    rows = mv.max(axis=1) > 0
    g, w_ = (to_np(got)[rows], want[rows]) if starting else (to_np(got)[:, rows], want[:, rows])
    assert_parity(g, w_, dtype, f"ungated triattn c_z={c_z} starting={starting}")


@pytest.mark.parametrize("starting", [True, False])
def test_general_triattn_weights_back_to_back_match_separate(starting):
    """The general tri-attn path projects q|k|v|g in one GEMM: over the
    caller's weights when they sit back to back in one buffer, else over a
    copy in the workspace. Both give the same bits (c_z = 384, 8 heads,
    n = 96, bf16)."""
    dtype = DTYPES["bf16"]
    n, c, heads = 96, 384, 8
    say(f"triattn back-to-back weights n={n} starting={starting}")
    z = device_tensor(syn.pair_input(n, c, seed=53), dtype)
    m = device_tensor(mask_case("random", n), dtype)
    sep = P.pack_triattn_protenix(P.triattn_to_protenix(syn.triattn_weights(c, heads, 32, seed=54)), dtype, "cuda")
    cat = torch.cat([sep.q_weight, sep.k_weight, sep.v_weight, sep.g_weight], dim=0)
    hd = sep.q_weight.shape[0]
    b2b = dataclasses.replace(sep, q_weight=cat[:hd], k_weight=cat[hd:2 * hd], v_weight=cat[2 * hd:3 * hd],
                              g_weight=cat[3 * hd:])
    a = kernels.triattn(z, m, sep, starting=starting, residual=z)
    b = kernels.triattn(z, m, b2b, starting=starting, residual=z)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
