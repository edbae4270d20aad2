"""Full-size GPU parity: BASELINE configs 3 (N=1024 block), 4 (N=2048 layer and
the 48-layer trunk) and 5 (N=3072 block, unchunked).

At these sizes the float64 oracle cannot hold the whole problem, but every
output position of a sublayer depends on only a few lines of its input. Each
test runs the product path on the device, copies the lines it needs back to
the host and evaluates ``oracle/triangle.py``'s per-position restatements
(``triangle_multiplication_at``, ``triangle_attention_at``,
``boltz2_attention_pair_bias_at``, ``pair_bias_at``) there. Positions include
the edges of the 256 x 256 contraction tiles, the padded tail and fully
masked lines, so the multi-tile addressing of the contraction and the
attention's handling of masked rows are compared, not only their finiteness.

Bar: per position, relative error <= 2e-2 (bf16 mode, north star) against
the float64 oracle on the same bf16 values; updates are checked on their own
(kernel without residual) and the fused-residual output that the layer
carries forward is checked as well.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from foldjax_amd import kernels
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn
from foldjax_amd.pairformer import PairformerLayerWeights
from oracle import triangle as O
from tests.gpu_util import BF16_REL, prep_tree, say

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
LOG2E = 1.4426950408889634


class Lines:
    """Row / column access to a device ``[N, N, ...]`` tensor as float64 numpy
    (``g[i]`` is row i, ``g[:, j]`` column j), cached."""

    def __init__(self, t: torch.Tensor):
        self.t = t
        self.rows, self.cols = {}, {}

    def __getitem__(self, idx):
        if isinstance(idx, tuple):
            j = int(idx[1])
            if j not in self.cols:
                self.cols[j] = self.t[:, j].float().cpu().numpy().astype(np.float64)
            return self.cols[j]
        i = int(idx)
        if i not in self.rows:
            self.rows[i] = self.t[i].float().cpu().numpy().astype(np.float64)
        return self.rows[i]


def device_normal(shape, seed: int, dtype: torch.dtype = BF16) -> torch.Tensor:
    """``N(0,1)`` drawn on the device (seeded), in ``dtype`` (bf16: rounded)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(dtype)


def positions(n: int, n_real: int, seed: int, extra: int = 8) -> list[tuple[int, int]]:
    """Pairs over the contraction tile edges (multiples of 256 and their
    neighbours), the first padded token, the last token, random pairs, and
    one pair inside every 256 x 256 contraction tile: a random row of each
    tile row crossed with a random column of each tile column, so the
    (n/256)^2 tiles are each reached while the oracle evaluates only 2n/256
    lines."""
    edges = sorted({v for v in (0, 1, 255, 256, 511, 512, n // 2 + 3, n_real - 1, n_real, n - 1) if 0 <= v < n})
    rng = np.random.default_rng(seed)
    pick = rng.choice(len(edges), size=(16, 2))
    pairs = {(edges[a], edges[b]) for a, b in pick}
    pairs |= {(0, n - 1), (n - 1, 0), (n_real - 1, n_real - 1)}
    pairs |= {tuple(int(v) for v in rng.integers(0, n, size=2)) for _ in range(extra)}
    tile_rows = [min(t0 + int(rng.integers(0, 256)), n - 1) for t0 in range(0, n, 256)]
    tile_cols = [min(t0 + int(rng.integers(0, 256)), n - 1) for t0 in range(0, n, 256)]
    pairs |= {(i, j) for i in tile_rows for j in tile_cols}
    return sorted(pairs)


# the fp32-mode bar (north star): max-abs error against the float64 oracle
FP32_ABS = 1e-4


def check_rows(got: np.ndarray, want: np.ndarray, what: str, tol: float = BF16_REL, absolute: bool = False) -> float:
    """Per-position relative error (bf16 mode) or, with ``absolute``, the
    largest absolute error of any element (fp32 mode) within ``tol``."""
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    if absolute:
        errs = np.max(np.abs(got - want).reshape(len(got), -1), axis=-1)
    else:
        errs = np.linalg.norm(got - want, axis=-1) / np.maximum(np.linalg.norm(want, axis=-1), 1e-30)
    worst = int(np.argmax(errs))
    assert errs[worst] <= tol, f"{what}: position {worst} relative error {errs[worst]:.3e} > {tol}"
    return float(errs.max())


def gather(t: torch.Tensor, pos) -> np.ndarray:
    idx = torch.tensor(pos, device=t.device, dtype=torch.long)
    return t[idx[:, 0], idx[:, 1]].float().cpu().numpy().astype(np.float64)


def bar(dtype: torch.dtype) -> dict:
    """check_rows' bar for the pair track's dtype."""
    return {"tol": FP32_ABS, "absolute": True} if dtype == torch.float32 else {}


def check_trimul(z, mask_np, w, wq, direction, pos, what):
    """Update-only parity at ``pos``, then the fused-residual output that is
    carried forward. Returns that output."""
    m = torch.from_numpy(mask_np).to("cuda", z.dtype)
    upd = kernels.trimul(z, m, w, direction)
    out = kernels.trimul(z, m, w, direction, residual=z)
    zl = Lines(z)
    want = O.triangle_multiplication_at(zl, mask_np, wq, direction, pos)
    check_rows(gather(upd, pos), want, f"{what} update", **bar(z.dtype))
    check_rows(gather(out, pos), gather(z, pos) + want, f"{what} z+update", **bar(z.dtype))
    return out


def check_triattn(z, mask_np, w, wq, starting, pos, what):
    if z.dtype == torch.float32:
        # fp32 mode leaves out attention rows whose keys are all masked (the
        # padded tail), as the small-size fp32 tests do: the reference adds
        # -1e9 to every key there in fp32, which rounds the scores away (a
        # uniform softmax), where the float64 oracle keeps them
        pos = [(i, q) for i, q in pos if (mask_np[i] if starting else mask_np[:, i]).max() > 0]
    m = torch.from_numpy(mask_np).to("cuda", z.dtype)
    upd = kernels.triattn(z, m, w, starting=starting)
    out = kernels.triattn(z, m, w, starting=starting, residual=z)
    zl = Lines(z)
    want = O.triangle_attention_at(zl, mask_np, wq, num_heads=4, starting=starting, positions=pos)
    opos = pos if starting else [(q, i) for i, q in pos]  # output index of grid entry (i, q)
    assert bool(torch.isfinite(upd).all()), f"{what}: non-finite update (fully masked rows included)"
    check_rows(gather(upd, opos), want, f"{what} update", **bar(z.dtype))
    check_rows(gather(out, opos), gather(z, opos) + want, f"{what} z+update", **bar(z.dtype))
    return out


def run_layer_checked(n: int, n_real: int, seed: int, tag: str, z: torch.Tensor | None = None,
                      s: torch.Tensor | None = None, dtype: torch.dtype = BF16):
    """One Boltz-2 Pairformer layer at size n on the product kernels (the
    weights of ``syn.pairformer_layer_weights(seed)``), sublayer by sublayer,
    each checked at sampled positions; from the given ``[n, n, 128]`` z and
    ``[n, 384]`` s, or from seeded random ones. ``dtype``: both tracks' (bf16:
    the relative bar, fp32: max-abs 1e-4). Returns the layer's s and z."""
    w = syn.pairformer_layer_weights(seed=seed)
    wq = prep_tree(w, dtype)
    layer = PairformerLayerWeights.from_fields(w, dtype, "cuda")
    b = bar(dtype)
    tri = layer.triangle
    pm = syn.pair_mask(n, n_real)
    tm = syn.token_mask(n, n_real)
    if z is None:
        z = device_normal((n, n, 128), seed=seed + 100, dtype=dtype)
    if s is None:
        s = torch.from_numpy(syn.single_input(n, 384, seed=1)).to("cuda", dtype)
    pos = positions(n, n_real, seed)
    say(f"{tag}: n={n} n_real={n_real} tri-mul outgoing")
    z = check_trimul(z, pm, tri.tri_mul_out, wq["tri_mul_out"], "outgoing", pos, f"{tag} tri-mul out")
    say(f"{tag}: tri-mul incoming")
    z = check_trimul(z, pm, tri.tri_mul_in, wq["tri_mul_in"], "incoming", pos, f"{tag} tri-mul in")
    say(f"{tag}: tri-attn starting")
    z = check_triattn(z, pm, tri.tri_att_start, wq["tri_att_start"], True, pos, f"{tag} tri-attn start")
    say(f"{tag}: tri-attn ending")
    z = check_triattn(z, pm, tri.tri_att_end, wq["tri_att_end"], False, pos, f"{tag} tri-attn end")

    say(f"{tag}: pair transition with the single attention's pair bias")
    z_in = z
    z, pb = kernels.transition(z_in, layer.transition_z, residual=z_in, pair_bias_for=layer.attention)
    rows_in = gather(z_in, pos)
    want = rows_in + O.transition(rows_in, wq["transition_z"])
    check_rows(gather(z, pos), want, f"{tag} pair transition", **b)
    att = wq["attention"]
    want_pb = O.pair_bias_at(att, Lines(z), pos)  # [P, H], from the GPU's transition output
    idx = torch.tensor(pos, device="cuda", dtype=torch.long)
    got_pb = (pb[0][:, idx[:, 0], idx[:, 1]].float().cpu().numpy().astype(np.float64).T) / LOG2E
    check_rows(got_pb, want_pb, f"{tag} prepared pair bias", **b)

    say(f"{tag}: single attention with pair bias")
    s_in = s
    s = kernels.single_attention(s_in, None, torch.from_numpy(tm).to("cuda", dtype), layer.attention,
                                 residual=s_in, pair_bias=pb)
    s_np = s_in.float().cpu().numpy().astype(np.float64)
    s_ln = O.layer_norm(s_np, att["pre_norm_s"]["weight"], att["pre_norm_s"]["bias"])
    queries = sorted(q for q in {0, 1, n_real - 1, n_real, n - 1, n // 3} if q < n)
    want_s = s_np[queries] + O.boltz2_attention_pair_bias_at(att, s_ln, Lines(z), tm, queries)
    got_s = s.float().cpu().numpy().astype(np.float64)
    # padded queries see the same keys; their rows are part of the output too
    check_rows(got_s[queries], want_s, f"{tag} single attention", **b)

    say(f"{tag}: single transition")
    s_in = s
    s = kernels.transition(s_in, layer.transition_s, residual=s_in)
    s_np = s_in.float().cpu().numpy().astype(np.float64)
    check_rows(s.float().cpu().numpy().astype(np.float64), s_np + O.transition(s_np, wq["transition_s"]),
               f"{tag} single transition", **b)
    torch.cuda.synchronize()
    return s, z


def test_config3_block_sublayers_n1024():
    """the headline block at N=1024 (973 real tokens),
    every sublayer checked at sampled positions."""
    run_layer_checked(1024, 1024 - 51, seed=2, tag="config3")


def test_config3_block_fp32_single_track_n1024():
    """The precision split that ``bench.py`` times at config 3: the pair track
    in bf16, s and the single-track weights in fp32, as Boltz-2 runs it
    (``B2K/pairformer.py:182-199``). The pair transition then writes the
    attention's bias in fp32 from its epilogue (``transition128_pbf32_kernel``,
    its persistent multi-tile walk at N=1024):

    * its z equals the plain bf16 transition's, bit for bit, and matches the
      oracle at sampled positions (bf16 bar);
    * its fp32 bias matches ``LN_z(z) W_z^T`` of the GPU's bf16 z at sampled
      positions to the fp32 bar (max-abs 1e-4), and the whole bias equals the
      standalone fp32 pair-bias pass within that bar;
    * the fp32 single attention fed that bias matches the oracle's rows (given
      the GPU's z) to the fp32 bar, and so does the fp32 single transition;
    * ``PairformerLayerWeights.forward`` -- the bench's step -- gives the same
      s and z, bit for bit, as the sublayer-by-sublayer run checked here."""
    n, n_real, seed = 1024, 1024 - 51, 2
    f32 = torch.float32
    w = syn.pairformer_layer_weights(seed=seed)
    wq = prep_tree(w, BF16)
    att = w["attention"]  # the single track keeps its float32 weights
    layer = PairformerLayerWeights.from_fields(w, BF16, "cuda", single_dtype=f32)
    assert layer.attention.z_weight.dtype == f32
    pm_np = syn.pair_mask(n, n_real)
    tm_np = syn.token_mask(n, n_real)
    pm = torch.from_numpy(pm_np[None]).to("cuda", BF16)
    tm = torch.from_numpy(tm_np[None]).to("cuda", f32)
    z0 = device_normal((1, n, n, 128), seed=seed + 200)
    s0 = torch.from_numpy(syn.single_input(n, 384, seed=1, batch=1)).to("cuda", f32)
    pos = positions(n, n_real, seed + 1)

    say("config3 fp32 single track: triangle sublayers (bf16 pair track)")
    z_tri = layer.triangle.forward(z0, pm)
    say("config3 fp32 single track: pair transition with the fp32 pair bias")
    plain = kernels.transition(z_tri, layer.transition_z, residual=z_tri)
    z1, pb = kernels.transition(z_tri, layer.transition_z, residual=z_tri, pair_bias_for=layer.attention)
    torch.cuda.synchronize()
    assert pb.dtype == f32 and tuple(pb.shape) == (1, 16, n, n)
    assert torch.equal(z1, plain), "pbf32 transition z differs from the plain transition"
    rows_in = gather(z_tri[0], pos)
    check_rows(gather(z1[0], pos), rows_in + O.transition(rows_in, wq["transition_z"]), "config3 pair transition")

    zl = Lines(z1[0])
    want_pb = O.pair_bias_at(att, zl, pos)  # [P, H] from the GPU's bf16 z, fp32 weights
    idx = torch.tensor(pos, device="cuda", dtype=torch.long)
    got_pb = pb[0][:, idx[:, 0], idx[:, 1]].double().cpu().numpy().T / LOG2E
    err_pb = float(np.max(np.abs(got_pb - want_pb)))
    say(f"  fp32 pair bias at {len(pos)} positions: max-abs {err_pb:.2e}")
    assert err_pb <= 1e-4, f"fused fp32 pair bias max-abs {err_pb:.2e} > 1e-4"

    say("config3 fp32 single track: single attention from the fused bias and from z itself")
    s1 = kernels.single_attention(s0, None, tm, layer.attention, residual=s0, pair_bias=pb)
    s1_z = kernels.single_attention(s0, z1, tm, layer.attention, residual=s0)
    torch.cuda.synchronize()
    assert s1.dtype == f32
    err_paths = float((s1 - s1_z).abs().max())
    assert err_paths <= 1e-4, f"fused-bias vs standalone-bias attention max-abs {err_paths:.2e}"
    s_np = s0[0].double().cpu().numpy()
    s_ln = O.layer_norm(s_np, att["pre_norm_s"]["weight"], att["pre_norm_s"]["bias"])
    queries = sorted(q for q in {0, 1, 255, 256, n // 3, n_real - 1, n_real, n - 1} if q < n)
    want_s = s_np[queries] + O.boltz2_attention_pair_bias_at(att, s_ln, zl, tm_np, queries)
    err_s = float(np.max(np.abs(s1[0].double().cpu().numpy()[queries] - want_s)))
    say(f"  fp32 single attention rows {queries}: max-abs {err_s:.2e}")
    assert err_s <= 1e-4, f"fp32 single attention max-abs {err_s:.2e} > 1e-4"

    say("config3 fp32 single track: single transition")
    s2 = kernels.transition(s1, layer.transition_s, residual=s1)
    s1_np = s1[0].double().cpu().numpy()
    want_s2 = s1_np + O.transition(s1_np, w["transition_s"])
    err_t = float(np.max(np.abs(s2[0].double().cpu().numpy() - want_s2)))
    say(f"  fp32 single transition: max-abs {err_t:.2e}")
    assert err_t <= 1e-4, f"fp32 single transition max-abs {err_t:.2e} > 1e-4"

    say("config3 fp32 single track: the bench's layer forward")
    fs, fz = layer.forward(s0, z0, tm, pm)
    torch.cuda.synchronize()
    assert torch.equal(fz, z1) and torch.equal(fs, s2), "layer.forward differs from the checked sublayer run"


@pytest.mark.parametrize("n,n_real", [(512, 490), (1024, 973)])
def test_fp32_block_sublayers(n, n_real):
    """fp32 mode at multi-tile sizes: a whole layer with both tracks in
    float32 at N=512 (490 real tokens) and at the headline N=1024 (973), every
    sublayer and the prepared pair bias checked at sampled positions to the
    north star's fp32 bar, max-abs 1e-4 against the float64 oracle. The fp32
    paths run other kernels than the bf16 ones at these sizes (the fp32
    contraction over 2 x 2 and 4 x 4 tiles of 256, the fp32 flash kernels
    over several query tiles and key blocks, the fp32 transition with its
    fp32 pair-bias epilogue)."""
    run_layer_checked(n, n_real, seed=11, tag=f"fp32 n{n}", dtype=torch.float32)


def test_config4_layer_n2048():
    """BASELINE config 4's layer at N=2048 (all-ones mask), sublayer by sublayer."""
    run_layer_checked(2048, 2048, seed=5, tag="config4")


def test_config5_block_sublayers_n3072():
    """one unchunked block at N=3072 (3012 real tokens);
    the whole pair tensor and every workspace stay in HBM."""
    run_layer_checked(3072, 3012, seed=8, tag="config5")


@pytest.mark.parametrize("n,n_real", [(512, 500), (300, 290)])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_multi_tile_sampled(n, n_real, direction):
    """The two contraction kernels past one tile: N=512 (LDS-DMA kernel, 2x2
    tiles of 256) and N=300 (register-staged kernel, ragged second tile)."""
    say(f"trimul multi-tile n={n} {direction}")
    w = syn.trimul_weights(seed=11)
    wt = P.pack_trimul_torch(P.trimul_to_protenix(w), BF16, "cuda")
    pm = syn.pair_mask(n, n_real)
    z = device_normal((n, n, 128), seed=12)
    pos = [(i, j) for i in (0, 255, 256, n - 1) for j in (0, 127, 255, 256, n_real, n - 1)]
    check_trimul(z, pm, wt, prep_tree(w, BF16), direction, pos, f"n={n} {direction}")


@pytest.mark.parametrize("c_z,c_h", [(48, 128), (64, 64)])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_general_width_multi_tile_sampled(c_z, c_h, direction):
    """The general-width tri-mul at N=512: its contraction is the LDS-DMA
    kernel with row-major (not tile-blocked) output over 2x2 tiles of 256,
    the store addressing the fused widths never reach."""
    n, n_real = 512, 500
    say(f"trimul general width c_z={c_z} c_h={c_h} n={n} {direction}")
    w = syn.trimul_weights(c_z, c_h, seed=13)
    wt = P.pack_trimul_torch(P.trimul_to_protenix(w), BF16, "cuda")
    pm = syn.pair_mask(n, n_real)
    z = device_normal((n, n, c_z), seed=14)
    pos = [(i, j) for i in (0, 255, 256, n - 1) for j in (0, 127, 255, 256, n_real, n - 1)]
    check_trimul(z, pm, wt, prep_tree(w, BF16), direction, pos, f"general c_z={c_z} c_h={c_h} n={n} {direction}")


def test_trimul_persistent_batch_n768():
    """The persistent LDS-DMA contraction walks each XCD's share of the
    (batch, channel, tile) space; at N=768 (3x3 tiles of 256 per channel) and
    a batch of 3 the shares cut across channels and batch items and the
    workgroups take unequal tile counts. Each item of the batched call equals
    the item run alone, bit for bit, and item 1 matches the oracle at sampled
    positions."""
    n, n_real, batch = 768, 750, 3
    say(f"trimul persistent contraction n={n} batch={batch}")
    w = syn.trimul_weights(seed=31)
    wt = P.pack_trimul_torch(P.trimul_to_protenix(w), BF16, "cuda")
    pm = syn.pair_mask(n, n_real)
    zb = device_normal((batch, n, n, 128), seed=32)
    mb = torch.from_numpy(np.stack([pm] * batch)).to("cuda", BF16)
    for direction in ("outgoing", "incoming"):
        out = kernels.trimul(zb, mb, wt, direction)
        for i in range(batch):
            torch.testing.assert_close(out[i], kernels.trimul(zb[i], mb[i], wt, direction), rtol=0, atol=0)
        pos = [(i, j) for i in (0, 255, 256, 511, 512, n - 1) for j in (0, 256, 511, 512, n_real, n - 1)]
        check_trimul(zb[1], pm, wt, prep_tree(w, BF16), direction, pos, f"n={n} batch item 1 {direction}")


def test_config4_trunk_48_layers_n2048():
    """the 48-layer trunk at N=2048 (all-ones mask, each
    layer with its own weights). The whole stack must stay finite and its
    pair activations keep a bounded, non-degenerate scale; the last layer,
    fed the state 47 layers deep, is checked against the oracle sublayer by
    sublayer at sampled positions (every contraction tile among them), and
    the trunk's own forward of that layer must equal the checked run bit for
    bit."""
    n, layers = 2048, 48
    say(f"config4 trunk {layers} layers n={n}")
    z = device_normal((1, n, n, 128), seed=300)
    s = torch.from_numpy(syn.single_input(n, 384, seed=1, batch=1)).to("cuda", BF16)
    tm = torch.ones((1, n), device="cuda", dtype=BF16)
    pm = torch.ones((1, n, n), device="cuda", dtype=BF16)
    rms = []
    for l in range(layers):
        layer = PairformerLayerWeights.random(BF16, "cuda", seed=1000 + 7 * l)
        if l == layers - 1:
            say(f"  layer {l}: checked against the oracle")
            s_chk, z_chk = run_layer_checked(n, n, seed=1000 + 7 * l, tag=f"config4 trunk layer {l}", z=z[0], s=s[0])
            s, z = layer.forward(s, z, tm, pm)
            torch.cuda.synchronize()
            assert torch.equal(z[0], z_chk) and torch.equal(s[0], s_chk), "trunk layer differs from the checked run"
        else:
            s, z = layer.forward(s, z, tm, pm)
        if l % 8 == 7 or l == layers - 1:
            zf = z.float()
            assert bool(torch.isfinite(zf).all()), f"layer {l}: non-finite z"
            assert bool(torch.isfinite(s.float()).all()), f"layer {l}: non-finite s"
            rms.append(float(zf.pow(2).mean().sqrt()))
            say(f"  layer {l}: rms(z) = {rms[-1]:.3f}")
    torch.cuda.synchronize()
    assert all(0.5 < r < 1e3 for r in rms), f"pair activation scale out of range: {rms}"
    assert float(z.float().std()) > 0.1
    assert not math.isnan(rms[-1])
