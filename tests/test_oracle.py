"""Pins for the CPU oracle (oracle/triangle.py), independent of any GPU.

Each check is chosen so that a plausible mistake in the oracle fails it:
brute-force loops (tests/_brute.py) catch transposed operands and wrong
indices; torch's CPU ``layer_norm`` and ``scaled_dot_product_attention`` pin
the special cases that reduce to library routines; the reference's own
invariants (``T/models/protenix/test_triangle.py:142-166`` ending == transposed
starting, ``T/models/openfold3/test_torch_parity_triangle.py:96-106``
outgoing != incoming, ``T/models/protenix/test_pairformer.py:91-132`` padding
isolation, ``T/models/boltz2/test_triangle_attention_chunk_parity.py:43-69``
chunk invariance) pin what the loops leave open at larger sizes. The
``planted`` tests show that mistakes planted into the oracle are caught.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from foldjax_amd import synthetic as syn
from oracle import triangle as O
from tests import _brute as B
from tests.port_fields import of3_apb_fields as _of3_apb_fields
from tests.port_fields import of3_block_fields as _of3_block_fields
from tests.port_fields import px_apb_fields as _px_apb_fields
from tests.port_fields import px_block_fields as _px_block_fields


def _of3_attn(p):
    return {"layer_norm": p["layer_norm"], "linear_z": p["linear"], "mha": p["attention"]}


def _small(seed=0, n=3, c_z=4, c_h=5, heads=2, d=3):
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((n, n, c_z))
    mask = rng.integers(0, 2, size=(n, n)).astype(np.float64)
    mask[0, :] = 1.0  # keep at least one valid key per row for the brute softmax
    tm = syn.trimul_weights(c_z, c_h, seed=seed + 10)
    ta = syn.triattn_weights(c_z, heads, d, seed=seed + 20)
    return z, mask, tm, ta


# --------------------------------------------------------------- brute force


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_matches_brute_force(direction):
    z, mask, tm, _ = _small(seed=1)
    want = np.array(B.trimul(z.tolist(), mask.tolist(), B.tolist(tm), direction == "outgoing"))
    got_px = O.protenix_triangle_multiplication(z, mask, tm, direction)
    got_of = O.openfold3_triangle_multiplication(z, tm, outgoing=direction == "outgoing", mask=mask)
    got_b2 = O.boltz2_triangle_multiplication(O.trimul_torch_to_boltz2(tm), z, mask, direction)
    for got in (got_px, got_of, got_b2):
        np.testing.assert_allclose(got, want, rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_matches_brute_force(starting):
    z, mask, _, ta = _small(seed=2, n=4, heads=2, d=3)
    want = np.array(B.triattn(z.tolist(), mask.tolist(), B.tolist(ta), 2, starting))
    got_px = O.protenix_triangle_attention(z, mask, ta, num_heads=2, starting=starting)
    got_of = O.openfold3_triangle_attention(z, _of3_attn(ta), no_heads=2, mask=mask, starting=starting)
    got_b2 = O.boltz2_triangle_attention(O.triattn_torch_to_boltz2(ta), z, mask, starting=starting)
    for got in (got_px, got_of, got_b2):
        np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


def test_contraction_brute_force_both_directions():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((5, 5, 2))
    b = rng.standard_normal((5, 5, 2))
    out = O.triangle_contract(a, b, "outgoing")
    inc = O.triangle_contract(a, b, "incoming")
    for i in range(5):
        for j in range(5):
            for c in range(2):
                assert abs(out[i, j, c] - sum(a[i, k, c] * b[j, k, c] for k in range(5))) < 1e-12
                assert abs(inc[i, j, c] - sum(a[k, i, c] * b[k, j, c] for k in range(5))) < 1e-12
    with pytest.raises(ValueError, match="Unsupported triangle multiplication direction"):
        O.triangle_contract(a, b, "sideways")


# ----------------------------------------------------------- library routines


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((7, 33)) * 3 + 1
    w = rng.standard_normal(33)
    b = rng.standard_normal(33)
    want = torch.nn.functional.layer_norm(
        torch.from_numpy(x), (33,), torch.from_numpy(w), torch.from_numpy(b), eps=1e-5
    ).numpy()
    np.testing.assert_allclose(O.layer_norm(x, w, b, 1e-5), want, rtol=1e-12, atol=1e-12)


def test_attention_rows_matches_torch_sdpa():
    """Zero-free bias + mask reduce the row attention to textbook SDPA."""
    rng = np.random.default_rng(5)
    i_rows, heads, n, d = 3, 2, 9, 4
    q = rng.standard_normal((i_rows, heads, n, d))
    k = rng.standard_normal((i_rows, heads, n, d))
    v = rng.standard_normal((i_rows, heads, n, d))
    mask = (rng.random((i_rows, n)) > 0.3).astype(np.float64)
    mask[:, 0] = 1
    mb = (1e9 * (mask - 1.0))[:, None, None, :]
    tb = rng.standard_normal((1, heads, n, n))
    got = O.attention_rows(q / np.sqrt(d), k, v, mb, tb)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
        attn_mask=torch.from_numpy(mb + tb),
    ).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


def test_attention_core_scale_applied_inside():
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((1, 2, 2, 5, 8)) for _ in range(3))
    tb = rng.standard_normal((1, 1, 2, 5, 5))
    mb = np.zeros((1, 2, 1, 1, 5))
    got = O.attention_core(q, k, v, tb, mb, scale=8 ** -0.5)
    want = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(t) for t in (q, k, v)), attn_mask=torch.from_numpy(tb + mb)
    ).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


# ------------------------------------------------------------- invariants


def _swap_ab(tm):
    out = dict(tm)
    out["linear_a_p"], out["linear_b_p"] = tm["linear_b_p"], tm["linear_a_p"]
    out["linear_a_g"], out["linear_b_g"] = tm["linear_b_g"], tm["linear_a_g"]
    return out


def test_incoming_is_swapped_outgoing_with_a_b_exchanged():
    """incoming(z)[i,j] = outgoing(z^T; a<->b)[j,i] (``B2T/triangle.py:112-121``)."""
    rng = np.random.default_rng(7)
    z = rng.standard_normal((9, 9, 8))
    mask = (rng.random((9, 9)) > 0.2).astype(np.float64)
    tm = syn.trimul_weights(8, 6, seed=7)
    inc = O.protenix_triangle_multiplication(z, mask, tm, "incoming")
    out_t = O.protenix_triangle_multiplication(
        np.swapaxes(z, 0, 1), mask.T, _swap_ab(tm), "outgoing"
    )
    np.testing.assert_allclose(inc, np.swapaxes(out_t, 0, 1), rtol=1e-11, atol=1e-11)


def test_outgoing_differs_from_incoming():
    z, mask, tm, _ = _small(seed=8, n=6, c_z=8, c_h=8)
    a = O.protenix_triangle_multiplication(z, mask, tm, "outgoing")
    b = O.protenix_triangle_multiplication(z, mask, tm, "incoming")
    assert np.max(np.abs(a - b)) > 1e-2


def test_ending_is_transposed_starting():
    rng = np.random.default_rng(9)
    z = rng.standard_normal((7, 7, 8))
    mask = (rng.random((7, 7)) > 0.2).astype(np.float64)
    ta = syn.triattn_weights(8, 2, 4, seed=9)
    end = O.protenix_triangle_attention(z, mask, ta, num_heads=2, starting=False)
    start_t = O.protenix_triangle_attention(np.swapaxes(z, 0, 1), mask.T, ta, num_heads=2, starting=True)
    np.testing.assert_allclose(end, np.swapaxes(start_t, 0, 1), rtol=1e-12, atol=1e-12)


def test_row_block_invariance():
    rng = np.random.default_rng(10)
    q, k, v = (rng.standard_normal((11, 2, 6, 4)) for _ in range(3))
    mb = (1e9 * ((rng.random((11, 6)) > 0.3) - 1.0))[:, None, None, :]
    tb = rng.standard_normal((1, 2, 6, 6))
    ref = O.attention_rows(q, k, v, mb, tb, row_block=11)
    for blk in (1, 4, 10, 16):
        np.testing.assert_allclose(O.attention_rows(q, k, v, mb, tb, row_block=blk), ref, rtol=0, atol=1e-14)


def test_fully_masked_row_is_finite():
    z, _, _, ta = _small(seed=11, n=5, heads=2, d=3)
    mask = np.ones((5, 5))
    mask[2, :] = 0.0
    out = O.protenix_triangle_attention(z, mask, ta, num_heads=2)
    assert np.all(np.isfinite(out))


@pytest.mark.parametrize("op", ["trimul_out", "trimul_in", "att_start", "att_end"])
def test_padding_isolation(op):
    """Adversarial padded tokens leave the valid region unchanged."""
    rng = np.random.default_rng(12)
    n, pad = 5, 3
    z = rng.standard_normal((n, n, 8))
    zp = np.pad(z, ((0, pad), (0, pad), (0, 0)))
    zp[n:, :, :] = -1.0e6
    zp[:, n:, :] = 1.0e6
    mask = syn.pair_mask(n + pad, n)
    tm = syn.trimul_weights(8, 8, seed=12)
    ta = syn.triattn_weights(8, 2, 4, seed=12)
    if op.startswith("trimul"):
        d = "outgoing" if op.endswith("out") else "incoming"
        want = O.protenix_triangle_multiplication(z, np.ones((n, n)), tm, d)
        got = O.protenix_triangle_multiplication(zp, mask, tm, d)
    else:
        s = op.endswith("start")
        want = O.protenix_triangle_attention(z, np.ones((n, n)), ta, num_heads=2, starting=s)
        got = O.protenix_triangle_attention(zp, mask, ta, num_heads=2, starting=s)
    np.testing.assert_allclose(got[:n, :n], want, rtol=1e-9, atol=1e-9)


def test_batch_axis_is_independent():
    rng = np.random.default_rng(13)
    z = rng.standard_normal((2, 6, 6, 8))
    mask = np.ones((2, 6, 6))
    tm = syn.trimul_weights(8, 8, seed=13)
    ta = syn.triattn_weights(8, 2, 4, seed=13)
    bm = O.protenix_triangle_multiplication(z, mask, tm, "incoming")
    ba = O.protenix_triangle_attention(z, mask, ta, num_heads=2, starting=False)
    for b in range(2):
        np.testing.assert_allclose(bm[b], O.protenix_triangle_multiplication(z[b], mask[b], tm, "incoming"), atol=1e-12)
        np.testing.assert_allclose(ba[b], O.protenix_triangle_attention(z[b], mask[b], ta, num_heads=2, starting=False), atol=1e-12)


# ----------------------------------------------- planted mistakes are caught


def test_planted_transposed_operand_is_caught(monkeypatch):
    z, mask, tm, _ = _small(seed=14)
    want = np.array(B.trimul(z.tolist(), mask.tolist(), B.tolist(tm), False))
    real = O.triangle_contract

    def wrong(a, b, direction):  # incoming computed as a[k,i] b[j,k]: b transposed
        if direction == "incoming":
            return real(a, np.swapaxes(b, -2, -3), "incoming")
        return real(a, b, direction)

    monkeypatch.setattr(O, "triangle_contract", wrong)
    got = O.protenix_triangle_multiplication(z, mask, tm, "incoming")
    assert np.max(np.abs(got - want)) > 1e-3


def test_planted_dropped_bias_term_is_caught(monkeypatch):
    z, mask, _, ta = _small(seed=15, n=4)
    want = np.array(B.triattn(z.tolist(), mask.tolist(), B.tolist(ta), 2, True))
    real = O.attention_rows
    monkeypatch.setattr(O, "attention_rows", lambda q, k, v, mb, tb, row_block=16: real(q, k, v, mb, 0.0 * tb))
    got = O.protenix_triangle_attention(z, mask, ta, num_heads=2)
    assert np.max(np.abs(got - want)) > 1e-3


def test_planted_wrong_bias_index_is_caught(monkeypatch):
    """A bias read as [h, key, query] instead of [h, query, key] is caught."""
    z, mask, _, ta = _small(seed=16, n=4)
    want = np.array(B.triattn(z.tolist(), mask.tolist(), B.tolist(ta), 2, True))
    real = O.attention_rows
    monkeypatch.setattr(O, "attention_rows", lambda q, k, v, mb, tb, row_block=16: real(q, k, v, mb, np.swapaxes(tb, -1, -2)))
    got = O.protenix_triangle_attention(z, mask, ta, num_heads=2)
    assert np.max(np.abs(got - want)) > 1e-3


# ------------------------------------------- transition, single attention


def test_transition_matches_brute_force():
    rng = np.random.default_rng(20)
    x = rng.standard_normal((3, 5))
    p = syn.transition_weights(5, seed=20)
    want = np.array([B.transition_row(row, B.tolist(p)) for row in x.tolist()])
    np.testing.assert_allclose(O.transition(x, p), want, rtol=1e-11, atol=1e-11)
    m = np.array([1.0, 0.0, 1.0])
    np.testing.assert_allclose(O.transition(x, p, mask=m), want * m[:, None], rtol=1e-11, atol=1e-11)


def test_attention_pair_bias_matches_torch_sdpa():
    """The Boltz-2 attention with pair bias equals gated torch SDPA with the
    pair bias and key mask as an additive mask (``B2P/attention.py:82-115``)."""
    rng = np.random.default_rng(21)
    b, n, c_s, c_z, h = 2, 7, 24, 8, 4
    s = rng.standard_normal((b, n, c_s))
    z = rng.standard_normal((b, n, n, c_z))
    mask = (rng.random((b, n)) > 0.3).astype(np.float64)
    mask[:, 0] = 1.0
    p = syn.single_attention_weights(c_s, c_z, h, seed=21)
    got = O.boltz2_attention_pair_bias(p, s, z, mask)
    T = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float64))  # noqa: E731
    lin = lambda x, name: x @ T(p[name]["weight"]).T  # noqa: E731
    st = T(s)
    q = (lin(st, "proj_q") + T(p["proj_q"]["bias"])).reshape(b, n, h, -1).transpose(1, 2)
    k = lin(st, "proj_k").reshape(b, n, h, -1).transpose(1, 2)
    v = lin(st, "proj_v").reshape(b, n, h, -1).transpose(1, 2)
    zl = torch.nn.functional.layer_norm(T(z), (c_z,), T(p["proj_z_norm"]["weight"]), T(p["proj_z_norm"]["bias"]), 1e-5)
    bias = (zl @ T(p["proj_z"]["weight"]).T).permute(0, 3, 1, 2)
    am = bias + ((1.0 - T(mask)) * -1e6)[:, None, None, :]
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=am).transpose(1, 2).reshape(b, n, c_s)
    want = (torch.sigmoid(lin(st, "proj_g")) * o) @ T(p["proj_o"]["weight"]).T
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-10)


def test_pairformer_layer_padding_isolation():
    """Padded tokens with adversarial values leave the valid region of both
    tracks unchanged (cf. ``T/models/protenix/test_pairformer.py:91-132``)."""
    rng = np.random.default_rng(22)
    n, pad, c_s, c_z = 4, 2, 16, 8
    w = syn.pairformer_layer_weights(c_s=c_s, c_z=c_z, heads_pair=2, heads_single=4, seed=22)
    s = rng.standard_normal((1, n, c_s))
    z = rng.standard_normal((1, n, n, c_z))
    want_s, want_z = O.boltz2_pairformer_layer(w, s, z, np.ones((1, n)), np.ones((1, n, n)))
    sp = np.pad(s, ((0, 0), (0, pad), (0, 0)))
    sp[:, n:] = 1e6
    zp = np.pad(z, ((0, 0), (0, pad), (0, pad), (0, 0)))
    zp[:, n:, :] = -1e6
    zp[:, :, n:] = 1e6
    tm = syn.token_mask(n + pad, n)[None]
    got_s, got_z = O.boltz2_pairformer_layer(w, sp, zp, tm, syn.pair_mask(n + pad, n)[None])
    np.testing.assert_allclose(got_s[:, :n], want_s, rtol=1e-8, atol=1e-8)
    np.testing.assert_allclose(got_z[:, :n, :n], want_z, rtol=1e-8, atol=1e-8)


# ------------------------------------- sampled positions (full-size checks)


def _all_positions(n):
    return [(i, j) for i in range(n) for j in range(n)]


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_at_matches_full_oracle(direction):
    """The per-position restatement equals the full tri-mul at every position,
    with a random mask, and at n = 3 equals the brute-force loops."""
    rng = np.random.default_rng(30)
    n, c = 9, 8
    z = rng.standard_normal((n, n, c))
    mask = (rng.random((n, n)) > 0.3).astype(np.float64)
    tm = syn.trimul_weights(c, c, seed=30)
    full = O.protenix_triangle_multiplication(z, mask, tm, direction)
    pos = _all_positions(n)
    got = O.triangle_multiplication_at(z, mask, tm, direction, pos)
    np.testing.assert_allclose(got, np.stack([full[i, j] for i, j in pos]), rtol=1e-11, atol=1e-11)
    zs, ms, tms, _ = _small(seed=31)
    want = np.array(B.trimul(zs.tolist(), ms.tolist(), B.tolist(tms), direction == "outgoing"))
    got = O.triangle_multiplication_at(zs, ms, tms, direction, _all_positions(3))
    np.testing.assert_allclose(got, want.reshape(9, -1), rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_at_matches_full_oracle(starting):
    rng = np.random.default_rng(32)
    n, c = 8, 8
    z = rng.standard_normal((n, n, c))
    mask = (rng.random((n, n)) > 0.3).astype(np.float64)
    mask[3, :] = 0.0  # a fully masked line
    ta = syn.triattn_weights(c, 2, 4, seed=32)
    full = O.protenix_triangle_attention(z, mask, ta, num_heads=2, starting=starting)
    pos = _all_positions(n)
    got = O.triangle_attention_at(z, mask, ta, num_heads=2, starting=starting, positions=pos)
    # (i, q) of the attention grid is [i, q] of the output (starting) or [q, i] (ending)
    want = np.stack([full[i, q] if starting else full[q, i] for i, q in pos])
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


def test_attention_pair_bias_at_matches_full_oracle():
    rng = np.random.default_rng(33)
    n, c_s, c_z, h = 9, 24, 8, 4
    s = rng.standard_normal((1, n, c_s))
    z = rng.standard_normal((1, n, n, c_z))
    mask = (rng.random((1, n)) > 0.3).astype(np.float64)
    mask[:, 0] = 1.0
    p = syn.single_attention_weights(c_s, c_z, h, seed=33)
    full = O.boltz2_attention_pair_bias(p, s, z, mask)[0]
    got = O.boltz2_attention_pair_bias_at(p, s[0], z[0], mask[0], list(range(n)))
    np.testing.assert_allclose(got, full, rtol=1e-10, atol=1e-10)
    pos = [(0, 0), (3, 7), (8, 2)]
    pb = O.pair_bias_at(p, z[0], pos)
    zl = O.layer_norm(z[0], p["proj_z_norm"]["weight"], p["proj_z_norm"]["bias"])
    for r, (i, j) in enumerate(pos):
        np.testing.assert_allclose(pb[r], zl[i, j] @ np.asarray(p["proj_z"]["weight"], np.float64).T, rtol=1e-12)


def test_planted_swapped_position_is_caught():
    """Reading z[j, i] instead of z[i, j] for the output gate is caught by the
    comparison with the full oracle."""
    rng = np.random.default_rng(34)
    n, c = 6, 8
    z = rng.standard_normal((n, n, c))
    tm = syn.trimul_weights(c, c, seed=34)
    full = O.protenix_triangle_multiplication(z, None, tm, "outgoing")
    got = O.triangle_multiplication_at(np.swapaxes(z, 0, 1).copy(), None, tm, "incoming", [(1, 4)])
    # incoming on z^T reads the same a/b lines as outgoing on z, but its gate
    # is z^T[1, 4] = z[4, 1]: the planted swap must differ from z's answer
    assert np.max(np.abs(got[0] - full[1, 4])) > 1e-3


# ------------------- Protenix / OpenFold3 single attention and Pairformer blocks


def test_gated_attention_matches_torch_sdpa():
    """The Protenix/OpenFold3 gated attention equals torch SDPA with the bias
    as an additive mask, gated and projected (``PXP/attention.py:60-99``)."""
    rng = np.random.default_rng(40)
    b, n, c, h = 2, 6, 12, 3
    x = rng.standard_normal((b, n, c))
    p = syn.single_attention_weights(c, 4, h, seed=40)
    att = _px_apb_fields(p)["attention"]
    bias = rng.standard_normal((b, h, n, n))
    got = O.gated_attention(x, x, att, h, (bias,))
    T = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float64))  # noqa: E731
    xt = T(x)
    lin = lambda name: xt @ T(p[name]["weight"]).T  # noqa: E731
    q = (lin("proj_q") + T(p["proj_q"]["bias"])).reshape(b, n, h, -1).transpose(1, 2)
    k = lin("proj_k").reshape(b, n, h, -1).transpose(1, 2)
    v = lin("proj_v").reshape(b, n, h, -1).transpose(1, 2)
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=T(bias)).transpose(1, 2).reshape(b, n, c)
    want = (torch.sigmoid(lin("proj_g")) * o) @ T(p["proj_o"]["weight"]).T
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-10)


def test_protenix_and_openfold3_attention_pair_bias_equal_boltz2():
    """With ``LN_a`` = Boltz-2's ``pre_norm_s`` the three ports' attentions with
    pair bias are one function: Protenix with an extra key bias ``inf (mask - 1)``
    (ranks [N, N] and [B, N, N] aligned as ``PXP/attention.py:140-150``),
    OpenFold3 with the key mask, Boltz-2 (pinned to torch SDPA above) on
    ``LN(s)``."""
    rng = np.random.default_rng(41)
    b, n, c_s, c_z, h = 2, 7, 24, 8, 4
    s = rng.standard_normal((b, n, c_s))
    z = rng.standard_normal((b, n, n, c_z))
    mask = (rng.random((b, n)) > 0.3).astype(np.float64)
    mask[:, 0] = 1.0
    p = syn.single_attention_weights(c_s, c_z, h, seed=41)
    s_ln = O.layer_norm(s, p["pre_norm_s"]["weight"], p["pre_norm_s"]["bias"])
    want = O.boltz2_attention_pair_bias(p, s_ln, z, mask, inf=1e9)
    of3 = O.openfold3_attention_pair_bias(s, z, _of3_apb_fields(p), no_heads=h, mask=mask, inf=1e9)
    np.testing.assert_allclose(of3, want, rtol=1e-10, atol=1e-10)
    extra = np.broadcast_to(((mask - 1.0) * 1e9)[:, None, :], (b, n, n))
    px = O.protenix_attention_pair_bias(s, z, _px_apb_fields(p), num_heads=h, extra_attn_bias=extra)
    np.testing.assert_allclose(px, want, rtol=1e-10, atol=1e-10)
    # a rank-2 extra bias broadcasts over batch and heads
    one = O.protenix_attention_pair_bias(s[:1], z[:1], _px_apb_fields(p), num_heads=h, extra_attn_bias=extra[0])
    np.testing.assert_allclose(one, want[:1], rtol=1e-10, atol=1e-10)


def test_protenix_block_unmasked_equals_boltz2_layer():
    """Without padding the Protenix block is the Boltz-2 layer under the field
    mapping (``PXK/pairformer.py:49-180`` vs ``B2K/pairformer.py:100-206``):
    same sublayer order, heads from the weight shapes, ``LN_a`` = ``pre_norm_s``."""
    rng = np.random.default_rng(42)
    n, c_s, c_z = 5, 16, 8
    w = syn.pairformer_layer_weights(c_s=c_s, c_z=c_z, heads_pair=2, heads_single=4, seed=42)
    s = rng.standard_normal((1, n, c_s))
    z = rng.standard_normal((1, n, n, c_z))
    want_s, want_z = O.boltz2_pairformer_layer(w, s, z, np.ones((1, n)), np.ones((1, n, n)))
    for pm in (None, np.ones((1, n, n))):
        got_s, got_z = O.protenix_pairformer_block(s, z, pm, _px_block_fields(w))
        np.testing.assert_allclose(got_z, want_z, rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(got_s, want_s, rtol=1e-10, atol=1e-10)


def test_protenix_block_isolates_adversarial_padded_tokens():
    """``T/models/protenix/test_pairformer.py:91-132``: padded tokens set to
    +-1e6 leave the real block unchanged, and the padded region of both tracks
    is exactly zero (the pair and single gates)."""
    rng = np.random.default_rng(43)
    n, pad, c_s, c_z = 3, 2, 16, 8
    w = syn.pairformer_layer_weights(c_s=c_s, c_z=c_z, heads_pair=2, heads_single=4, seed=43)
    s = rng.standard_normal((1, n, c_s))
    z = rng.standard_normal((1, n, n, c_z))
    want_s, want_z = O.protenix_pairformer_block(s, z, np.ones((1, n, n)), _px_block_fields(w))
    sp = np.pad(s, ((0, 0), (0, pad), (0, 0)))
    sp[:, n:] = 1e6
    zp = np.pad(z, ((0, 0), (0, pad), (0, pad), (0, 0)))
    zp[:, n:] = -1e6
    zp[:, :, n:] = 1e6
    got_s, got_z = O.protenix_pairformer_block(sp, zp, syn.pair_mask(n + pad, n)[None], _px_block_fields(w))
    np.testing.assert_allclose(got_s[:, :n], want_s, rtol=1e-8, atol=1e-8)
    np.testing.assert_allclose(got_z[:, :n, :n], want_z, rtol=1e-8, atol=1e-8)
    assert not np.any(got_s[:, n:]) and not np.any(got_z[:, n:]) and not np.any(got_z[:, :, n:])


def test_protenix_block_gate_is_boolean_and_masked_pairs_are_zero():
    """A pair mask with a hole between two valid tokens and a fractional entry:
    the hole is zero in z, the fractional entry is gated as True
    (``pair_valid = bool(pair_mask)``, ``PXK/pairformer.py:74-76``), and the
    entry values of z at the hole do not matter (z is gated on entry)."""
    rng = np.random.default_rng(44)
    n, c_s, c_z = 5, 16, 8
    w = syn.pairformer_layer_weights(c_s=c_s, c_z=c_z, heads_pair=2, heads_single=4, seed=44)
    s = rng.standard_normal((1, n, c_s))
    z = rng.standard_normal((1, n, n, c_z))
    pm = np.ones((1, n, n))
    pm[0, 1, 3] = 0.0
    pm[0, 2, 4] = 0.5
    got_s, got_z = O.protenix_pairformer_block(s, z, pm, _px_block_fields(w))
    assert not np.any(got_z[0, 1, 3]) and np.all(np.abs(got_z[0, 2, 4]) > 0)
    z2 = z.copy()
    z2[0, 1, 3] = 50.0
    s2, zz2 = O.protenix_pairformer_block(s, z2, pm, _px_block_fields(w))
    np.testing.assert_array_equal(zz2, got_z)
    np.testing.assert_array_equal(s2, got_s)


def test_openfold3_block_equals_boltz2_layer_without_transition_masks():
    """With ``mask_transition=False`` the OpenFold3 block is the Boltz-2 layer
    (``OF3/pairformer.py:42-102`` vs ``B2K/pairformer.py:100-206``): the key
    masks differ only in ``inf`` (1e9 vs 1e6), which underflows the same."""
    rng = np.random.default_rng(45)
    n, n_real, c_s, c_z = 6, 4, 16, 8
    w = syn.pairformer_layer_weights(c_s=c_s, c_z=c_z, heads_pair=2, heads_single=4, seed=45)
    s = rng.standard_normal((1, n, c_s))
    z = rng.standard_normal((1, n, n, c_z))
    tm = syn.token_mask(n, n_real)[None]
    pm = syn.pair_mask(n, n_real)[None]
    want_s, want_z = O.boltz2_pairformer_layer(w, s, z, tm, pm)
    got_s, got_z = O.openfold3_pairformer_block(s, z, _of3_block_fields(w), single_mask=tm, pair_mask=pm,
                                                no_heads_pair=2, no_heads_pair_bias=4, mask_transition=False)
    np.testing.assert_allclose(got_z, want_z, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(got_s, want_s, rtol=1e-10, atol=1e-10)
    # with the transition masks the padded rows of both tracks are zeroed updates
    ms, mz = O.openfold3_pairformer_block(s, z, _of3_block_fields(w), single_mask=tm, pair_mask=pm,
                                          no_heads_pair=2, no_heads_pair_bias=4, mask_transition=True)
    v = slice(0, n_real)
    np.testing.assert_allclose(mz[:, v, v], want_z[:, v, v], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(ms[:, v], want_s[:, v], rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_row_subset_equals_full_rows(starting):
    """``rows=`` gives exactly those rows of the attention grid (the CPU
    baseline times a row sample), and float32 mode stays close to float64."""
    rng = np.random.default_rng(50)
    n, c = 11, 8
    z = rng.standard_normal((n, n, c))
    mask = (rng.random((n, n)) > 0.2).astype(np.float64)
    w = syn.triattn_weights(c, 2, 4, seed=50)
    full = O.protenix_triangle_attention(z, mask, w, num_heads=2, starting=starting)
    grid = full if starting else np.swapaxes(full, 0, 1)
    rows = [0, 4, 10]
    got = O.protenix_triangle_attention(z, mask, w, num_heads=2, starting=starting, rows=rows)
    np.testing.assert_allclose(got, grid[rows], rtol=1e-12, atol=1e-12)
    with O.compute_dtype(np.float32):
        f32 = O.protenix_triangle_attention(z, mask, w, num_heads=2, starting=starting, rows=rows)
    assert f32.dtype == np.float32
    np.testing.assert_allclose(f32, grid[rows], rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------ golden fixtures


def test_oracle_matches_golden_fixtures():
    """Every committed fixture (inputs and the brute-force loops' outputs,
    tests/golden/make_golden.py) against the oracle, both directions and
    nodes, float32 and bf16-rounded inputs."""
    from tests.golden import fixtures

    n_cases = 0
    for c in fixtures.cases("trimul"):
        for d in ("outgoing", "incoming"):
            got = O.protenix_triangle_multiplication(c["z"], c["mask"], c["w"], d)
            np.testing.assert_allclose(got, c["out"][d], rtol=1e-9, atol=1e-9, err_msg=f"{c['tag']} {c['name']} {d}")
            n_cases += 1
    for c in fixtures.cases("triattn"):
        for node in ("starting", "ending"):
            got = O.protenix_triangle_attention(c["z"], c["mask"], c["w"], num_heads=c["heads"],
                                                starting=node == "starting")
            np.testing.assert_allclose(got, c["out"][node], rtol=1e-9, atol=1e-9,
                                       err_msg=f"{c['tag']} {c['name']} {node}")
            n_cases += 1
    assert n_cases == 40


# ---------------------------------------------------------------------------
# bfloat16 programs (analysis mode of the oracle)
# ---------------------------------------------------------------------------


def test_bf16_rounding_equals_torch():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(4096) * 10.0 ** rng.integers(-30, 30, 4096),
        # exact ties between two bfloat16 neighbours, both parities
        (np.arange(1, 257, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40]),
    ]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float64).numpy()
    got = O.bf16(x)
    assert np.array_equal(got, want)
    assert np.isnan(O.bf16(np.array([np.nan])))[0]


def _ta_case(seed, n, scale):
    rng = np.random.default_rng(seed)
    z = O.bf16(rng.standard_normal((n, n, 16)))
    w = syn.cast_tree(syn.triattn_weights(16, 2, 8, seed=seed + 1), O.bf16)
    for name in ("linear_q", "linear_k"):  # logits of size ~ scale
        w["attention"][name]["weight"] = O.bf16(np.asarray(w["attention"][name]["weight"]) * np.sqrt(scale))
    return z, w


def test_bf16_programs_round_only_inside_their_context():
    z, w = _ta_case(0, 6, 1.0)
    m = np.ones((6, 6))
    exact = O.protenix_triangle_attention(z, m, w, num_heads=2)
    with O.bf16_program("protenix"):
        px = O.protenix_triangle_attention(z, m, w, num_heads=2)
    with O.bf16_program(None):
        none = O.protenix_triangle_attention(z, m, w, num_heads=2)
    assert np.array_equal(none, exact)
    assert np.array_equal(O.protenix_triangle_attention(z, m, w, num_heads=2), exact)
    # bfloat16 storage moves the result, by a bfloat16-sized amount
    rel = np.linalg.norm(px - exact) / np.linalg.norm(exact)
    assert 1e-4 < rel < 2e-2, rel
    with pytest.raises(ValueError):
        with O.bf16_program("alphafold"):
            pass


def test_protenix_program_rounds_logits_boltz2_program_does_not():
    """On bfloat16 q, k, v: with logits of a few hundred, bfloat16 logits
    (spacing 1-2) move the softmax weights by factors of e, while Boltz-2's
    float32 scores leave only the output rounding."""
    rng = np.random.default_rng(5)
    errs = {}
    for scale in (1.0, 300.0):
        q = O.bf16(rng.standard_normal((4, 2, 16, 8)) * np.sqrt(scale / 8))
        k = O.bf16(rng.standard_normal((4, 2, 16, 8)) * np.sqrt(scale / 8))
        v = O.bf16(rng.standard_normal((4, 2, 16, 8)))
        mb = np.zeros((4, 1, 1, 16))
        tb = O.bf16(rng.standard_normal((1, 2, 16, 16)))
        exact = O.attention_rows(q, k, v, mb, tb)
        for port in ("boltz2", "protenix"):
            with O.bf16_program(port):
                got = O.attention_rows(q, k, v, mb, tb)
            errs[port, scale] = np.linalg.norm(got - exact) / np.linalg.norm(exact)
    assert errs["boltz2", 300.0] < 4e-3  # the output's own rounding only
    assert errs["protenix", 300.0] > 5 * errs["boltz2", 300.0], errs
    assert errs["protenix", 1.0] < 2e-2


def test_boltz2_program_layernorm_rounds_normalized_value_before_affine():
    rng = np.random.default_rng(3)
    x = O.bf16(rng.standard_normal((64, 32)) * 3.0 + 1.0)
    w = O.bf16(rng.standard_normal(32))
    b = O.bf16(rng.standard_normal(32))
    with O.bf16_program("boltz2"):
        got = O.layer_norm(x, w, b)
    mean = x.mean(-1, keepdims=True)
    normed = O.bf16((x - mean) / np.sqrt(np.square(x - mean).mean(-1, keepdims=True) + 1e-5))
    assert np.array_equal(got, O.bf16(O.bf16(normed * w) + b))
    with O.bf16_program("protenix"):
        px = O.layer_norm(x, w, b)
    assert not np.array_equal(px, got)  # every op rounded: a different program
    assert np.abs(px - got).max() < 0.1
