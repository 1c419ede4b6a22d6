"""The CPU oracle against the committed golden fixtures (tests/golden/*.npz).

The fixtures come from tests/golden/make_golden.py, an independent element-by-element
brute force (Python floats, arithmetic float32/bf16 rounding) of the reference's
formulas; the reference itself ships no golden vectors for this path.
"""

import os

import numpy as np
import pytest

from oracle import path as P
from oracle import w8a8 as Q
from oracle.numerics import bf16_ulp, from_bf16_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def test_rope_tables_match_bruteforce():
    g = load("rope.npz")
    ids = g["ids"]
    pe = P.embed_nd(ids)[0, 0]
    lanes = P.lane_pair(P.embed_nd(ids))
    assert pe.shape == g["pe"].shape
    # An ulp of omega (numpy's vector powf vs its scalar powf may differ by one) grows with
    # the position into the angle, so the tolerance scales with the largest id of the row.
    for t in range(len(ids)):
        atol = 4e-7 * max(1.0, float(np.abs(ids[t]).max()))
        np.testing.assert_allclose(pe[t], g["pe"][t], rtol=0, atol=atol)
        np.testing.assert_allclose(lanes.cos[t], g["cos"][t], rtol=0, atol=atol)
        np.testing.assert_allclose(lanes.sin[t], g["sin"][t], rtol=0, atol=atol)


@pytest.mark.parametrize("which", ["1", "g"])
def test_qk_prep_matches_bruteforce_bit_exact(which):
    g = load("qk.npz")
    heads = int(g["heads"])
    gain = 1.0 if which == "1" else float(g["gain"])
    qkv = from_bf16_bits(g["qkv"])
    freqs = P.lane_pair(P.embed_nd(g["ids"]), gain)
    q, k, v = P.qk_prep_fused(qkv, from_bf16_bits(g["q_scale"]), from_bf16_bits(g["k_scale"]), freqs, heads)
    np.testing.assert_array_equal(q, from_bf16_bits(g["q" + which]))
    np.testing.assert_array_equal(k, from_bf16_bits(g["k" + which]))
    np.testing.assert_array_equal(v, from_bf16_bits(g["v" + which]))


def test_qk_prep_plain_matches_bruteforce_at_gain_one():
    g = load("qk.npz")
    q, k, v = P.qk_prep_plain(from_bf16_bits(g["qkv"]), from_bf16_bits(g["q_scale"]),
                              from_bf16_bits(g["k_scale"]), P.embed_nd(g["ids"]), int(g["heads"]))
    np.testing.assert_array_equal(q, from_bf16_bits(g["q1"]))
    np.testing.assert_array_equal(k, from_bf16_bits(g["k1"]))


def _within_one_ulp(got, exact):
    bound = bf16_ulp(exact).astype(np.float64) + 1e-6
    return np.all(np.abs(got.astype(np.float64) - exact) <= bound)


def test_sdpa_matches_exact_attention():
    g = load("attn.npz")
    q, k, v = (from_bf16_bits(g[n])[None] for n in ("q_plain", "k", "v"))
    got = P.sdpa(q, k, v)[0]
    assert _within_one_ulp(got, g["sdpa"].astype(np.float64))


def test_bounded_attention_matches_exact():
    g = load("attn.npz")
    q, k, v = (from_bf16_bits(g[n])[None] for n in ("q_pre", "k", "v"))
    got = P.attend_bounded(q, k, v)[0]
    assert _within_one_ulp(got, g["bounded"].astype(np.float64))


def test_w8a8_matches_bruteforce_bit_exact():
    g = load("w8a8.npz")
    x, w = from_bf16_bits(g["x"]), from_bf16_bits(g["w"])
    s = Q.smooth_factors(np.abs(x).max(0), np.abs(w).max(1))
    np.testing.assert_array_equal(s, g["smooth"])
    inv_s = Q.inverse(s)
    np.testing.assert_array_equal(inv_s, g["inv_smooth"])
    wq, w_scale = Q.quantize_weight(w, s)
    np.testing.assert_array_equal(wq, g["wq"])
    np.testing.assert_array_equal(w_scale, g["w_scale"])
    y, acc, xq, a_scale = Q.w8a8_linear(x, inv_s, wq, w_scale)
    np.testing.assert_array_equal(xq, g["xq"])
    np.testing.assert_array_equal(a_scale, g["a_scale"])
    np.testing.assert_array_equal(acc, g["acc"])
    np.testing.assert_array_equal(y, from_bf16_bits(g["y"]))
