"""Randomized properties of the oracle that the mathematics fixes (hypothesis, CPU only).

Each property is chosen so that a plausible slip in the restatement fails it:
* attention is invariant to the order of the keys when K and V rows move together (a K/V
  index mismatch or a per-position term breaks it);
* the int8 GEMM is exactly linear in its activation operand and agrees with the
  transposed product (a transposed operand or a dropped term breaks it);
* activation quantisation codes lie in [-127, 127], the row maximum maps to +-127, and
  every code is within half a step of the scaled value (floor instead of rint, or the wrong
  reduction axis, breaks it);
* the lane form of RoPE is a rotation: each (2j, 2j+1) pair keeps its length.
"""

import numpy as np
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import path as P
from oracle import w8a8 as Q
from oracle.numerics import bf16_round, bf16_ulp

SETTINGS = settings(max_examples=25, deadline=None, suppress_health_check=[HealthCheck.too_slow])


@SETTINGS
@given(seed=st.integers(0, 2 ** 31 - 1), length=st.integers(2, 40), dim=st.sampled_from([8, 16, 32]))
def test_attention_invariant_to_key_order(seed, length, dim):
    rng = np.random.default_rng(seed)
    q = bf16_round((0.3 * rng.standard_normal((1, 2, length, dim))).astype(np.float32))
    k = bf16_round(rng.standard_normal((1, 2, length, dim)).astype(np.float32))
    v = bf16_round(rng.standard_normal((1, 2, length, dim)).astype(np.float32))
    perm = rng.permutation(length)
    base = P.attend_bounded(q, k, v)
    moved = P.attend_bounded(q, k[:, :, perm], v[:, :, perm])
    # only the summation order differs: within an ulp of the f32 result, one bf16 ulp after rounding
    assert np.all(np.abs(moved - base) <= bf16_ulp(base) + 1e-7)
    # and so does the plain softmax path
    np.testing.assert_allclose(P.sdpa(q, k[:, :, perm], v[:, :, perm]), P.sdpa(q, k, v), atol=1e-2)


@SETTINGS
@given(seed=st.integers(0, 2 ** 31 - 1), m=st.integers(1, 12), k=st.integers(1, 40), n=st.integers(1, 12))
def test_int_gemm_linear_and_transposes(seed, m, k, n):
    rng = np.random.default_rng(seed)
    x1 = rng.integers(-63, 64, (m, k), dtype=np.int8)
    x2 = rng.integers(-63, 64, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (k, n), dtype=np.int8)
    total = (x1.astype(np.int16) + x2.astype(np.int16)).astype(np.int8)   # |x1 + x2| <= 126
    np.testing.assert_array_equal(Q.int_gemm(total, w), Q.int_gemm(x1, w) + Q.int_gemm(x2, w))
    np.testing.assert_array_equal(Q.int_gemm(x1, w).T, Q.int_gemm(w.T, x1.T))


@SETTINGS
@given(seed=st.integers(0, 2 ** 31 - 1), rows=st.integers(1, 6), cols=st.sampled_from([8, 64, 200]),
       spread=st.floats(1e-3, 1e3))
def test_quantize_act_codes_and_error(seed, rows, cols, spread):
    rng = np.random.default_rng(seed)
    x = bf16_round((spread * rng.standard_normal((rows, cols))).astype(np.float32))
    inv = bf16_round((0.5 + rng.random(cols)).astype(np.float32))
    xq, a = Q.quantize_act(x, inv)
    xh = (x * inv[None, :]).astype(np.float32)
    assert xq.dtype == np.int8 and np.all(np.abs(xq.astype(np.int32)) <= 127)
    np.testing.assert_array_equal(a, (np.abs(xh).max(1) / np.float32(127)).astype(np.float32))
    top = np.abs(xh).argmax(1)
    assert np.all(np.abs(xq[np.arange(rows), top].astype(np.int32)) == 127)
    err = np.abs(xq.astype(np.float64) * a[:, None].astype(np.float64) - xh.astype(np.float64))
    assert np.all(err <= a[:, None].astype(np.float64) * (0.5 + 1e-5))


@SETTINGS
@given(seed=st.integers(0, 2 ** 31 - 1), length=st.integers(1, 30))
def test_lane_rope_is_a_rotation(seed, length):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, 512, (length, 4)).astype(np.float32)
    lanes = P.lane_pair(P.embed_nd(ids))
    y = rng.standard_normal((length, 128)).astype(np.float32)
    r = (lanes.cos * y + lanes.sin * y.reshape(length, 64, 2)[..., ::-1].reshape(length, 128)).astype(np.float64)
    pair_in = (y.astype(np.float64).reshape(length, 64, 2) ** 2).sum(-1)
    pair_out = (r.reshape(length, 64, 2) ** 2).sum(-1)
    np.testing.assert_allclose(pair_out, pair_in, rtol=1e-5, atol=1e-6)
