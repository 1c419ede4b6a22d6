"""Pins of the CPU oracle by closed forms, invariants and independent formulations.

Each check is chosen so that a plausible mistake in the restatement -- a sign flip in
the rotation, a transposed pair, a wrong axis offset, a dropped epsilon, the gain
applied at the wrong rounding point, a missing max subtraction -- fails it.
"""

import math

import numpy as np
import pytest
import torch

from oracle import path as P
from oracle import w8a8 as Q
from oracle.numerics import bf16_round, bf16_ulp


# ----------------------------------------------------------------------------- bf16 rounding
def test_bf16_round_matches_torch_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-6, 6, 20000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 3.3895314e38, -3.3895314e38,
                                  np.inf, -np.inf], np.float32)]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(bf16_round(x), want)
    assert np.isnan(bf16_round(np.array([np.nan], np.float32)))[0]


def test_bf16_round_ties_to_even():
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties to the even mantissa (1.0)
    assert bf16_round(np.float32(1 + 2 ** -8)) == 1.0
    # 1 + 3*2^-8 is halfway between 1 + 2^-7 and 1 + 2^-6: ties to 1 + 2^-6 (even)
    assert bf16_round(np.float32(1 + 3 * 2 ** -8)) == np.float32(1 + 2 ** -6)


# ----------------------------------------------------------------------------- RoPE tables
def test_rope_freqs_closed_form():
    pos = np.array([0, 1, 5, 300], np.float32)
    pe = P.rope_freqs(pos, 32, 2000.0)
    assert pe.shape == (4, 16, 2, 2)
    for i, x in enumerate(pos):
        for k in range(16):
            ang = float(x) * 2000.0 ** (-2 * k / 32)
            c, s = math.cos(ang), math.sin(ang)
            np.testing.assert_allclose(pe[i, k], [[c, -s], [s, c]], atol=2e-7 * max(1, float(x)))


def test_apply_rope_is_complex_rotation():
    rng = np.random.default_rng(1)
    ids = rng.integers(0, 64, size=(7, 4)).astype(np.float32)
    pe = P.embed_nd(ids)
    x = rng.standard_normal((1, 1, 7, 128)).astype(np.float32)
    got, _ = P.apply_rope(x, x, pe, out_bf16=False)
    z = x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]
    ang = np.angle(pe[..., 0, 0] + 1j * pe[..., 1, 0])            # angle of (cos, sin)
    rot = z * np.exp(1j * ang)
    np.testing.assert_allclose(got[..., 0::2], rot.real, atol=1e-5)
    np.testing.assert_allclose(got[..., 1::2], rot.imag, atol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(got, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


def test_embed_nd_axis_placement():
    # only axis a non-zero -> only pairs 16a..16a+15 rotate; pair 16a itself by angle = id
    for a in range(4):
        ids = np.zeros((1, 4), np.float32)
        ids[0, a] = 3.0
        pe = P.embed_nd(ids)[0, 0, 0]                                # (64, 2, 2)
        identity = np.all(np.isclose(pe, np.eye(2)), axis=(1, 2))
        assert not identity[16 * a:16 * a + 16].any()
        assert identity[:16 * a].all() and identity[16 * a + 16:].all()
        np.testing.assert_allclose(pe[16 * a], [[math.cos(3), -math.sin(3)], [math.sin(3), math.cos(3)]],
                                   atol=1e-6)


def test_ids_known_answers():
    np.testing.assert_array_equal(P.txt_ids(3)[0], [[0, 0, 0, 0], [0, 0, 0, 1], [0, 0, 0, 2]])
    np.testing.assert_array_equal(P.img_ids(2, 3)[0], [[0, 0, 0, 0], [0, 0, 1, 0], [0, 0, 2, 0],
                                                       [0, 1, 0, 0], [0, 1, 1, 0], [0, 1, 2, 0]])
    seq = P.sequence_ids(2, 2, 2)
    np.testing.assert_array_equal(seq[:2], P.txt_ids(2)[0])
    np.testing.assert_array_equal(seq[2:], P.img_ids(2, 2)[0])


def test_lane_pair_rotation_equals_pair_matrices():
    """The fused kernel's lane form (cos2*x + sin2*swap(x)) and rope.apply_rope's 2x2 form are
    two formulations of one rotation."""
    rng = np.random.default_rng(2)
    ids = rng.integers(0, 128, size=(9, 4)).astype(np.float32)
    pe = P.embed_nd(ids)
    lanes = P.lane_pair(pe)
    x = bf16_round(rng.standard_normal((9, 128)).astype(np.float32))
    swap = np.empty_like(x)
    swap[:, 0::2], swap[:, 1::2] = x[:, 1::2], x[:, 0::2]
    lane_form = (lanes.cos * x + lanes.sin * swap).astype(np.float32)
    pair_form, _ = P.apply_rope(x[None, None], x[None, None], pe, out_bf16=False)
    np.testing.assert_array_equal(lane_form, pair_form[0, 0])
    # sign convention: sin lane is -sin on even lanes, +sin on odd lanes
    np.testing.assert_array_equal(lanes.sin[:, 0::2], -pe[0, 0, :, :, 1, 0])
    np.testing.assert_array_equal(lanes.sin[:, 1::2], pe[0, 0, :, :, 1, 0])


# ----------------------------------------------------------------------------- QK norm / heads
def test_rms_norm_constant_row():
    for c in (0.5, -3.0, 1e-4):
        x = np.full((1, 128), c, np.float32)
        got = P.rms_norm(x, np.ones(128, np.float32))
        want = bf16_round(np.float32(math.copysign(1.0, c) / math.sqrt(1.0 + 1e-6 / c ** 2)))
        np.testing.assert_array_equal(got, np.full((1, 128), want, np.float32))


def test_rms_norm_bruteforce():
    rng = np.random.default_rng(3)
    x = bf16_round(rng.standard_normal((4, 128)).astype(np.float32) * 3)
    s = bf16_round((1 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    got = P.rms_norm(x, s)
    for r in range(4):
        ms = math.fsum(float(v) ** 2 for v in x[r]) / 128
        inv = 1.0 / math.sqrt(ms + 1e-6)
        for d in range(128):
            normed = bf16_round(np.float32(float(x[r, d]) * inv))
            want = bf16_round(np.float32(float(normed) * float(s[d])))
            assert abs(float(got[r, d]) - float(want)) <= float(bf16_ulp(want))


def test_heads_index_map_and_merge_inverse():
    b, length, h, d = 2, 3, 4, 5
    qkv = np.arange(b * length * 3 * h * d, dtype=np.float32).reshape(b, length, 3 * h * d)
    q, k, v = P.heads(qkv, h)
    for sec, t_ in enumerate((q, k, v)):
        assert t_.shape == (b, h, length, d)
        for bb, hh, tt, dd in [(0, 0, 0, 0), (1, 3, 2, 4), (1, 2, 1, 3)]:
            assert t_[bb, hh, tt, dd] == qkv[bb, tt, (sec * h + hh) * d + dd]
    np.testing.assert_array_equal(P.merge_heads(q), qkv[..., : h * d])


def _case(seed, heads=3, length=11):
    rng = np.random.default_rng(seed)
    qkv = bf16_round(rng.standard_normal((1, length, 3 * heads * 128)).astype(np.float32))
    qs = bf16_round((1 + 0.05 * rng.standard_normal(128)).astype(np.float32))
    ks = bf16_round((1 + 0.05 * rng.standard_normal(128)).astype(np.float32))
    ids = rng.integers(0, 200, size=(length, 4)).astype(np.float32)
    return qkv, qs, ks, ids


def test_fused_at_gain_one_equals_plain_branch():
    qkv, qs, ks, ids = _case(4)
    pe = P.embed_nd(ids)
    plain = P.qk_prep_plain(qkv, qs, ks, pe, 3)
    fused = P.qk_prep_fused(qkv, qs, ks, P.lane_pair(pe, 1.0), 3)
    for a, b in zip(plain, fused):
        np.testing.assert_array_equal(a, b)


def test_gain_is_applied_after_rotation_before_rounding():
    qkv, qs, ks, ids = _case(5)
    pe = P.embed_nd(ids)
    gain = 1 / math.sqrt(128)
    q_g, k_g, v_g = P.qk_prep_fused(qkv, qs, ks, P.lane_pair(pe, gain), 3)
    _, _, _, yq, _ = P.qk_prep_fused(qkv, qs, ks, P.lane_pair(pe, 1.0), 3, return_normed=True)
    q1, k1, v1 = P.qk_prep_fused(qkv, qs, ks, P.lane_pair(pe, 1.0), 3)
    np.testing.assert_array_equal(k_g, k1)                  # gain touches q only
    np.testing.assert_array_equal(v_g, v1)
    lanes = P.lane_pair(pe)
    swap = np.empty_like(yq)
    swap[..., 0::2], swap[..., 1::2] = yq[..., 1::2], yq[..., 0::2]
    rot = (lanes.cos * yq + lanes.sin * swap).astype(np.float32)
    np.testing.assert_array_equal(q_g, bf16_round((np.float32(gain) * rot).astype(np.float32)))
    # rounding the unscaled rotation first and scaling after would differ somewhere
    assert not np.array_equal(q_g, bf16_round((np.float32(gain) * q1).astype(np.float32)))


def test_qkv_prep_gate_follows_row_tile():
    """modules.py:76-80: the fused form (lanes and q_gain) iff freqs is given and a row tile
    divides L, else the plain branch from pe with no gain.  Pinned by the rows' RMS: RoPE is
    orthogonal, so with unit norm scales a prepared row has RMS 1 on the plain branch and RMS
    q_gain on the fused one; k is never scaled."""
    gain = 1 / math.sqrt(128)
    ones = np.ones(128, np.float32)
    for length, fused in ((11, False), (100, False), (257, False), (64, True), (128, True)):
        qkv, _, _, ids = _case(7 + length, heads=2, length=length)
        pe = P.embed_nd(ids)
        for freqs in (P.lane_pair(pe, gain), None):
            q, k, v = P.qkv_prep(qkv, ones, ones, pe, freqs, 2)
            rms_q = np.sqrt((q.astype(np.float64) ** 2).mean(-1))
            rms_k = np.sqrt((k.astype(np.float64) ** 2).mean(-1))
            np.testing.assert_allclose(rms_k, 1.0, atol=1e-2)
            want = gain if (fused and freqs is not None) else 1.0
            np.testing.assert_allclose(rms_q, want, rtol=1e-2)
            np.testing.assert_array_equal(v, P.heads(qkv, 2)[2])


def test_qk_prep_invariants():
    qkv, qs, ks, ids = _case(6, heads=2, length=64)
    q, k, v = P.qk_prep_fused(qkv, np.ones(128, np.float32), np.ones(128, np.float32),
                              P.lane_pair(P.embed_nd(ids)), 2)
    _, _, vv = P.heads(qkv, 2)
    np.testing.assert_array_equal(v, vv)                    # v is a copy
    rms = np.sqrt((k.astype(np.float64) ** 2).mean(-1))    # unit scale: RMS 1 up to bf16
    np.testing.assert_allclose(rms, 1.0, atol=1e-2)


# ----------------------------------------------------------------------------- attention
def _attn_case(seed, length=9, dim=16, heads=2, scale=1.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((3, 1, heads, length, dim))
    x[:2] /= np.sqrt((x[:2] ** 2).mean(-1, keepdims=True))
    q, k, v = (bf16_round((x[i] * (scale if i < 2 else 1)).astype(np.float32)) for i in range(3))
    return q, k, v


def _softmax_attention_bruteforce(q, k, v, scale):
    out = np.zeros(q.shape)
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            for i in range(q.shape[2]):
                logits = [scale * math.fsum(float(q[b, h, i, d]) * float(k[b, h, j, d]) for d in range(q.shape[3]))
                          for j in range(q.shape[2])]
                w = [math.exp(s) for s in logits]                 # no max: independent of sdpa's
                z = math.fsum(w)
                for d in range(q.shape[3]):
                    out[b, h, i, d] = math.fsum(w[j] * float(v[b, h, j, d]) for j in range(q.shape[2])) / z
    return out


def test_sdpa_bruteforce():
    q, k, v = _attn_case(7, scale=2.0)
    want = _softmax_attention_bruteforce(q, k, v, 1 / math.sqrt(q.shape[-1]))
    got = P.sdpa(q, k, v)
    assert np.all(np.abs(got - want) <= bf16_ulp(want) + 1e-7)


def test_attend_bounded_bruteforce_with_rounded_p():
    q, k, v = _attn_case(8)
    q = bf16_round((q / np.float32(4.0)).astype(np.float32))
    got = P.attend_bounded(q, k, v)
    want = np.zeros(q.shape)
    for h in range(q.shape[1]):
        for i in range(q.shape[2]):
            s = [np.float32(math.fsum(float(q[0, h, i, d]) * float(k[0, h, j, d]) for d in range(16)))
                 for j in range(q.shape[2])]
            p = [float(bf16_round(np.float32(math.exp(float(x))))) for x in s]
            for d in range(16):
                want[0, h, i, d] = math.fsum(p[j] * float(v[0, h, j, d]) for j in range(len(p))) / math.fsum(p)
    assert np.all(np.abs(got - want) <= bf16_ulp(want) + 1e-7)


def test_attention_special_cases():
    q, k, v = _attn_case(9, length=16)
    k_same = np.broadcast_to(k[:, :, :1], k.shape).copy()
    o = P.attend_bounded(q, k_same, v)
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(axis=2, keepdims=True), o.shape), atol=2e-2)
    # one dominant key: logit 60 against 0 for the rest
    qd = np.zeros((1, 1, 8, 16), np.float32)
    qd[..., 0] = 15.0
    kd = np.zeros((1, 1, 8, 16), np.float32)
    kd[0, 0, 5, 0] = 4.0
    vd = _attn_case(10, length=8, heads=1)[2]
    np.testing.assert_allclose(P.attend_bounded(qd, kd, vd), np.broadcast_to(vd[:, :, 5:6], (1, 1, 8, 16)),
                               atol=1e-6)


def test_bounded_equals_plain_path_within_tolerance():
    """The bounded path (bf16 pre-scaled q, bf16 P, no max) against plain sdpa (f32 scale, max
    subtraction) on the same prepped rows: the path's stated 2e-2 / 2e-3 gate."""
    q, k, v = _attn_case(11, length=256, dim=128, heads=2, scale=1.1)
    o_plain = P.sdpa(q, k, v)
    o_bound = P.attend_bounded(bf16_round((q / np.float32(math.sqrt(128))).astype(np.float32)), k, v)
    diff = np.abs(o_plain - o_bound)
    assert diff.max() <= 2e-2 and diff.mean() <= 2e-3


def test_logit_bound_holds_and_threshold():
    rng = np.random.default_rng(12)
    for scale in (1.0, 2.0):
        qs = (scale * (1 + 0.05 * rng.standard_normal(128))).astype(np.float32)
        ks = (scale * (1 + 0.05 * rng.standard_normal(128))).astype(np.float32)
        qkv = bf16_round(rng.standard_normal((1, 64, 3 * 128)).astype(np.float32) * 5)
        q, k, _ = P.qk_prep_fused(qkv, qs, ks, P.lane_pair(P.embed_nd(rng.integers(0, 50, (64, 4))),
                                                         1 / math.sqrt(128)), 1, scale_is_bf16=False)
        s = q[0, 0].astype(np.float64) @ k[0, 0].astype(np.float64).T
        assert np.abs(s).max() <= float(P.logit_bound(qs, ks)) * (1 + 2e-2)  # bf16 slack
    assert math.isclose(float(P.logit_bound(np.full(128, 3.0), np.full(128, 3.0))), math.sqrt(128) * 9,
                        rel_tol=1e-6)

    def blocks(v):
        d = {f"{s}_attn.norm.{n}.scale": np.full((5, 128), v, np.float32) for s in ("img", "txt")
             for n in ("query_norm", "key_norm")}
        sg = {f"norm.{n}.scale": np.ones((20, 128), np.float32) for n in ("query_norm", "key_norm")}
        return {"double_blocks": d, "single_blocks": sg}

    P.check_logit_bound(blocks(1.0))
    with pytest.raises(ValueError, match="needs logits under 80"):
        P.check_logit_bound(blocks(3.0))                     # 101.8 >= 80


# ----------------------------------------------------------------------------- W8A8
def test_int_gemm_bruteforce_and_range():
    rng = np.random.default_rng(13)
    xq = rng.integers(-127, 128, (5, 40)).astype(np.int8)
    wq = rng.integers(-127, 128, (40, 7)).astype(np.int8)
    np.testing.assert_array_equal(Q.int_gemm(xq, wq), Q.int_gemm_bruteforce(xq, wq))
    full = np.full((2, 3072), 127, np.int8)
    assert Q.int_gemm(full, full.T.copy())[0, 0] == 3072 * 127 * 127   # 49.5 M < 2^31


def test_quantize_ties_clamp_and_zero_rows():
    x = np.array([[0.5, 1.5, 2.5, -0.5, 127.0], [0, 0, 0, 0, 0]], np.float32)
    xq, a = Q.quantize_act(x, np.ones(5, np.float32))
    assert a[0] == np.float32(127.0) / np.float32(127) and a[1] == 1.0
    np.testing.assert_array_equal(xq[1], 0)
    np.testing.assert_array_equal(xq[0], np.rint(x[0] / a[0]).astype(np.int8))
    assert np.abs(xq).max() <= 127
    assert Q._quantize(np.array([0.5, 1.5, 2.5, 400.0, -400.0], np.float32), np.float32(1)).tolist() == \
        [0, 2, 2, 127, -127]


def test_w8a8_error_is_small_against_bf16_linear():
    rng = np.random.default_rng(14)
    x = bf16_round(rng.standard_normal((64, 256)).astype(np.float32))
    x[:, :3] *= 20
    w = bf16_round((0.02 * rng.standard_normal((256, 96))).astype(np.float32))
    s = Q.smooth_factors(np.abs(x).max(0), np.abs(w).max(1))
    wq, ws = Q.quantize_weight(w, s)
    y, _, _, _ = Q.w8a8_linear(x, Q.inverse(s), wq, ws)
    ref = x.astype(np.float64) @ w.astype(np.float64)
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 0.03, rel


def _layer_norm_loop(row):
    """Element loop in exact rationals where possible: f64 mean/variance of the f32 values,
    each rounded to f32, then per element f32 subtract, square, product and bf16 rounding."""
    vals = [float(np.float32(v)) for v in row]
    mean = np.float32(sum(vals) / len(vals))
    d = [np.float32(np.float32(v) - mean) for v in vals]
    var = np.float32(sum(float(np.float32(e * e)) for e in d) / len(d))
    inv = np.float32(1.0) / np.float32(math.sqrt(np.float32(var + np.float32(1e-6))))
    return np.array([bf16_round(np.float32(e * inv)) for e in d], dtype=np.float32)


def test_layer_norm_bruteforce_and_invariants():
    rng = np.random.default_rng(11)
    x = bf16_round((3.0 * rng.standard_normal((4, 2, 96)) + 0.7).astype(np.float32))
    got = Q.layer_norm(x)
    for idx in np.ndindex(x.shape[:-1]):
        np.testing.assert_array_equal(got[idx], _layer_norm_loop(x[idx]))
    # unit statistics before rounding, a constant row normalises to zero
    assert np.abs(got.mean(-1)).max() < 0.02 and np.abs(got.var(-1) - 1).max() < 0.02
    np.testing.assert_array_equal(Q.layer_norm(np.full((1, 1, 64), 2.5, np.float32)), 0.0)


def test_modulate_known_answers():
    rng = np.random.default_rng(12)
    x = bf16_round(rng.standard_normal((2, 5, 64)).astype(np.float32))
    zero = np.zeros((2, 64), np.float32)
    np.testing.assert_array_equal(Q.modulate(x, zero, zero), Q.layer_norm(x))            # identity modulation
    shift = bf16_round(rng.standard_normal((2, 64)).astype(np.float32))
    np.testing.assert_array_equal(Q.modulate(x, shift, np.full((2, 64), -1.0, np.float32)),
                                  np.broadcast_to(shift[:, None, :], x.shape))            # scale -1 keeps the shift
    scale = bf16_round(0.1 * rng.standard_normal((2, 64)).astype(np.float32))
    got = Q.modulate(x, shift, scale)
    base = Q.layer_norm(x)
    for b, t, j in np.ndindex(x.shape):      # per-element loop of the three bf16 roundings
        one = bf16_round(np.float32(1.0) + np.float32(scale[b, j]))
        want = bf16_round(np.float32(bf16_round(np.float32(one * base[b, t, j])) + np.float32(shift[b, j])))
        assert got[b, t, j] == want


# Rows whose quotient v / a lands next to a half-integer: a = fl(amax / 127), v = amax / 2, so
# v / a is within an ulp of 63.5.  Found by exhaustive search over bf16 v for these amax.
NEAR_TIE_ROWS = (2.359375, 108.0, 144.0, 53.25, 422.0)


def _exact_f32_quotient_rint(v: float, a: float) -> int:
    """rint of the correctly rounded f32 quotient, from exact rationals (no float division)."""
    from fractions import Fraction
    z = Fraction(v) / Fraction(a)
    lo = np.float32(float(z))                      # nearest double, then nearest f32 ...
    cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
    q = min(cands, key=lambda c: (abs(Fraction(float(c)) - z), int(np.float32(c).view(np.int32)) & 1))
    return int(np.rint(q))


def test_quantize_near_ties_known_answers():
    """The oracle quantises with the correctly rounded division: its codes equal the ones
    derived from exact rationals, and a reciprocal multiply would give other codes."""
    for amax in NEAR_TIE_ROWS:
        v = np.float32(amax / 2)
        x = np.zeros((1, 8), np.float32)
        x[0, 0], x[0, 1] = amax, v
        xq, a = Q.quantize_act(x, np.ones(8, np.float32))
        assert a[0] == np.float32(np.float32(amax) / np.float32(127))
        assert xq[0, 0] == 127
        assert xq[0, 1] == _exact_f32_quotient_rint(float(v), float(a[0])), amax
        recip = int(np.rint(np.float32(v * np.float32(np.float32(1) / a[0]))))
        assert recip != xq[0, 1], f"amax {amax}: the vector does not separate division from reciprocal"
