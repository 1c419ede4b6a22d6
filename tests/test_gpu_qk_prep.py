"""qk_prep on the GPU (flk_qk_prep) against the CPU restatement of kernels.py:35-91.

Gate: v is a bit-exact copy.  For q and k at most 0.01% of elements may differ from the
oracle, and each difference must be explainable by one intermediate bf16 rounding
landing one ulp apart: the oracle's mean of squares is exact while the kernel's is a
float32 tree sum, so bf16(x * rsqrt(ms + eps)) can flip by an ulp on a rounding tie;
the rotation then carries that flip into both outputs of the pair.  Bound per element:
gain * 2 * (ulp(y_i) + ulp(y_pair)) + ulp(out_i), y = the normed-and-scaled input.
"""

import math

import numpy as np
import pytest
import torch

from flicker_amd import kernels, modules
from oracle import path as P
from oracle.numerics import bf16_ulp
from tests._util import describe, to_np, ulp_stats

pytestmark = pytest.mark.gpu
D = 128


def make_case(batch, length, heads, seed, scale_dtype=torch.bfloat16, scale_sd=0.05):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(batch, length, 3 * heads * D, generator=g).to(torch.bfloat16)
    qs = (1 + scale_sd * torch.randn(D, generator=g)).to(scale_dtype)
    ks = (1 + scale_sd * torch.randn(D, generator=g)).to(scale_dtype)
    ids = torch.randint(0, 128, (length, 4), generator=g).float().numpy()
    return qkv, qs, ks, ids


def oracle_tables(ids, gain):
    return P.lane_pair(P.embed_nd(ids), gain)


def gpu_freqs(tables, device):
    return kernels.Freqs(torch.from_numpy(tables.cos).to(device), torch.from_numpy(tables.sin).to(device),
                         tables.q_gain)


def check_qkv(label, got, want, gain):
    """want = qk_prep_fused(..., return_normed=True) output: (q, k, v, yq, yk)."""
    gq, gk, gv = (to_np(t) for t in got)
    wq, wk, wv, yq, yk = want
    assert np.array_equal(gv, wv), f"{label}: v is not a bit-exact copy"
    for name, g, w, y, gn in (("q", gq, wq, yq, gain), ("k", gk, wk, yk, 1.0)):
        st = ulp_stats(g, w)
        ulp_y = bf16_ulp(y)
        ulp_pair = np.empty_like(ulp_y)
        ulp_pair[..., 0::2], ulp_pair[..., 1::2] = ulp_y[..., 1::2], ulp_y[..., 0::2]
        bound = np.float32(gn) * 2 * (ulp_y + ulp_pair) + bf16_ulp(w)
        excess = float((np.abs(g.astype(np.float64) - w) / bound).max())
        print(describe(f"{label} {name}", st), f"diff/bound={excess:.3g}")
        assert st["mismatch"] <= 1e-4, f"{label} {name}: {st}"
        assert excess <= 1.0, f"{label} {name}: a difference exceeds one intermediate ulp flip ({excess})"


@pytest.mark.parametrize("batch,length,heads,gain", [
    (1, 64, 24, 1 / math.sqrt(128)),
    (2, 128, 24, 1.0),
    (1, 1536, 24, 1 / math.sqrt(128)),
    (3, 256, 6, 0.5),
    (1, 512, 5, 1 / math.sqrt(128)),
])
def test_qk_prep_matches_oracle(device, batch, length, heads, gain):
    qkv, qs, ks, ids = make_case(batch, length, heads, seed=length + heads)
    tables = oracle_tables(ids, gain)
    got = kernels.qk_prep(qkv.to(device), qs.to(device), ks.to(device), gpu_freqs(tables, device), heads)
    torch.cuda.synchronize()
    want = P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), tables, heads, return_normed=True)
    check_qkv(f"B{batch} L{length} H{heads} gain{gain:.4f}", got, want, gain)


@pytest.mark.parametrize("length", [1, 17, 100, 4352])
def test_qk_prep_ragged_length(device, length):
    """Lengths that are not multiples of the 16-token block, through qkv_prep: L = 1, 17 and
    100 have no row tile and take the plain branch (lanes from pe), 4352 = 17 * 256 the fused
    one; at gain 1 both compute the same values."""
    qkv, qs, ks, ids = make_case(1, length, 24, seed=length)
    pe = P.embed_nd(ids)
    tables = P.lane_pair(pe, 1.0)
    got = modules.qkv_prep(qkv.to(device), qs.to(device), ks.to(device), torch.from_numpy(pe).to(device),
                           gpu_freqs(tables, device), 24)
    torch.cuda.synchronize()
    check_qkv(f"L{length}", got, P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), tables, 24,
                                                return_normed=True), 1.0)


@pytest.mark.parametrize("batch,length,pe_batch", [(1, 100, 1), (1, 257, 1), (2, 100, 2), (1, 256, 1)])
def test_qkv_prep_gate(device, batch, length, pe_batch):
    """modules.py:76-80 with the bounded path's q_gain = 1/sqrt(128): a length with no row tile
    (100, 257) takes the plain branch -- rotation by pe, no gain -- and 256 the fused kernel
    with the gain; each against the oracle's gate (oracle.path.qkv_prep).  pe with a batch
    axis rotates each batch element by its own table (apply_rope broadcasts pe)."""
    gain = 1 / math.sqrt(128)
    qkv, qs, ks, ids = make_case(batch, length, 24, seed=900 + length + batch)
    if pe_batch > 1:
        g = np.random.default_rng(length)
        ids = np.stack([ids] + [g.integers(0, 128, ids.shape).astype(np.float32) for _ in range(pe_batch - 1)])
    pe = P.embed_nd(ids)
    freqs = P.lane_pair(pe, gain)
    got = modules.qkv_prep(qkv.to(device), qs.to(device), ks.to(device), torch.from_numpy(pe).to(device),
                           gpu_freqs(freqs, device), 24)
    torch.cuda.synchronize()
    want = P.qkv_prep(to_np(qkv), to_np(qs), to_np(ks), pe, freqs, 24)
    fused = P.row_tile(length) is not None
    normed = P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), P.lane_pair(pe[:1], 1.0), 24,
                             return_normed=True)[3:]
    if pe_batch > 1:   # the normed rows do not depend on the table; q, k of batch b on pe[b]
        for b in range(batch):
            rows = P.qk_prep_fused(to_np(qkv)[b:b + 1], to_np(qs), to_np(ks), P.lane_pair(pe[b:b + 1], 1.0), 24)
            assert all(np.array_equal(w[b:b + 1], r) for w, r in zip(want, rows))
    check_qkv(f"gate B{batch} L{length} {'fused' if fused else 'plain'}", got, tuple(want) + tuple(normed),
              gain if fused else 1.0)
    rms = np.sqrt((to_np(got[0]).astype(np.float64) ** 2).mean(-1)).mean()
    assert abs(rms - (gain if fused else 1.0)) < 0.05 * (gain if fused else 1.0), rms


def test_qk_prep_f32_scales(device):
    qkv, qs, ks, ids = make_case(1, 128, 24, seed=7, scale_dtype=torch.float32)
    tables = oracle_tables(ids, 1 / math.sqrt(128))
    got = kernels.qk_prep(qkv.to(device), qs.to(device), ks.to(device), gpu_freqs(tables, device), 24)
    torch.cuda.synchronize()
    want = P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), tables, 24, scale_is_bf16=False,
                           return_normed=True)
    check_qkv("f32 scales", got, want, tables.q_gain)


@pytest.mark.parametrize("batch,length,pe_batch", [(1, 100, 1), (2, 257, 2)])
def test_qkv_prep_plain_branch_f32_scales(device, batch, length, pe_batch):
    """The plain branch (modules.py:78-80) with float32 norm scales returns float32 q and k:
    rms_norm's bf16(normed) * scale promotes to float32 (nn.py:27) and apply_rope casts the
    float32 rotation back to that dtype (rope.py:28), so nothing is rounded after the normed
    value; v stays the bf16 split.  Against oracle.path.qk_prep_plain(..., scale_is_bf16=False):
    v bit-exact; q and k equal except where the kernel's float32 mean of squares flips the
    intermediate bf16(x * rsqrt) by one ulp, each such difference within that flip carried
    through the rotation."""
    qkv, qs, ks, ids = make_case(batch, length, 24, seed=1300 + length, scale_dtype=torch.float32)
    if pe_batch > 1:
        g = np.random.default_rng(length)
        ids = np.stack([ids] + [g.integers(0, 128, ids.shape).astype(np.float32) for _ in range(pe_batch - 1)])
    pe = P.embed_nd(ids)
    assert P.row_tile(length) is None, "the case must take the plain branch"
    got = modules.qkv_prep(qkv.to(device), qs.to(device), ks.to(device), torch.from_numpy(pe).to(device),
                           gpu_freqs(P.lane_pair(pe[:1], 1 / math.sqrt(D)), device), 24)
    torch.cuda.synchronize()
    assert got[0].dtype == got[1].dtype == torch.float32 and got[2].dtype == torch.bfloat16
    wq, wk, wv = P.qk_prep_plain(to_np(qkv), to_np(qs), to_np(ks), pe, 24, scale_is_bf16=False)
    assert wq.dtype == np.float32
    assert np.array_equal(to_np(got[2]), wv), "v is not a bit-exact copy"
    for name, g, w, sc in (("q", got[0], wq, to_np(qs)), ("k", got[1], wk, to_np(ks))):
        g = g.cpu().numpy()
        diff = np.abs(g.astype(np.float64) - w.astype(np.float64))
        # one flip of the normed bf16 value n in element i or its pair partner moves the output by at
        # most ulp(n_i) |sc_i| + ulp(n_pair) |sc_pair| (|cos|, |sin| <= 1); |n| < 16 for unit-RMS rows
        flip = np.float64(2.0 ** -8 * 16) * np.abs(sc).max() * 2
        mismatch = float((diff > 0).mean())
        print(f"plain f32 B{batch} L{length} {name}: mismatch {mismatch:.3g} max diff {diff.max():.3g}")
        assert mismatch <= 1e-4, (name, mismatch)
        assert diff.max() <= flip, (name, diff.max())
    rms = np.sqrt((got[0].cpu().numpy().astype(np.float64) ** 2).mean(-1)).mean()
    assert abs(rms - 1.0) < 0.05, rms   # no query gain on the plain branch


def test_qk_prep_gain_one_equals_plain_path(device):
    """At q_gain = 1 the fused kernel computes the plain-XLA branch (modules.py:78-80)."""
    qkv, qs, ks, ids = make_case(2, 256, 24, seed=11)
    pe = P.embed_nd(ids)
    got = modules.qkv_prep(qkv.to(device), qs.to(device), ks.to(device), torch.from_numpy(pe).to(device),
                           None, 24)
    torch.cuda.synchronize()
    plain = P.qk_prep_plain(to_np(qkv), to_np(qs), to_np(ks), pe, 24)
    fused = P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), P.lane_pair(pe, 1.0), 24, return_normed=True)
    assert all(np.array_equal(a, b) for a, b in zip(plain, fused[:3]))
    check_qkv("plain", got, plain + fused[3:], 1.0)


def test_qk_prep_strided_single_block_view(device):
    """The qkv part of a single block's fused linear1 output (modules.py:185-189), as a view."""
    length, heads = 256, 24
    g = torch.Generator().manual_seed(3)
    lin1 = torch.randn(1, length, 3 * heads * D + 2 * 9216, generator=g).to(torch.bfloat16)
    _, qs, ks, ids = make_case(1, length, heads, seed=4)
    tables = oracle_tables(ids, 1 / math.sqrt(128))
    dev = lin1.to(device)
    view = dev[..., : 3 * heads * D]
    assert not view.is_contiguous()
    got = kernels.qk_prep(view, qs.to(device), ks.to(device), gpu_freqs(tables, device), heads)
    torch.cuda.synchronize()
    want = P.qk_prep_fused(to_np(lin1)[..., : 3 * heads * D], to_np(qs), to_np(ks), tables, heads,
                           return_normed=True)
    check_qkv("strided", got, want, tables.q_gain)


def test_qk_prep_out_offset_fills_joint_buffer(device):
    """Text and image streams written at their offsets equal separate calls concatenated."""
    heads, n_txt, n_img = 24, 512, 256
    txt, qs_t, ks_t, ids_t = make_case(1, n_txt, heads, seed=21)
    img, qs_i, ks_i, ids_i = make_case(1, n_img, heads, seed=22)
    ft = gpu_freqs(oracle_tables(ids_t, 0.125), device)
    fi = gpu_freqs(oracle_tables(ids_i, 0.125), device)
    joint = tuple(torch.full((1, heads, n_txt + n_img, D), float("nan"), dtype=torch.bfloat16, device=device)
                  for _ in range(3))
    kernels.qk_prep(txt.to(device), qs_t.to(device), ks_t.to(device), ft, heads, out=joint, out_offset=0)
    kernels.qk_prep(img.to(device), qs_i.to(device), ks_i.to(device), fi, heads, out=joint, out_offset=n_txt)
    sep_t = kernels.qk_prep(txt.to(device), qs_t.to(device), ks_t.to(device), ft, heads)
    sep_i = kernels.qk_prep(img.to(device), qs_i.to(device), ks_i.to(device), fi, heads)
    torch.cuda.synchronize()
    for j, a, b in zip(joint, sep_t, sep_i):
        assert torch.equal(j, torch.cat([a, b], dim=2))


def test_qk_prep_klein_1024_full(device):
    """The headline shape: (1, 4608, 9216) with the workload's own tables and scales."""
    from flicker_amd import workloads
    w = workloads.WORKLOADS["klein_1024"]
    qkv, (qs, ks), ids = workloads.make_qkv(w), workloads.make_scales(w), workloads.make_ids(w)
    tables = oracle_tables(ids, workloads.q_gain(w))
    got = kernels.qk_prep(qkv.to(device), qs.to(device), ks.to(device), gpu_freqs(tables, device), 24)
    torch.cuda.synchronize()
    check_qkv("klein_1024", got, P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), tables, 24,
                                                  return_normed=True), tables.q_gain)


def _ids_and_tables_paths(device, qkv, qs, ks, ids, heads, gain):
    """qk_prep through position ids (cos/sin in-kernel) and through rope_lanes tables; also
    returns those tables (whose agreement with the oracle's is test_gpu_rope's)."""
    from flicker_amd import rope
    ids_dev = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.float32)).to(device)
    args = (qkv.to(device), qs.to(device), ks.to(device))
    freqs = rope.rope_lanes(ids_dev, gain)
    # the launch below kernels.qk_prep's row-tile check, so that any L reaches the kernel
    via_ids = kernels._launch_qk_prep(*args, rope.position_ids(ids_dev, gain), heads, None, 0)
    via_tables = kernels._launch_qk_prep(*args, freqs, heads, None, 0)
    torch.cuda.synchronize()
    return via_ids, via_tables, P.Freqs(to_np(freqs.cos), to_np(freqs.sin), gain)


@pytest.mark.parametrize("batch,length,heads,gain", [
    (1, 64, 24, 1 / math.sqrt(128)),
    (2, 100, 24, 1.0),
    (1, 1536, 6, 0.5),
    (1, 17, 5, 1 / math.sqrt(128)),
    (3, 256, 3, 1 / math.sqrt(128)),
])
def test_qk_prep_ids_equals_table_path(device, batch, length, heads, gain):
    """flk_qk_prep_ids computes the same cos/sin bits as flk_rope_lanes, so the outputs are
    identical to the table path's; against the oracle fed those same lane values, the usual
    qk_prep gate.  (With the oracle's own numpy tables, f32 cos/sin one ulp apart flip a few
    bf16 output roundings -- within the per-element bound, but not an exact-table count.)"""
    qkv, qs, ks, ids = make_case(batch, length, heads, seed=100 + length + heads)
    via_ids, via_tables, lanes = _ids_and_tables_paths(device, qkv, qs, ks, ids, heads, gain)
    for name, a, b in zip("qkv", via_ids, via_tables):
        assert torch.equal(a, b), f"{name}: ids path differs from the table path"
    want = P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), lanes, heads, return_normed=True)
    check_qkv(f"ids B{batch} L{length} H{heads}", via_ids, want, gain)


@pytest.mark.parametrize("name", ["klein_1024", "klein_2048"])
def test_qk_prep_ids_klein_positions(device, name):
    """The workloads' real text|image ids (text positions up to 511, image rows/cols up to 127
    at 2048^2) through both RoPE sources; two heads keep the 2048^2 case small."""
    from flicker_amd import workloads
    w = workloads.WORKLOADS[name]
    ids = workloads.make_ids(w)
    length, heads = ids.shape[0], 2
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(1, length, 3 * heads * D, generator=g).to(torch.bfloat16)
    qs, ks = workloads.make_scales(w)
    via_ids, via_tables, _ = _ids_and_tables_paths(device, qkv, qs, ks, ids, heads, workloads.q_gain(w))
    for n, a, b in zip("qkv", via_ids, via_tables):
        assert torch.equal(a, b), f"{name} {n}: ids path differs from the table path"


def test_double_attention_with_position_ids(device):
    """A double block's attention section is identical with ids or tables as the RoPE source."""
    from flicker_amd import rope
    heads, n_txt, n_img = 24, 512, 256
    txt, qs_t, ks_t, _ = make_case(1, n_txt, heads, seed=31)
    img, qs_i, ks_i, _ = make_case(1, n_img, heads, seed=32)
    ids = torch.from_numpy(rope.sequence_ids(n_txt, 16, 16)).to(device)
    dev = lambda *ts: tuple(t.to(device) for t in ts)  # noqa: E731
    out = []
    for src in (rope.position_ids(ids, 1 / math.sqrt(128)), rope.rope_lanes(ids, 1 / math.sqrt(128))):
        out.append(modules.double_attention(*dev(txt, img), dev(qs_t, ks_t), dev(qs_i, ks_i), src, heads))
    torch.cuda.synchronize()
    assert torch.equal(out[0][0], out[1][0]) and torch.equal(out[0][1], out[1][1])


def test_qk_prep_random_shapes(device):
    """Seeded random shapes (batch, ragged length, any head count, so every heads-per-group
    variant; gains; bf16 or f32 scales): the position-id form equals the table form bit for
    bit, and both hold the oracle gate."""
    rng = np.random.default_rng(31)
    for trial in range(8):
        batch, length, heads = int(rng.integers(1, 4)), int(rng.integers(1, 700)), int(rng.integers(1, 26))
        gain = float(rng.choice([1.0, 1 / math.sqrt(128), 0.37]))
        f32 = trial % 3 == 2
        label = f"random B{batch} L{length} H{heads} gain{gain:.4f} {'f32' if f32 else 'bf16'} scales"
        print(label, flush=True)
        qkv, qs, ks, ids = make_case(batch, length, heads, seed=300 + trial,
                                     scale_dtype=torch.float32 if f32 else torch.bfloat16)
        via_ids, via_tables, lanes = _ids_and_tables_paths(device, qkv, qs, ks, ids, heads, gain)
        for name, a, b in zip("qkv", via_ids, via_tables):
            assert torch.equal(a, b), f"{label}: {name} of the ids form differs from the table form"
        want = P.qk_prep_fused(to_np(qkv), to_np(qs), to_np(ks), lanes, heads, scale_is_bf16=not f32,
                               return_normed=True)
        check_qkv(label, via_tables, want, gain)
