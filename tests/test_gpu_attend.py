"""attend on the GPU (flk_attend) against the CPU restatement of kernels.py:105-145.

Two gates:
  * tight, against the bounded-attention restatement (same P rounding, same l):
    max |diff| <= 2 bf16 ulps of the largest output plus at most 1% of elements off;
  * the path's tolerance against the plain-XLA restatement (nn.py:35-44):
    max-abs <= 2e-2 and mean-abs <= 2e-3 on the bf16 output.
"""

import math

import numpy as np
import pytest
import torch

from flicker_amd import _lib, kernels
from oracle import path as P
from tests._util import abs_stats, describe, to_np

pytestmark = pytest.mark.gpu
D = 128
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def prepped_case(batch, heads, length, seed, scale=1.0):
    """q, k, v as qk_prep makes them: unit-RMS rows * scale, q pre-scaled by 1/sqrt(D)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(3, batch, heads, length, D, generator=g)
    x = x / x.pow(2).mean(-1, keepdim=True).sqrt()
    q = (x[0] * scale / math.sqrt(D)).to(torch.bfloat16)
    k = (x[1] * scale).to(torch.bfloat16)
    v = torch.randn(batch, heads, length, D, generator=g).to(torch.bfloat16)
    return q, k, v


def run_attend(q, k, v, device, splits=None):
    """Launch below kernels.attend's score-tile check, so any L can be tested; splits=None
    takes flk_attend_plan's choice (the key-split path on small grids)."""
    q, k, v = (t.to(device) for t in (q, k, v))
    out = torch.empty_like(q)
    kernels._launch_attend(q.contiguous(), k.contiguous(), v.contiguous(), out, out.stride()[:3], splits)
    torch.cuda.synchronize()
    return to_np(out)


def tight_gate(label, got, want):
    diff = np.abs(got.astype(np.float64) - want)
    scale = float(np.abs(want).max())
    ulp = 2.0 ** (math.floor(math.log2(scale)) - 7)
    st = {"max_abs": float(diff.max()), "mean_abs": float(diff.mean()),
          "max_ulps_of_max": float(diff.max() / ulp), "mismatch": float(np.mean(diff > 0))}
    print(describe(label, st))
    assert st["max_ulps_of_max"] <= 2.0, st
    assert st["mismatch"] <= 0.01, st


@pytest.mark.parametrize("batch,heads,length", [
    (1, 2, 64), (1, 2, 128), (2, 3, 1536), (1, 2, 4352),
    (1, 1, 1), (1, 2, 63), (1, 2, 65), (1, 2, 100), (1, 2, 257),
])
def test_attend_matches_bounded_oracle(device, batch, heads, length):
    q, k, v = prepped_case(batch, heads, length, seed=length)
    got = run_attend(q, k, v, device)
    want = P.attend_bounded(to_np(q), to_np(k), to_np(v))
    tight_gate(f"B{batch} H{heads} L{length}", got, want)


@pytest.mark.parametrize("heads,length", [(24, 1536), (5, 1000), (3, 4608), (2, 193)])
def test_attend_192_query_tiles_equal_256_query_tiles(device, heads, length):
    """A grid that fits the 256 CUs in one round with 192-query tiles as with 256-query ones
    runs the 192-query kernel (waves of two and of one 16-query group); every query's
    arithmetic is the 256-query kernel's, so the output is the same bit for bit.  The same
    heads repeated over a batch with more than 256 tiles of 256 queries run that kernel."""
    q, k, v = prepped_case(1, heads, length, seed=40 + length)
    small = run_attend(q, k, v, device, splits=1)
    reps = 256 // (heads * -(-length // 256)) + 1
    big = run_attend(*(t.expand(reps, -1, -1, -1) for t in (q, k, v)), device, splits=1)
    for b in range(reps):
        assert np.array_equal(big[b].view(np.uint32), small[0].view(np.uint32)), b
    tight_gate(f"192-query tiles H{heads} L{length}", small, P.attend_bounded(to_np(q), to_np(k), to_np(v)))


@pytest.mark.parametrize("batch,heads,length", [(1, 24, 4608), (1, 24, 4352), (1, 48, 1536), (3, 7, 4100)])
def test_attend_rounds_launch_equals_one_head_at_a_time(device, batch, heads, length):
    """Grids of more than one round run whole rounds of 256-query tiles per XCD and re-tile
    the queries of the tiles left over by 192 (leftover head segments that start mid-head,
    tiles cut short at a segment's end).  Each query's arithmetic is unchanged, so every head
    equals the same head launched alone (a one-round grid), bit for bit; two heads are also
    held to the bounded oracle."""
    q, k, v = prepped_case(batch, heads, length, seed=50 + length)
    got = run_attend(q, k, v, device, splits=1)
    for b in range(batch):
        for h in range(heads):
            one = run_attend(*(t[b:b + 1, h:h + 1] for t in (q, k, v)), device, splits=1)
            assert np.array_equal(got[b:b + 1, h:h + 1].view(np.uint32), one.view(np.uint32)), (b, h)
    for b, h in ((0, 0), (batch - 1, heads - 1)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        tight_gate(f"rounds B{batch} H{heads} L{length} head {b},{h}", got[sl],
                   P.attend_bounded(*(to_np(t[sl]) for t in (q, k, v))))


@pytest.mark.parametrize("batch,heads,length,kernel", [
    (1, 16, 4096, "attend_kernel"),           # exactly 256 tiles of 256 queries: one round
    (1, 16, 4097, "attend_rounds_kernel"),    # one tile per head more: the rounds launch
    (1, 11, 4608, "attend_kernel"),           # one round of 256-query tiles, not of 192
    (1, 10, 4608, "attend_tile192_kernel"),   # one round with either tiling
    (1, 28, 4608, "attend_kernel"),           # leftover needs more than one round of 192-query tiles
])
def test_attend_launch_boundaries_equal_one_head_at_a_time(device, batch, heads, length, kernel):
    """Shapes on either side of flk_attend's tiling choices take the kernel it names, and every
    head equals the same head launched alone, bit for bit."""
    assert _lib.attend_kernel_name(batch, heads, length) == kernel
    q, k, v = prepped_case(batch, heads, length, seed=60 + heads)
    got = run_attend(q, k, v, device, splits=1)
    for h in range(heads):
        one = run_attend(*(t[:, h:h + 1] for t in (q, k, v)), device, splits=1)
        assert np.array_equal(got[:, h:h + 1].view(np.uint32), one.view(np.uint32)), (kernel, h)


def test_attend_long_single_head_same_in_every_tiling(device):
    """One head of 65537 tokens (257 tiles of 256 queries: the rounds launch, its leftover
    segments inside that one head) equals itself batched twice (514 tiles, another split into
    rounds and leftover), bit for bit."""
    length = 65537
    assert _lib.attend_kernel_name(1, 1, length) == "attend_rounds_kernel"
    q, k, v = prepped_case(1, 1, length, seed=65)
    one = run_attend(q, k, v, device, splits=1)
    two = run_attend(*(t.expand(2, -1, -1, -1) for t in (q, k, v)), device, splits=1)
    for b in range(2):
        assert np.array_equal(two[b:b + 1].view(np.uint32), one.view(np.uint32)), b


def test_attend_random_shapes_every_launch_equals_one_head_at_a_time(device):
    """Seeded random shapes, each launched whole (flk_attend picks 256-query tiles, 192-query
    tiles or the rounds launch; the name it reports is checked against the three) and one head
    at a time: every head is the same bit for bit, whatever tiling the whole grid took."""
    rng = np.random.default_rng(2024)
    seen = set()
    for trial in range(8):
        while True:   # alternately more and fewer than 256 tiles of 256 queries
            batch, heads, length = int(rng.integers(1, 4)), int(rng.integers(1, 41)), int(rng.integers(1, 5200))
            tiles = batch * heads * -(-length // 256)
            if (256 < tiles <= 700) if trial % 2 == 0 else (tiles <= 256):
                break
        name = _lib.attend_kernel_name(batch, heads, length)
        assert name in ("attend_kernel", "attend_tile192_kernel", "attend_rounds_kernel"), name
        seen.add(name)
        q, k, v = prepped_case(batch, heads, length, seed=100 + trial)
        got = run_attend(q, k, v, device, splits=1)
        for b in range(batch):
            for h in range(heads):
                one = run_attend(*(t[b:b + 1, h:h + 1] for t in (q, k, v)), device, splits=1)
                assert np.array_equal(got[b:b + 1, h:h + 1].view(np.uint32), one.view(np.uint32)), \
                    (batch, heads, length, name, b, h)
    print("launches exercised:", sorted(seen))


def test_attend_peaked_logits(device):
    """Large norm scales (bound 11.3 * 2.4^2 = 65 < 80): far-from-uniform attention."""
    q, k, v = prepped_case(1, 2, 512, seed=5, scale=2.4)
    got = run_attend(q, k, v, device)
    want = P.attend_bounded(to_np(q), to_np(k), to_np(v))
    tight_gate("peaked", got, want)


def test_attend_uniform_keys_give_mean_of_values(device):
    """All keys equal -> every weight is 1/L -> o = mean(v) (rounded to bf16)."""
    q, k, v = prepped_case(1, 2, 256, seed=6)
    k = k[:, :, :1].expand_as(k).contiguous()
    got = run_attend(q, k, v, device)
    mean_v = to_np(v).astype(np.float64).mean(axis=2, keepdims=True)
    st = abs_stats(got, np.broadcast_to(mean_v, got.shape))
    print(describe("uniform keys", st))
    assert st["max_abs"] <= 2e-3


def test_attend_dominant_key_selects_its_value(device):
    """One key aligned with the query at logit ~ 60 outweighs 255 others at ~0."""
    length = 256
    q = torch.zeros(1, 1, length, D)
    q[..., 0] = 60.0 / math.sqrt(D) / 4          # q . k_0 = 60
    k = torch.zeros(1, 1, length, D)
    k[:, :, 7, 0] = 4 * math.sqrt(D)
    g = torch.Generator().manual_seed(8)
    v = torch.randn(1, 1, length, D, generator=g)
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    got = run_attend(q, k, v, device)
    want = np.broadcast_to(to_np(v)[:, :, 7:8], got.shape)
    st = abs_stats(got, want)
    print(describe("dominant key", st))
    assert st["max_abs"] <= 1e-2


def test_attend_python_api_errors(device):
    q, k, v = (t.to(device) for t in prepped_case(1, 1, 100, seed=1))
    with pytest.raises(StopIteration):
        kernels.attend(q, k, v)                 # no score tile divides 100, as in the reference
    with pytest.raises(ValueError):
        kernels.attend(q, k, v, block=64)
    with pytest.raises(ValueError):
        kernels.attend(q, k, v, interpret=True)


@pytest.mark.parametrize("batch,heads,length", [(1, 3, 100), (2, 2, 257), (1, 24, 1536), (1, 24, 4608), (1, 48, 1536)])
def test_attend_merged_equals_merge_heads_of_attend(device, batch, heads, length):
    """The token-major epilogue (flk_attend_to) writes exactly merge_heads(attend(q, k, v))
    (modules.py:63-65): same kernel, different store address -> bit-identical."""
    from flicker_amd import modules
    q, k, v = (t.to(device) for t in prepped_case(batch, heads, length, seed=11 + length))
    want = modules.merge_heads(kernels.attend(q, k, v, block=None if length % 128 == 0 else length))
    got = kernels.attend_merged(q, k, v)
    torch.cuda.synchronize()
    assert got.shape == (batch, length, heads * D)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # into the attention columns of a wider, row-strided buffer (e.g. a fused projection input)
    wide = torch.full((batch, length, heads * D + 64), 7.0, dtype=torch.bfloat16, device=device)
    kernels.attend_merged(q, k, v, out=wide[..., 32:32 + heads * D])
    torch.cuda.synchronize()
    assert torch.equal(wide[..., 32:32 + heads * D].view(torch.int16), want.view(torch.int16))
    assert bool((wide[..., :32] == 7.0).all()) and bool((wide[..., 32 + heads * D:] == 7.0).all())


@pytest.mark.parametrize("batch,heads,length,splits", [
    (1, 3, 4608, None), (1, 3, 4608, 2), (1, 2, 4352, None), (2, 3, 1536, 3), (1, 1, 1000, 4),
    (1, 1, 513, 3),
])
def test_attend_key_split_matches_oracle(device, batch, heads, length, splits):
    """The key-split path (flk_attend_split_to): each range's partial acc and l, then their
    plain sums -- the same gate as the one-pass kernel, and within rounding of it."""
    planned, _ = _lib.attend_plan(batch, heads, length)
    if splits is None:
        assert planned > 1, "the shape is meant to take the split path"
    q, k, v = prepped_case(batch, heads, length, seed=length + 3)
    got = run_attend(q, k, v, device, splits)
    want = P.attend_bounded(to_np(q), to_np(k), to_np(v))
    tight_gate(f"split {splits or planned} B{batch} H{heads} L{length}", got, want)
    one = run_attend(q, k, v, device, 1)
    diff = np.abs(got.astype(np.float64) - one)
    assert np.all(diff <= 2 * np.abs(one) * 2.0 ** -8 + 1e-6)   # one bf16 ulp of either value
    assert np.mean(diff > 0) <= 0.01


def test_attend_key_split_dominant_key_in_last_range(device):
    """A key near the end (the last of 4 ranges) at logit ~ 60 outweighs the others, so the
    merged output is its value row: the ranges' l and acc must be summed, not overwritten."""
    length = 2048
    q = torch.zeros(1, 1, length, D)
    q[..., 0] = 60.0 / math.sqrt(D) / 4
    k = torch.zeros(1, 1, length, D)
    k[:, :, 1900, 0] = 4 * math.sqrt(D)
    v = torch.randn(1, 1, length, D, generator=torch.Generator().manual_seed(9))
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    got = run_attend(q, k, v, device, 4)
    st = abs_stats(got, np.broadcast_to(to_np(v)[:, :, 1900:1901], got.shape))
    print(describe("split dominant key", st))
    assert st["max_abs"] <= 1e-2
    # uniform keys across ranges: o = mean(v) over all 2048 keys
    ku = torch.zeros(1, 1, length, D).to(torch.bfloat16)
    got = run_attend(q, ku, v, device, 4)
    mean_v = to_np(v).astype(np.float64).mean(axis=2, keepdims=True)
    assert abs_stats(got, np.broadcast_to(mean_v, got.shape))["max_abs"] <= 2e-3


def test_attend_merged_key_split(device):
    """attend_merged on the split path writes exactly merge_heads of the split attend."""
    from flicker_amd import modules
    q, k, v = (t.to(device) for t in prepped_case(1, 3, 4608, seed=21))
    assert _lib.attend_plan(1, 3, 4608)[0] > 1
    want = modules.merge_heads(kernels.attend(q, k, v))
    got = kernels.attend_merged(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    with pytest.raises(ValueError):
        kernels.attend(q, k, v, splits=19)     # more ranges than 256-key groups


def test_attend_key_split_long_sequence_matches_unsplit(device):
    """2048^2 Klein length (L = 16896) on one head: 66 query tiles plan 3 key ranges of 88
    tiles.  Too long for the oracle, so the split path is held to the one-pass kernel: the
    same sums in another f32 order, so at most one bf16 ulp apart on a few elements."""
    length = 16896
    planned, _ = _lib.attend_plan(1, 1, length)
    assert planned == 3
    q, k, v = prepped_case(1, 1, length, seed=31)
    split = run_attend(q, k, v, device)
    one = run_attend(q, k, v, device, 1)
    diff = np.abs(split.astype(np.float64) - one)
    assert np.all(diff <= 2 * np.abs(one) * 2.0 ** -8 + 1e-6)
    assert np.mean(diff > 0) <= 0.01


def test_attend_key_split_random_small_grids(device):
    """Seeded random small grids (fewer than 192 tiles of 256 queries), each on the range count
    flk_attend_plan picks: within one bf16 ulp of the one-pass kernel on at most 1% of
    elements, and at the tight oracle gate where the oracle is quick."""
    rng = np.random.default_rng(512)
    for trial in range(6):
        while True:
            batch, heads, length = int(rng.integers(1, 3)), int(rng.integers(1, 5)), int(rng.integers(200, 3000))
            planned, _ = _lib.attend_plan(batch, heads, length)
            if planned > 1:
                break
        label = f"split {planned} B{batch} H{heads} L{length}"
        print(label, flush=True)
        q, k, v = prepped_case(batch, heads, length, seed=700 + trial)
        got = run_attend(q, k, v, device)
        one = run_attend(q, k, v, device, 1)
        diff = np.abs(got.astype(np.float64) - one)
        assert np.all(diff <= 2 * np.abs(one) * 2.0 ** -8 + 1e-6), label
        assert np.mean(diff > 0) <= 0.01, label
        if length <= 1200:
            tight_gate(label, got, P.attend_bounded(to_np(q), to_np(k), to_np(v)))
