"""The balanced attend (flk_attend_balanced_to: one persistent block per CU; the key tiles of
each XCD's tiles left over after its full rounds shared out in equal ranges over its CUs, the
pieces of a tile summed in a fixed order by whichever finishes last) against the bounded
oracle and against the one-block-per-tile kernel.

Gates: the tight bounded-oracle gate of test_gpu_attend; against flk_attend_to only the cut
tiles may differ, by the f32 order of two partial sums (at most one bf16 ulp of the largest
output); every output element is written (a NaN sentinel survives nowhere); repeated calls
are bit-identical (the merge order does not depend on which piece arrives first, and the
hand-off counters, tagged with each call's epoch, need no reset between calls); a workspace
whose counters hold any stale state -- a foreign epoch, a completed count, as left by calls
that overlapped on it -- gives the same result; a captured graph replays to the eager result."""

import math

import numpy as np
import pytest
import torch

from flicker_amd import _lib, kernels
from oracle import path as P
from tests._util import to_np
from tests.test_gpu_attend import prepped_case, tight_gate

pytestmark = pytest.mark.gpu
D = 128


def run(q, k, v, splits=None, balanced=True):
    out = torch.full_like(q, float("nan"))
    kernels._launch_attend(q, k, v, out, out.stride()[:3], splits, balanced)
    torch.cuda.synchronize()
    return out


def repeatable(q, k, v, first):
    """A second balanced call on the same workspace (its counters as the first call left them)
    gives the same bits."""
    return torch.equal(run(q, k, v), first)


def counters_of(q):
    batch, heads, length, _ = q.shape
    _, nbytes, off = _lib.attend_balanced_plan(batch, heads, length)
    ws = _lib._BALANCED_WORKSPACE[(q.device.index, _lib.stream_of(q))]
    return ws[off:nbytes].view(torch.int32)


@pytest.mark.parametrize("batch,heads,length", [(1, 128, 512), (1, 64, 1000), (2, 32, 1024), (1, 5, 1536),
                                                 (1, 9, 4352), (1, 40, 1000)])
def test_balanced_matches_oracle(device, batch, heads, length):
    """Exactly 256 (b, h, 256-query tile) units: no cut (L = 1000: a masked last key tile);
    30 units (3-4 tiles per XCD: every tile in 8-11 pieces); 153 units at 68 key tiles (19-20
    tiles per XCD, two pieces each); 160 units at L = 1000 (20 tiles per XCD, pieces ending
    on the masked last key tile)."""
    print(f"balanced B={batch} H={heads} L={length}", flush=True)
    q, k, v = prepped_case(batch, heads, length, seed=length + heads)
    qd, kd, vd = (t.to(device) for t in (q, k, v))
    got = run(qd, kd, vd)
    assert not torch.isnan(got).any(), "an output tile was never written"
    want = P.attend_bounded(to_np(q), to_np(k), to_np(v))
    tight_gate(f"balanced B{batch} H{heads} L{length}", to_np(got), want.astype(np.float64))
    plain = run(qd, kd, vd, splits=1, balanced=False)
    diff = (got.float() - plain.float()).abs()
    scale = float(plain.float().abs().max())
    assert float(diff.max()) <= 2.0 ** (math.floor(math.log2(scale)) - 7), float(diff.max())
    assert repeatable(qd, kd, vd, got)


def test_balanced_klein_1024_deterministic(device):
    """The headline shape (432 tiles): bit-identical over repeated calls, every element written,
    within one ulp of the one-block-per-tile kernel."""
    from flicker_amd import workloads
    w = workloads.WORKLOADS["klein_1024"]
    q, k, v = (t.to(device) for t in prepped_case(1, w.num_heads, w.length, seed=3))
    first = run(q, k, v)
    assert not torch.isnan(first).any()
    for i in range(10):
        again = run(q, k, v)
        assert torch.equal(first, again), f"call {i} differs"
    plain = run(q, k, v, splits=1, balanced=False)
    diff = (first.float() - plain.float()).abs()
    scale = float(plain.float().abs().max())
    assert float(diff.max()) <= 2.0 ** (math.floor(math.log2(scale)) - 7)
    print(f"klein_1024 balanced vs plain: mismatch {float((diff > 0).float().mean()):.3g}")
    # sampled rows of two heads against the oracle
    heads_sel, rows = [3, 17], np.linspace(0, w.length - 1, 256).astype(int)
    qs, ks, vs = (to_np(t)[:, heads_sel] for t in (q, k, v))
    want = P.attend_bounded(qs, ks, vs)[:, :, rows]
    tight_gate("klein_1024 sampled", to_np(first)[:, heads_sel][:, :, rows], want.astype(np.float64))


def test_balanced_graph_replay(device):
    """Captured on a side stream (workspace from the capture's pool, its counters zeroed by a
    captured fill), replayed three times with eager balanced calls between replays; 160
    tiles, so every tile is cut and merged through the counters.  Every replay carries the
    epoch of the captured call: each replay finds the previous one's counts complete and
    starts afresh."""
    heads, length = 40, 1024
    g = torch.Generator().manual_seed(9)

    def fresh():
        x = torch.randn(3, 1, heads, length, D, generator=g)
        x[:2] /= x[:2].pow(2).mean(-1, keepdim=True).sqrt()
        x[0] /= math.sqrt(D)
        return tuple(t.to(torch.bfloat16).to(device) for t in x)

    static = fresh()
    static_o = torch.empty_like(static[0])
    def attend(q, k, v, out=None):
        out = torch.empty_like(q) if out is None else out
        kernels._launch_attend(q, k, v, out, out.stride()[:3], None, True)
        return out

    attend(*static, out=static_o)      # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        attend(*static, out=static_o)
    for _ in range(3):
        new = fresh()
        for s, n in zip(static, new):
            s.copy_(n)
        graph.replay()
        eager = attend(*fresh())         # eager balanced work between replays
        torch.cuda.synchronize()
        want = attend(*new)
        torch.cuda.synchronize()
        assert torch.equal(static_o, want)
        assert eager.shape == want.shape


def test_balanced_ragged_batch_uneven_xcds(device):
    """B = 2, L = 1100: a partial last query tile (76 rows) and a masked last key tile (12
    keys); 50 tiles, so the XCDs hold 6 or 7 (units % 8 = 2) and every tile is shared."""
    q, k, v = prepped_case(2, 5, 1100, seed=21)
    qd, kd, vd = (t.to(device) for t in (q, k, v))
    got = run(qd, kd, vd)
    assert not torch.isnan(got).any()
    tight_gate("balanced B2 H5 L1100", to_np(got), P.attend_bounded(to_np(q), to_np(k), to_np(v)).astype(np.float64))
    plain = run(qd, kd, vd, splits=1, balanced=False)
    scale = float(plain.float().abs().max())
    assert float((got.float() - plain.float()).abs().max()) <= 2.0 ** (math.floor(math.log2(scale)) - 7)
    assert repeatable(qd, kd, vd, got)


def test_balanced_token_major_output(device):
    """O through the token-major strides of attend_merged (B, L, H*D): the same bits as the
    head-major output of the same launch, and the rows between heads untouched."""
    batch, heads, length = 1, 40, 1024
    q, k, v = (t.to(device) for t in prepped_case(batch, heads, length, seed=22))
    head_major = run(q, k, v)
    merged = torch.full((batch, length, heads * D + 8), float("nan"), dtype=torch.bfloat16, device=device)
    view = merged[..., :heads * D]
    kernels._launch_attend(q, k, v, view, (merged.stride(0), D, merged.stride(1)), None, True)
    torch.cuda.synchronize()
    assert torch.equal(view.view(batch, length, heads, D).transpose(1, 2), head_major)
    assert torch.isnan(merged[..., heads * D:]).all(), "a store landed past the head columns"
    assert repeatable(q, k, v, head_major)


@pytest.mark.parametrize("seed", range(6))
def test_three_launches_agree_on_random_shapes(device, seed):
    """Seeded random shapes (B <= 2, H <= 6, L in [1, 1300]): one block per tile, the key
    split at its planned (or a forced) range count, and the balanced launch each pass the tight
    oracle gate, and the split and balanced outputs stay within one bf16 ulp of the plain one."""
    rng = np.random.default_rng(100 + seed)
    batch, heads, length = int(rng.integers(1, 3)), int(rng.integers(1, 7)), int(rng.integers(1, 1301))
    q, k, v = prepped_case(batch, heads, length, seed=1000 + seed)
    want = P.attend_bounded(to_np(q), to_np(k), to_np(v)).astype(np.float64)
    qd, kd, vd = (t.to(device) for t in (q, k, v))
    groups = max(1, -(-length // 256))
    outs = {"plain": run(qd, kd, vd, splits=1, balanced=False),
            "split": run(qd, kd, vd, splits=min(groups, int(rng.integers(2, 5))) if groups > 1 else 1,
                         balanced=False),
            "balanced": run(qd, kd, vd)}
    print(f"seed {seed}: B={batch} H={heads} L={length}", flush=True)
    scale = float(outs["plain"].float().abs().max())
    for name, got in outs.items():
        assert not torch.isnan(got).any(), name
        tight_gate(f"{name} B{batch} H{heads} L{length}", to_np(got), want)
        d = float((got.float() - outs["plain"].float()).abs().max())
        assert d <= 2.0 ** (math.floor(math.log2(scale)) - 7), (name, d)
    assert repeatable(qd, kd, vd, outs["balanced"])


def test_balanced_recovers_from_stale_counters(device):
    """The hand-off counters hold (epoch << 8) | arrivals.  Whatever an earlier call left in
    them -- zero (a fresh workspace), a completed count, a count in the never-issued epoch 0,
    a partial count of a foreign epoch (two calls that overlapped on one workspace) -- the next
    call counts its own arrivals from zero and gives the bits of a call on a fresh workspace.
    160 tiles over 256 CUs: every tile is cut and merged through its counter."""
    heads, length = 40, 1024
    q, k, v = (t.to(device) for t in prepped_case(1, heads, length, seed=31))
    want = run(q, k, v)
    counters = counters_of(q)
    for name, value in (("zero", 0), ("epoch 0, 3 arrivals", 3), ("all ones", -1),
                        ("foreign epoch, 1 arrival", (0x7ABCDE << 8) | 1),
                        ("foreign epoch, 31 arrivals", (0x123456 << 8) | 31)):
        print(f"stale counters: {name}", flush=True)
        counters.fill_(value)
        torch.cuda.synchronize()
        got = run(q, k, v)
        assert torch.equal(got, want), name
