"""The C ABI on torch's current stream: side streams and captured HIP graphs.

Every entry point launches on the stream it is given (the Python wrappers pass torch's
current stream) and allocates nothing, so the path runs unchanged on a side stream and
inside a captured graph.  Graph tests replay several times with new inputs, with eager
work and synchronisations between the replays, and check every replay against the eager
result of the same input.
"""

import math

import pytest
import torch

from flicker_amd import kernels, rope, w8a8, workloads

pytestmark = pytest.mark.gpu
D = 128


def _case(seed, length=700, heads=8):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(1, length, 3 * heads * D, generator=g).to(torch.bfloat16)
    qs = (1 + 0.05 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ks = (1 + 0.05 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ids = rope.sequence_ids(188, 16, 32)   # 188 text + 512 image tokens = 700
    return qkv, qs, ks, ids, heads


def _attention(qkv, qs, ks, freqs, heads):
    q, k, v = kernels.qk_prep(qkv, qs, ks, freqs, heads, rows=qkv.shape[1])
    return kernels.attend(q, k, v, block=qkv.shape[1])


def test_side_stream_matches_default_stream(device):
    qkv, qs, ks, ids, heads = _case(1)
    qkv, qs, ks = qkv.to(device), qs.to(device), ks.to(device)
    freqs = rope.rope_lanes(ids, 1 / math.sqrt(D), device=device)
    want = _attention(qkv, qs, ks, freqs, heads)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()   # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = _attention(qkv, qs, ks, freqs, heads)
    side.synchronize()
    assert torch.equal(got, want)

    # the int8 projection too
    x, w = workloads.make_projection(workloads.Projection("t", 300, 384, 768))
    xd, wd = x.to(device), w.to(device)
    qw = w8a8.quantize_linear(wd, w8a8.absmax_cols(xd))
    y_want = w8a8.linear(xd, qw)
    torch.cuda.synchronize()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y_got = w8a8.linear(xd, qw)
    side.synchronize()
    assert torch.equal(y_got, y_want)


def test_graph_replay_qk_prep_attend(device):
    qkv0, qs, ks, ids, heads = _case(2)
    qs, ks = qs.to(device), ks.to(device)
    freqs = rope.rope_lanes(ids, 1 / math.sqrt(D), device=device)
    length = qkv0.shape[1]
    static_in = qkv0.to(device)
    outs = tuple(torch.empty((1, heads, length, D), dtype=torch.bfloat16, device=device) for _ in range(3))
    static_o = torch.empty_like(outs[0])

    def section():
        kernels.qk_prep(static_in, qs, ks, freqs, heads, rows=length, out=outs)
        kernels.attend(*outs, block=length, out=static_o)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        section()                      # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        section()

    for seed in (3, 4, 5):
        fresh = _case(seed)[0].to(device)
        static_in.copy_(fresh)
        graph.replay()
        torch.cuda.synchronize()
        replayed = static_o.clone()
        eager = _attention(fresh, qs, ks, freqs, heads)   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay with input seed {seed} differs from eager"


def test_graph_replay_attend_rounds(device):
    """The rounds launch (whole rounds of 256-query tiles, the leftover re-tiled by 192) keeps
    no state between calls, so a captured attend replays exactly: the Klein 1024^2 shape."""
    from flicker_amd import _lib
    heads, length = 24, 4608
    assert _lib.attend_kernel_name(1, heads, length) == "attend_rounds_kernel"

    def inputs(seed):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(3, 1, heads, length, D, generator=g)
        x[:2] = x[:2] / x[:2].pow(2).mean(-1, keepdim=True).sqrt()
        x[0] = x[0] / math.sqrt(D)
        return [t.to(torch.bfloat16).to(device) for t in x]

    static = inputs(20)
    static_o = torch.empty_like(static[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kernels.attend(*static, out=static_o)      # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.attend(*static, out=static_o)
    for seed in (21, 22, 23):
        fresh = inputs(seed)
        for dst, src in zip(static, fresh):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        replayed = static_o.clone()
        eager = kernels.attend(*fresh)                # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay with input seed {seed} differs from eager"


def test_graph_replay_int8_projection(device):
    proj = workloads.Projection("t", 512, 384, 3 * 2 * D)
    x0, w = workloads.make_projection(proj)
    wd = w.to(device)
    static_x = x0.to(device)
    qw = w8a8.quantize_linear(wd, w8a8.absmax_cols(static_x))
    static_y = torch.empty((proj.tokens, proj.out_features), dtype=torch.bfloat16, device=device)

    def section():
        xq, a = w8a8.quantize_act(static_x, qw.inv_smooth)
        w8a8.gemm(xq, a, qw.wq_t, qw.w_scale, out=static_y)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        section()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        section()

    for seed in (7, 8, 9):
        g = torch.Generator().manual_seed(seed)
        fresh = torch.randn(proj.tokens, proj.hidden, generator=g).to(torch.bfloat16).to(device)
        static_x.copy_(fresh)
        graph.replay()
        torch.cuda.synchronize()
        replayed = static_y.clone()
        eager = w8a8.linear(fresh, qw)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay with input seed {seed} differs from eager"


def test_graph_replay_attend_key_split(device):
    """The key-split path inside a graph: its workspace comes from torch's allocator during
    capture (the graph's own pool), and every replay equals the eager split result."""
    from flicker_amd import _lib
    heads, length = 3, 2048
    assert _lib.attend_plan(1, heads, length)[0] > 1

    def qkv_of(seed):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(3, 1, heads, length, D, generator=g)
        x = x / x.pow(2).mean(-1, keepdim=True).sqrt()
        return (x[0] / math.sqrt(D)).to(torch.bfloat16), x[1].to(torch.bfloat16), x[2].to(torch.bfloat16)

    static = tuple(t.to(device) for t in qkv_of(10))
    static_o = torch.empty_like(static[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kernels.attend(*static, out=static_o)      # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.attend(*static, out=static_o)
    for seed in (11, 12, 13):
        fresh = tuple(t.to(device) for t in qkv_of(seed))
        for dst, src in zip(static, fresh):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        replayed = static_o.clone()
        eager = kernels.attend(*fresh)                # eager split work between replays
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay with input seed {seed} differs from eager"
