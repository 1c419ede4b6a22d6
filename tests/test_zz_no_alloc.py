"""flk_attend_split_static_to (the key-split attend with the library's fixed scratch buffer
instead of a caller workspace) against flk_attend_split_to on the same inputs, through the C
ABI.  Both run the same split and merge kernels, so the outputs must be bit-identical.  Two
calls in a row, the second on a smaller problem, show that the shared buffer's leftovers from
the first call do not leak into the second.  The entry point exists for callers that cannot
allocate, such as code under HIP graph capture, so it is also captured into a graph and
replayed: once after an eager call has looked up the buffer's address, and once as the very
first call of a fresh process (the lookup then happens during the capture).  The refusal of
oversized requests is a host-side check, tested without a GPU in tests/test_host.py."""

import numpy as np
import pytest
import torch

from flicker_amd import _lib
from oracle import path as P
from tests._util import to_np
from tests.test_gpu_attend import tight_gate

pytestmark = pytest.mark.gpu
D = 128


def qkv(batch, heads, length, seed, device):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(3, batch, heads, length, D, generator=g)
    x[:2] /= x[:2].pow(2).mean(-1, keepdim=True).sqrt()   # unit-RMS rows, as after QK-RMSNorm
    x[0] /= D ** 0.5                                       # q pre-scaled by 1/sqrt(D)
    return tuple(t.to(torch.bfloat16).to(device) for t in x)


def both(q, k, v, splits):
    """(O of flk_attend_split_to with a torch workspace, O of flk_attend_split_static_to)."""
    batch, heads, length, _ = q.shape
    lib = _lib.lib()
    stream = _lib.stream_of(q)
    strides = (heads * length * D, length * D, D)
    nbytes = splits * batch * heads * -(-length // 256) * 512 * 65 * 4
    assert nbytes <= _lib.ATTEND_STATIC_SCRATCH_BYTES
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    o_ws, o_static = torch.empty_like(q), torch.empty_like(q)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr())
    _lib.check(lib.flk_attend_split_to(*args, o_ws.data_ptr(), batch, heads, length, D, *strides, splits,
                                       workspace.data_ptr(), nbytes, stream), "flk_attend_split_to")
    _lib.check(lib.flk_attend_split_static_to(*args, o_static.data_ptr(), batch, heads, length, D, *strides,
                                              splits, stream), "flk_attend_split_static_to")
    torch.cuda.synchronize()
    return o_ws, o_static


@pytest.mark.parametrize("first,second", [
    ((1, 3, 4608, None, 11), (1, 1, 1000, None, 12)),      # the head share, then a ragged single head
    ((1, 2, 4608, 7, 13), (2, 1, 700, 2, 14)),             # 33.5 MB of the buffer, then a smaller batch
])
def test_static_scratch_split_equals_workspace_split(device, first, second):
    for batch, heads, length, splits, seed in (first, second):
        print(f"no-alloc split: B={batch} H={heads} L={length} splits={splits} seed={seed}", flush=True)
        q, k, v = qkv(batch, heads, length, seed, device)
        planned, _ = _lib.attend_plan(batch, heads, length)
        splits = splits or planned
        assert splits > 1, "the case must take the split path"
        o_ws, o_static = both(q, k, v, splits)
        assert torch.equal(o_ws, o_static), f"B={batch} H={heads} L={length} splits={splits}"
        if length <= 1000:   # and both agree with the bounded oracle within attend's gate
            tight_gate(f"static split L={length}", to_np(o_static),
                       P.attend_bounded(to_np(q), to_np(k), to_np(v)).astype(np.float64))


def _inputs(batch, heads, length, seed, device):
    q, k, v = qkv(batch, heads, length, seed, device)
    return q.contiguous(), k.contiguous(), v.contiguous()


def test_static_scratch_split_replays_in_a_graph(device):
    """Captured on a side stream after an eager call, replayed with new inputs (eager work and
    synchronisations between replays): every replay equals flk_attend_split_to's output."""
    batch, heads, length, splits = 1, 3, 4608, 4
    lib = _lib.lib()
    static = list(_inputs(batch, heads, length, 21, device))
    static_o = torch.empty_like(static[0])
    strides = (heads * length * D, length * D, D)

    def call_static():
        _lib.check(lib.flk_attend_split_static_to(*(t.data_ptr() for t in static), static_o.data_ptr(), batch,
                                                  heads, length, D, *strides, splits, _lib.stream_of(static_o)),
                   "flk_attend_split_static_to")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call_static()                  # eager: the buffer's address is looked up here
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call_static()
    for seed in (22, 23, 24):
        print(f"graph replay: B={batch} H={heads} L={length} splits={splits} seed={seed}", flush=True)
        fresh = _inputs(batch, heads, length, seed, device)
        for dst, src in zip(static, fresh):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        replayed = static_o.clone()
        o_ws, _ = both(*fresh, splits)   # eager split work between the replays
        assert torch.equal(replayed, o_ws), f"replay with input seed {seed} differs from the eager split"


_FIRST_CALL_UNDER_CAPTURE = r"""
import sys, torch
sys.path.insert(0, {root!r})
from flicker_amd import _lib
from tests.test_zz_no_alloc import both, _inputs, D
dev = torch.device("cuda:0")
batch, heads, length, splits = 1, 2, 2048, 4
lib = _lib.lib()
static = list(_inputs(batch, heads, length, 31, dev))
static_o = torch.empty_like(static[0])
strides = (heads * length * D, length * D, D)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):   # the first call of flk_attend_split_static_to in this process
    _lib.check(lib.flk_attend_split_static_to(*(t.data_ptr() for t in static), static_o.data_ptr(), batch, heads,
                                              length, D, *strides, splits, _lib.stream_of(static_o)),
               "flk_attend_split_static_to")
for seed in (31, 32):
    fresh = _inputs(batch, heads, length, seed, dev)
    for dst, src in zip(static, fresh):
        dst.copy_(src)
    graph.replay()
    torch.cuda.synchronize()
    replayed = static_o.clone()
    o_ws, _ = both(*fresh, splits)
    assert torch.equal(replayed, o_ws), seed
    print("replay", seed, "equal", flush=True)
print("OK")
"""


def test_static_scratch_first_call_under_capture():
    """The first call on a GPU looks up the buffer's device address; made during a graph
    capture (torch's default global capture mode), the lookup is allowed and the captured
    launches replay bit-equal to the eager split.  Run in a fresh process, so that no earlier
    call has done the lookup."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("first static call under capture, in a child process: B=1 H=2 L=2048 splits=4", flush=True)
    proc = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE.format(root=root)], cwd=root,
                          capture_output=True, text=True, timeout=240)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0 and proc.stdout.strip().endswith("OK"), proc.returncode
