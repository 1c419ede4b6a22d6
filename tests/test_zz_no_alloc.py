"""flk_attend_split_static_to (the key-split attend with the library's fixed scratch buffer
instead of a caller workspace) against flk_attend_split_to on the same inputs, through the C
ABI.  Both run the same split and merge kernels, so the outputs must be bit-identical.  Two
calls in a row, the second on a smaller problem, show that the shared buffer's leftovers from
the first call do not leak into the second; a third, oversized request is refused before
anything is launched."""

import ctypes

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


def test_static_scratch_refuses_oversized_calls(device):
    q, k, v = qkv(1, 1, 64, 0, device)
    lib = _lib.lib()
    o = torch.empty_like(q)
    # 24 heads x 66 query tiles x 2 ranges = 3168 partial blocks: far beyond the fixed buffer
    st = lib.flk_attend_split_static_to(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), 1, 24, 16896, D,
                                        24 * 16896 * D, 16896 * D, D, 2, _lib.stream_of(q))
    assert st == _lib.FLK_E_SCRATCH
    assert "scratch" in _lib.status_string(st)
    assert isinstance(ctypes.c_int(st).value, int)
