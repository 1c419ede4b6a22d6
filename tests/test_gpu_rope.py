"""RoPE tables on the GPU (flk_rope_embed / flk_lane_pair / flk_rope_lanes) against the
CPU restatement of rope.py:9-21 and kernels.py:28-31.

Device powf/cosf/sinf and the host's may differ by an ulp of the angle; for positions
up to 511 that moves cos/sin by < 1e-4, far below one bf16 ulp of the rotated output.
"""

import numpy as np
import pytest
import torch

from flicker_amd import kernels, rope
from oracle import path as P
from tests._util import to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-4


def ids_cases():
    g = np.random.default_rng(0)
    return {
        "klein_1024": P.sequence_ids(512, 64, 64),
        "klein_2048": P.sequence_ids(512, 128, 128),
        "random": g.integers(0, 512, size=(333, 4)).astype(np.float32),
    }


@pytest.mark.parametrize("case", list(ids_cases()))
def test_embed_nd_matches_oracle(device, case):
    ids = ids_cases()[case]
    got = to_np(rope.embed_nd(ids, device=device))
    want = P.embed_nd(ids)
    assert got.shape == want.shape
    err = np.abs(got - want).max()
    print(case, "embed_nd max abs", err)
    assert err <= ATOL


@pytest.mark.parametrize("case", list(ids_cases()))
def test_rope_lanes_and_lane_pair(device, case):
    ids = ids_cases()[case]
    fused = rope.rope_lanes(ids, 0.125, device=device)
    two_step = kernels.lane_pair(rope.embed_nd(ids, device=device), 0.125)
    want = P.lane_pair(P.embed_nd(ids), 0.125)
    for got in (fused, two_step):
        assert got.q_gain == 0.125
        for g, w in ((got.cos, want.cos), (got.sin, want.sin)):
            err = np.abs(to_np(g) - w).max()
            print(case, "lane table max abs", err)
            assert err <= ATOL
    # the fused kernel and the two-kernel route evaluate the same device expressions
    assert torch.equal(fused.cos, two_step.cos) and torch.equal(fused.sin, two_step.sin)


def test_rope_freqs_single_axis(device):
    pos = np.arange(0, 300, dtype=np.float32)
    got = to_np(rope.rope_freqs(pos, 32, device=device))
    want = P.rope_freqs(pos, 32)
    assert got.shape == want.shape == (300, 16, 2, 2)
    assert np.abs(got - want).max() <= ATOL
