"""The HIP kernels against the committed golden fixtures (tests/golden/*.npz), which are an
independent brute force of the reference's formulas (see tests/golden/make_golden.py)."""

import os

import numpy as np
import pytest
import torch

from flicker_amd import kernels, rope
from oracle.numerics import bf16_ulp, from_bf16_bits
from tests._util import to_np

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def bf16_tensor(bits, device):
    return torch.from_numpy(from_bf16_bits(bits)).to(torch.bfloat16).to(device)


def test_rope_lanes_golden(device):
    g = load("rope.npz")
    f = rope.rope_lanes(g["ids"], 1.0, device=device)
    for t in range(len(g["ids"])):
        atol = 4e-7 * max(1.0, float(np.abs(g["ids"][t]).max()))
        np.testing.assert_allclose(to_np(f.cos)[t], g["cos"][t], rtol=0, atol=atol)
        np.testing.assert_allclose(to_np(f.sin)[t], g["sin"][t], rtol=0, atol=atol)


@pytest.mark.parametrize("which", ["1", "g"])
def test_qk_prep_golden(device, which):
    g = load("qk.npz")
    gain = 1.0 if which == "1" else float(g["gain"])
    lanes = rope.rope_lanes(g["ids"], gain, device=device)
    # use the fixture's own tables' arithmetic: the kernel reads the oracle-exact tables
    from oracle import path as P
    ref = P.lane_pair(P.embed_nd(g["ids"]), gain)
    lanes = kernels.Freqs(torch.from_numpy(ref.cos).to(device), torch.from_numpy(ref.sin).to(device), gain)
    qkv = bf16_tensor(g["qkv"], device)
    q, k, v = kernels._launch_qk_prep(qkv, bf16_tensor(g["q_scale"], device), bf16_tensor(g["k_scale"], device),
                                      lanes, int(g["heads"]), None, 0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(v), from_bf16_bits(g["v" + which]))
    for got, want in ((q, g["q" + which]), (k, g["k" + which])):
        w = from_bf16_bits(want)
        diff = np.abs(to_np(got).astype(np.float64) - w)
        assert np.all(diff <= 2 * bf16_ulp(w) * (1 + abs(gain)) + 1e-7)
        assert np.mean(diff > 0) <= 0.01


def test_attend_golden(device):
    g = load("attn.npz")
    q, k, v = (bf16_tensor(g[n], device)[None] for n in ("q_pre", "k", "v"))
    o = torch.empty_like(q)
    kernels._launch_attend(q.contiguous(), k.contiguous(), v.contiguous(), o, o.stride()[:3], None)
    torch.cuda.synchronize()
    want = g["bounded"].astype(np.float64)
    diff = np.abs(to_np(o)[0] - want)
    assert np.all(diff <= 2 * bf16_ulp(want) + 1e-6), diff.max()
