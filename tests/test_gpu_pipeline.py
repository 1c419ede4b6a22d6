"""The whole path on the GPU -- rope tables, qk_prep (gain 1/sqrt(D)), attend -- against the
plain-XLA restatement the reference falls back to (modules.py:78-80 + nn.py:35-44).

Gate (the path's stated tolerance): max-abs <= 2e-2 and mean-abs <= 2e-3 on the bf16
attention output.  Full-size workloads check a subset of heads against the oracle
(heads are independent) and the whole output for finiteness.
"""

import numpy as np
import pytest
import torch

from flicker_amd import kernels, modules, rope, workloads
from oracle import path as P
from tests._util import abs_stats, describe, to_np

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def run_path(w, device):
    qkv = workloads.make_qkv(w)
    qs, ks = workloads.make_scales(w)
    ids = workloads.make_ids(w)
    freqs = rope.rope_lanes(ids, workloads.q_gain(w), device=device)
    q, k, v = kernels.qk_prep(qkv.to(device), qs.to(device), ks.to(device), freqs, w.num_heads)
    o = kernels.attend(q, k, v)
    torch.cuda.synchronize()
    return qkv, qs, ks, ids, to_np(o)


def plain_path(qkv, qs, ks, ids, heads_sel, num_heads):
    q, k, v = P.qk_prep_plain(to_np(qkv), to_np(qs), to_np(ks), P.embed_nd(ids), num_heads)
    return P.sdpa(q[:, heads_sel], k[:, heads_sel], v[:, heads_sel])


@pytest.mark.parametrize("name,heads_sel", [
    ("klein_512", list(range(24))),
    ("klein_1024", [0, 7, 13, 23]),
    ("klein_1536x640", [3, 19]),
])
def test_path_matches_plain_xla(device, name, heads_sel):
    w = workloads.WORKLOADS[name]
    qkv, qs, ks, ids, got = run_path(w, device)
    assert np.isfinite(got).all()
    want = plain_path(qkv, qs, ks, ids, heads_sel, w.num_heads)
    st = abs_stats(got[:, heads_sel], want)
    print(describe(name, st))
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st


def test_path_batch4_stress_channels(device):
    """Batch 4 with 5% of QKV channels x8: the bound check passes and holds at run time."""
    from flicker_amd.loader import check_logit_bound
    w = workloads.WORKLOADS["klein_1024_b4"]
    qs, ks = workloads.make_scales(w)
    stacked = {"double_blocks": {f"{s}_attn.norm.{n}.scale": (qs if n == "query_norm" else ks)[None]
                                 for s in ("img", "txt") for n in ("query_norm", "key_norm")},
               "single_blocks": {"norm.query_norm.scale": qs[None], "norm.key_norm.scale": ks[None]}}
    check_logit_bound(stacked)
    bound = float(kernels.logit_bound(qs.float(), ks.float()))
    qkv, qs, ks, ids, got = run_path(w, device)
    assert np.isfinite(got).all()
    # runtime logits of batch 3, head 5 stay under the bound
    q, k, _ = P.qk_prep_fused(to_np(qkv[3:4]), to_np(qs), to_np(ks),
                              P.lane_pair(P.embed_nd(ids), workloads.q_gain(w)), w.num_heads)
    s = q[0, 5].astype(np.float64) @ k[0, 5].astype(np.float64).T
    assert np.abs(s).max() <= bound
    want = plain_path(qkv[3:4], qs, ks, ids, [5], w.num_heads)
    st = abs_stats(got[3:4, [5]], want)
    print(describe("klein_1024_b4 b3 h5", st), "max|S|", np.abs(s).max(), "bound", bound)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st


def test_double_block_attention_section(device):
    """Double block: txt and img streams prepped separately into one joint buffer, attended
    jointly, merged and split (modules.py:127-139,157-158) == the plain path on the
    concatenated sequence."""
    heads, n_txt, h, wd = 24, 512, 16, 16
    g = torch.Generator().manual_seed(31)
    txt = torch.randn(1, n_txt, 9216, generator=g).to(torch.bfloat16)
    img = torch.randn(1, h * wd, 9216, generator=g).to(torch.bfloat16)
    scales = [(1 + 0.05 * torch.randn(128, generator=g)).to(torch.bfloat16) for _ in range(4)]
    ids = P.sequence_ids(n_txt, h, wd)
    freqs = rope.rope_lanes(ids, 1 / np.sqrt(128), device=device)
    t_attn, i_attn = modules.double_attention(txt.to(device), img.to(device),
                                              (scales[0].to(device), scales[1].to(device)),
                                              (scales[2].to(device), scales[3].to(device)), freqs, heads)
    torch.cuda.synchronize()
    pe = P.embed_nd(ids)
    qt, kt, vt = P.qk_prep_plain(to_np(txt), to_np(scales[0]), to_np(scales[1]), pe[:, :, :n_txt], heads)
    qi, ki, vi = P.qk_prep_plain(to_np(img), to_np(scales[2]), to_np(scales[3]), pe[:, :, n_txt:], heads)
    o = P.sdpa(np.concatenate([qt, qi], 2), np.concatenate([kt, ki], 2), np.concatenate([vt, vi], 2))
    want = P.merge_heads(o)
    got = np.concatenate([to_np(t_attn), to_np(i_attn)], axis=1)
    st = abs_stats(got, want)
    print(describe("double block", st))
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st


def test_single_block_attention_section(device):
    heads, length = 24, 768
    g = torch.Generator().manual_seed(41)
    lin1 = torch.randn(1, length, 9216 + 18432, generator=g).to(torch.bfloat16)
    qs, ks = [(1 + 0.05 * torch.randn(128, generator=g)).to(torch.bfloat16) for _ in range(2)]
    ids = P.sequence_ids(256, 16, 32)
    freqs = rope.rope_lanes(ids, 1 / np.sqrt(128), device=device)
    attn, mlp = modules.single_attention(lin1.to(device), qs.to(device), ks.to(device), freqs, heads, 3072)
    torch.cuda.synchronize()
    q, k, v = P.qk_prep_plain(to_np(lin1)[..., :9216], to_np(qs), to_np(ks), P.embed_nd(ids), heads)
    st = abs_stats(to_np(attn), P.merge_heads(P.sdpa(q, k, v)))
    print(describe("single block", st))
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
    assert torch.equal(mlp.cpu(), lin1[..., 9216:])


def test_path_2048_long_sequence_sampled(device):
    """2048^2 Klein shape (512 text + 128x128 image tokens = 16896), full size on the GPU.
    The oracle restates two heads for 512 query rows spread over the sequence (text and
    image positions) against all 16896 keys -- attention rows are independent."""
    w = workloads.WORKLOADS["klein_2048"]
    qkv, qs, ks, ids, got = run_path(w, device)
    assert np.isfinite(got).all()
    heads_sel = [5, 17]
    rows = np.unique(np.concatenate([np.arange(0, 512, 16), np.linspace(512, w.length - 1, 480).astype(int)]))
    cols = [np.arange(s * w.num_heads * 128 + h * 128, s * w.num_heads * 128 + (h + 1) * 128)
            for s in range(3) for h in heads_sel]
    qkv_sel = to_np(qkv)[..., np.concatenate(cols)]
    q, k, v = P.qk_prep_plain(qkv_sel, to_np(qs), to_np(ks), P.embed_nd(ids), len(heads_sel))
    want = P.sdpa(q[:, :, rows], k, v)
    st = abs_stats(got[:, heads_sel][:, :, rows], want)
    print(describe("klein_2048 sampled", st))
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
