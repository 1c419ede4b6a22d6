"""The attention sections of the Klein DiT blocks, wired to the HIP kernels.

Reference: src/flicker/modules.py -- heads :56-60, merge_heads :63-65, qkv_prep :68-80,
double_prepare_qkv :96-140 with double_block :156-158, single_prepare_qkv :180-191 with
single_block :197-198.  These functions take the already-projected QKV activations
(the linear/modulate parts of the blocks are outside this path) and return the
merged attention output, in the same order and layout as the reference; the merge is
done by the attention kernel's epilogue (kernels.attend_merged).
"""

from __future__ import annotations

import torch

from .kernels import Freqs, PositionIds, _launch_qk_prep, attend_merged, lane_pair, row_tile


def heads(qkv: torch.Tensor, num_heads: int):
    """modules.py:56-60 -- (B, L, 3*H*D) -> three (B, H, L, D) views (no copy)."""
    b, length, width = qkv.shape
    head_dim = width // (3 * num_heads)
    split = qkv.reshape(b, length, 3, num_heads, head_dim).permute(2, 0, 3, 1, 4)
    return split[0], split[1], split[2]


def merge_heads(x: torch.Tensor) -> torch.Tensor:
    """modules.py:63-65 -- (B, H, L, D) -> (B, L, H*D)."""
    b, h, n, d = x.shape
    return x.transpose(1, 2).reshape(b, n, h * d)


def qkv_prep(qkv, q_scale, k_scale, pe, freqs: Freqs | PositionIds | None, num_heads: int, *, out=None,
             out_offset: int = 0):
    """modules.py:68-80 -- QK-RMSNorm + RoPE + head split, with the reference's gate (:76):
    the fused form (``freqs``' lanes and ``freqs.q_gain``) when ``freqs`` is given and a row
    tile divides L; otherwise the plain branch (:78-80), which rotates by ``pe`` and applies
    no query gain.  Both branches run the one HIP kernel: the plain branch's lane tables are
    built from ``pe`` at gain 1 (lane_pair), whose rotation is bit-identical to apply_rope's
    2x2 form.  ``pe`` is (B_pe, 1, L, D/2, 2, 2); with B_pe > 1 each batch element is
    rotated by its own table, as apply_rope broadcasts it.

    The plain branch's output dtype follows the reference's promotion: with bfloat16 scales q
    and k are bfloat16; with float32 scales rms_norm's bf16(normed) * scale is float32
    (nn.py:27) and apply_rope casts its float32 rotation back to that dtype (rope.py:28), so
    q and k are float32, unrounded (flk_qk_prep_f32).  v is the bfloat16 split either way."""
    if freqs is not None and row_tile(qkv.shape[1]) is not None:
        return _launch_qk_prep(qkv, q_scale, k_scale, freqs, num_heads, out, out_offset)
    if pe is None:
        raise ValueError(f"qkv_prep: L={qkv.shape[1]} has no row tile (or freqs is None), so the plain "
                         "branch needs pe")
    qk_f32 = q_scale.dtype == torch.float32
    if pe.dim() < 6 or pe.shape[0] == 1:
        return _launch_qk_prep(qkv, q_scale, k_scale, lane_pair(pe, 1.0), num_heads, out, out_offset, qk_f32)
    batch = qkv.shape[0]
    if pe.shape[0] != batch:
        raise ValueError(f"pe batch {pe.shape[0]} does not broadcast against qkv batch {batch}")
    if out is None:
        shape = (batch, num_heads, qkv.shape[1], qkv.shape[2] // (3 * num_heads))
        qk_dtype = torch.float32 if qk_f32 else torch.bfloat16
        out = tuple(torch.empty(shape, dtype=dt, device=qkv.device) for dt in (qk_dtype, qk_dtype, torch.bfloat16))
    for b in range(batch):
        _launch_qk_prep(qkv[b:b + 1], q_scale, k_scale, lane_pair(pe[b:b + 1], 1.0), num_heads,
                        tuple(t[b:b + 1] for t in out), out_offset, qk_f32)
    return tuple(out)


def _slice(freqs, start: int, stop: int):
    """Rows start:stop of the RoPE source of the joint sequence (tables or position ids)."""
    if isinstance(freqs, PositionIds):
        ids = freqs.ids[0] if freqs.ids.dim() == 3 else freqs.ids
        return freqs._replace(ids=ids[start:stop])
    return Freqs(freqs.cos[start:stop], freqs.sin[start:stop], freqs.q_gain)


def double_attention(txt_qkv, img_qkv, txt_scales, img_scales, freqs: Freqs | PositionIds,
                     num_heads: int, *, pe=None, pe_ctx=None):
    """modules.py:127-139 + 157-158 -- per-stream qk prep, joint text|image attention, merge,
    split back into (txt_attn, img_attn), each (B, L_stream, H*D).

    Both qk_prep calls write into one (B, H, L_txt + L_img, D) buffer at their sequence
    offsets, which replaces the reference's three concatenations.  ``pe_ctx`` / ``pe`` are the
    text / image rope tables the reference hands each stream's qkv_prep (modules.py:129,133);
    they are read only by a stream whose length has no row tile (the gate's plain branch)."""
    batch, num_txt, width = txt_qkv.shape
    num_img = img_qkv.shape[1]
    for name, length, scales in (("text", num_txt, txt_scales), ("image", num_img, img_scales)):
        if row_tile(length) is None and scales[0].dtype == torch.float32:
            raise TypeError(f"double_attention: the {name} stream (L={length}, no row tile) takes qkv_prep's plain "
                            "branch, whose float32 norm scales give float32 q and k; attend takes bf16 operands only")
    head_dim = width // (3 * num_heads)
    shape = (batch, num_heads, num_txt + num_img, head_dim)
    joint = tuple(torch.empty(shape, dtype=torch.bfloat16, device=txt_qkv.device) for _ in range(3))
    qkv_prep(txt_qkv, *txt_scales, pe_ctx, _slice(freqs, 0, num_txt), num_heads, out=joint, out_offset=0)
    qkv_prep(img_qkv, *img_scales, pe, _slice(freqs, num_txt, num_txt + num_img), num_heads,
             out=joint, out_offset=num_txt)
    attn = attend_merged(*joint)   # merge_heads fused into the attention epilogue
    return attn[:, :num_txt], attn[:, num_txt:]


def double_attention_int8(txt_x, img_x, txt_qw, img_qw, txt_scales, img_scales, freqs: Freqs | PositionIds,
                          num_heads: int, *, modulation=None):
    """double_attention on the int8 path from the blocks' inputs: both streams' modulate +
    int8 quantisation in one launch and both projections with their qk prep in another
    (``w8a8.qk_prep_pair``, replacing modules.py:127-139), then the joint attention with
    merge_heads fused (modules.py:157-158).  ``modulation`` is ((shift, scale) of txt_mod,
    (shift, scale) of img_mod) or None for already-modulated inputs.  Returns (txt_attn,
    img_attn), each (B, L_stream, H*D)."""
    from . import w8a8
    num_txt = txt_x.shape[1]
    if isinstance(freqs, PositionIds):
        from .rope import rope_lanes
        freqs = rope_lanes(freqs.ids, freqs.q_gain, freqs.axes_dim, freqs.theta)
    txt = (txt_x, txt_qw, *txt_scales, _slice(freqs, 0, num_txt))
    img = (img_x, img_qw, *img_scales, _slice(freqs, num_txt, num_txt + img_x.shape[1]))
    joint = w8a8.qk_prep_pair(txt, img, num_heads, modulation=modulation)
    attn = attend_merged(*joint)
    return attn[:, :num_txt], attn[:, num_txt:]


def single_attention(linear1_out, q_scale, k_scale, freqs: Freqs | PositionIds, num_heads: int,
                     hidden: int, *, pe=None):
    """modules.py:185-191 + 198 -- the qkv part of the fused linear1 output (a strided view,
    consumed without a copy) -> qk prep -> attention -> merge; returns (attn, mlp).  ``pe``
    is the joint sequence's rope table, read only by the gate's plain branch (no row tile)."""
    qkv, mlp = linear1_out[..., : 3 * hidden], linear1_out[..., 3 * hidden:]
    q, k, v = qkv_prep(qkv, q_scale, k_scale, pe, freqs, num_heads)
    return attend_merged(q, k, v), mlp
