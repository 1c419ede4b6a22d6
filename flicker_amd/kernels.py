"""Drop-in replacements for kelechi-c/flicker's ``kernels`` module (src/flicker/kernels.py).

Same names, call signatures, argument meaning and errors as the reference, over torch
tensors on an MI355X; every computation runs in the HIP kernels of libflicker_hip.so.

  Freqs, EPS, ROW_TILES, row_tile, lane_pair     kernels.py:12-31
  qk_prep                                         kernels.py:57-91  -> flk_qk_prep
  SCORE_TILES, EXP_LIMIT, logit_bound             kernels.py:94-101
  attend                                          kernels.py:105-145 -> flk_attend
  attend_merged = merge_heads(attend(...))        + modules.py:63-65 -> flk_attend_to

Beyond the reference, ``qk_prep`` takes optional ``out=(q, k, v)`` / ``out_offset`` so
the text and image streams of a double block can be written straight into one
concatenated buffer, and it accepts a strided ``qkv`` view (e.g. the qkv part of a
single block's fused linear1 output) without a copy.  In place of ``Freqs`` it also
accepts ``PositionIds``: the kernel then computes the RoPE lanes from the position ids
(rope.py:9-21 + kernels.py:28-31, -> flk_qk_prep_ids) instead of reading two f32 tables.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch

from . import _lib

HEAD_DIM = 128  # the only head width the HIP kernels are built for (Klein 4B: 3072 / 24)


class Freqs(NamedTuple):
    """kernels.py:12-16 -- (L, 128) float32 cos / sin lane tables and the static query gain."""

    cos: torch.Tensor
    sin: torch.Tensor
    q_gain: float = 1.0


class PositionIds(NamedTuple):
    """Position ids (L, n_axes) float32 on the GPU and the RoPE constants from which qk_prep
    computes its cos / sin lanes in-kernel; the values equal ``rope.rope_lanes(ids, q_gain,
    axes_dim, theta)`` bit for bit.  Defaults are Klein 4B's (config.py:36: four axes of 32,
    theta 2000)."""

    ids: torch.Tensor
    q_gain: float = 1.0
    axes_dim: tuple = (32, 32, 32, 32)
    theta: float = 2000.0


EPS = 1e-6
ROW_TILES = (2304, 1536, 1152, 512, 256, 128, 64)


def row_tile(length: int) -> int | None:
    """kernels.py:23-24 -- the first row tile dividing ``length``, else None."""
    for size in ROW_TILES:
        if length % size == 0:
            return size
    return None


def _on_gpu(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} is on {t.device}; flicker_amd runs its kernels on the GPU only")


def _dense_rows(t: torch.Tensor) -> torch.Tensor:
    """Keep a view whose last axis is contiguous and whose other strides keep 16-byte rows;
    anything else is compacted on the device first."""
    ok = t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def lane_pair(freqs: torch.Tensor, q_gain: float = 1.0) -> Freqs:
    """kernels.py:28-31 -- rope table (1, 1, L, P, 2, 2) -> (L, 2P) cos / sin lanes
    (batch 0, head-broadcast 0), computed by flk_lane_pair."""
    _on_gpu("freqs", freqs)
    if freqs.dim() < 3 or freqs.shape[-2:] != (2, 2):
        raise ValueError(f"freqs must end in (..., L, P, 2, 2), got {tuple(freqs.shape)}")
    pe = freqs
    while pe.dim() > 4:
        pe = pe[0]
    pe = pe.to(torch.float32).contiguous()
    length, pairs = pe.shape[0], pe.shape[1]
    cos = torch.empty((length, 2 * pairs), dtype=torch.float32, device=pe.device)
    sin = torch.empty_like(cos)
    _lib.run("flk_lane_pair", (pe, cos, sin), pe.data_ptr(), length, pairs, cos.data_ptr(), sin.data_ptr(),
             _lib.stream_of(pe))
    return Freqs(cos, sin, float(q_gain))


def _table_args(freqs: Freqs, length: int, head_dim: int):
    cos, sin, _ = freqs
    for name, t in (("freqs.cos", cos), ("freqs.sin", sin)):
        _on_gpu(name, t)
    if cos.shape != (length, head_dim) or sin.shape != (length, head_dim):
        raise ValueError(f"freqs tables must be ({length}, {head_dim}), got {tuple(cos.shape)} / {tuple(sin.shape)}")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise TypeError("freqs.cos / freqs.sin must be float32")
    cos = cos if cos.stride(1) == 1 and cos.stride(0) % 4 == 0 and cos.data_ptr() % 16 == 0 else cos.contiguous()
    sin = sin if sin.stride(1) == 1 and sin.stride(0) % 4 == 0 and sin.data_ptr() % 16 == 0 else sin.contiguous()
    if sin.stride(0) != cos.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    return cos, sin


def _id_args(pos: PositionIds, length: int, head_dim: int):
    ids = pos.ids
    _on_gpu("ids", ids)
    if ids.dim() == 3:
        ids = ids[0]   # batch 0, as lane_pair takes (kernels.py:30)
    if ids.dim() != 2 or ids.shape[0] != length or ids.shape[1] != len(pos.axes_dim):
        raise ValueError(f"ids must be ({length}, {len(pos.axes_dim)}), got {tuple(pos.ids.shape)}")
    if ids.dtype != torch.float32:
        raise TypeError(f"ids must be float32, got {ids.dtype}")
    if sum(pos.axes_dim) != head_dim:
        raise ValueError(f"axes_dim {tuple(pos.axes_dim)} must sum to head_dim {head_dim}")
    return ids if ids.stride(1) == 1 else ids.contiguous()


def _launch_qk_prep(qkv, q_scale, k_scale, freqs, num_heads: int, out, out_offset: int,
                    qk_f32: bool = False):
    """qk_prep's launch.  ``qk_f32``: the plain branch of qkv_prep with float32 scales
    (modules.py:78-80, where rms_norm's product and apply_rope's result stay float32): q and
    k come out float32, unrounded and without a query gain (flk_qk_prep_f32); v stays bf16."""
    batch, length, width = qkv.shape
    head_dim = width // (3 * num_heads)
    if 3 * num_heads * head_dim != width:
        raise ValueError(f"qkv width {width} is not 3 * num_heads({num_heads}) * head_dim")
    if head_dim != HEAD_DIM:
        raise ValueError(f"qk_prep: head_dim {head_dim} unsupported (kernels are built for {HEAD_DIM})")
    if qkv.dtype != torch.bfloat16:
        raise TypeError(f"qkv must be bfloat16, got {qkv.dtype}")
    if isinstance(freqs, PositionIds):
        rope = _id_args(freqs, length, head_dim)
    elif isinstance(freqs, Freqs) or (isinstance(freqs, tuple) and len(freqs) == 3):
        freqs = Freqs(*freqs)
        rope = _table_args(freqs, length, head_dim)
    else:
        raise TypeError(f"freqs must be Freqs or PositionIds, got {type(freqs).__name__}")
    q_gain = freqs.q_gain
    for name, t in (("q_scale", q_scale), ("k_scale", k_scale)):
        _on_gpu(name, t)
    if q_scale.numel() != head_dim or k_scale.numel() != head_dim:
        raise ValueError(f"q_scale / k_scale must hold {head_dim} values")
    if q_scale.dtype != k_scale.dtype or q_scale.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("q_scale and k_scale must share one dtype, bfloat16 or float32")
    if qk_f32 and (q_scale.dtype != torch.float32 or isinstance(freqs, PositionIds) or q_gain != 1.0):
        raise ValueError("float32 q / k outputs are the plain branch's: float32 scales, lane tables, gain 1")
    qk_dtype = torch.float32 if qk_f32 else torch.bfloat16
    qkv = _dense_rows(qkv)
    q_scale = q_scale.reshape(-1).contiguous()
    k_scale = k_scale.reshape(-1).contiguous()

    if out is None:
        if out_offset:
            raise ValueError("out_offset needs out=(q, k, v)")
        shape = (batch, num_heads, length, head_dim)
        out = tuple(torch.empty(shape, dtype=dt, device=qkv.device) for dt in (qk_dtype, qk_dtype, torch.bfloat16))
        out_length = length
    else:
        out = tuple(out)
        if len(out) != 3:
            raise ValueError("out must be a (q, k, v) triple")
        out_length = out[0].shape[2]
        for t, dt in zip(out, (qk_dtype, qk_dtype, torch.bfloat16)):
            _on_gpu("out", t)
            if (t.dtype != dt or t.dim() != 4 or t.shape[0] != batch or t.shape[1] != num_heads
                    or t.shape[3] != head_dim or t.shape[2] != out_length or not t.is_contiguous()):
                raise ValueError(f"out tensors must be contiguous (B, H, L_out, D) of one shape, q and k "
                                 f"{qk_dtype}, v bfloat16")
        if out_offset < 0 or out_offset + length > out_length:
            raise ValueError(f"out_offset {out_offset} + L {length} exceeds the output length {out_length}")

    if qk_f32:
        cos, sin = rope
        _lib.run("flk_qk_prep_f32", (qkv, cos, sin, q_scale, k_scale, *out),
                 qkv.data_ptr(), qkv.stride(0), qkv.stride(1), cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 q_scale.data_ptr(), k_scale.data_ptr(), batch, length, num_heads, head_dim,
                 out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), out_length, out_offset,
                 _lib.stream_of(qkv))
        return out
    common = (q_scale.data_ptr(), k_scale.data_ptr(), int(q_scale.dtype == torch.float32), float(q_gain),
              batch, length, num_heads, head_dim, out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
              out_length, out_offset, _lib.stream_of(qkv))
    if isinstance(freqs, PositionIds):
        _lib.run("flk_qk_prep_ids", (qkv, rope, q_scale, k_scale, *out),
                 qkv.data_ptr(), qkv.stride(0), qkv.stride(1), rope.data_ptr(), rope.stride(0),
                 len(freqs.axes_dim), _lib.int_array(freqs.axes_dim), float(freqs.theta), *common)
    else:
        cos, sin = rope
        _lib.run("flk_qk_prep", (qkv, cos, sin, q_scale, k_scale, *out),
                 qkv.data_ptr(), qkv.stride(0), qkv.stride(1), cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 *common)
    return out


def qk_prep(qkv: torch.Tensor, q_scale: torch.Tensor, k_scale: torch.Tensor,
            freqs: Freqs | PositionIds, num_heads: int, *, rows: int | None = None,
            interpret: bool = False,
            out=None, out_offset: int = 0):
    """kernels.py:57-91 -- fused head transpose + QK-RMSNorm + RoPE (+ q_gain on q).

    qkv (B, L, 3*H*D) bf16 -> q, k, v (B, H, L, D) bf16.  ``freqs`` is a Freqs (lane
    tables) or a PositionIds (lanes computed in-kernel, same values).  As in the reference, ``rows``
    (or the default row tile) must divide L; the HIP kernel itself tiles by 16 tokens."""
    if interpret:
        raise ValueError("interpret=True is Pallas' CPU emulation; flicker_amd has one HIP path")
    if qkv.dim() != 3:
        raise ValueError(f"qkv must be (B, L, 3*H*D), got {tuple(qkv.shape)}")
    length = qkv.shape[1]
    tile_rows = rows or row_tile(length)
    if tile_rows is None or length % tile_rows:
        raise ValueError(f"qk_prep needs a row tile dividing L={length} (rows={tile_rows})")
    _on_gpu("qkv", qkv)
    return _launch_qk_prep(qkv, q_scale, k_scale, freqs, num_heads, out, out_offset)


SCORE_TILES = (2304, 1536, 1152, 512, 256, 128)
EXP_LIMIT = 80.0


def logit_bound(q_scale, k_scale):
    """kernels.py:99-101 -- sqrt(D) * max|q_scale| * max|k_scale| over the last axis: an upper
    bound on |q.k|/sqrt(D) after QK-RMSNorm (unit-RMS rows, orthogonal RoPE, Cauchy-Schwarz)."""
    q_scale = torch.as_tensor(q_scale, dtype=torch.float32)
    k_scale = torch.as_tensor(k_scale, dtype=torch.float32)
    width = q_scale.shape[-1]
    return math.sqrt(width) * q_scale.abs().amax(-1) * k_scale.abs().amax(-1)


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block: int | None = None,
           interpret: bool = False, out: torch.Tensor | None = None,
           splits: int | None = None) -> torch.Tensor:
    """kernels.py:105-145 -- bounded flash attention (no running max), q pre-scaled by
    1/sqrt(D).  q, k, v (B, H, L, D) bf16 -> o (B, H, L, D) bf16.

    Grids too small to fill the GPU (few heads or short sequences) cut the keys into ranges
    whose partial sums are added afterwards (flk_attend_split_to); ``splits`` overrides the
    automatic choice (1 = never split)."""
    if interpret:
        raise ValueError("interpret=True is Pallas' CPU emulation; flicker_amd has one HIP path")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != 4:
            raise ValueError(f"{name} must be (B, H, L, D), got {tuple(t.shape)}")
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    batch, heads, length, dim = q.shape
    # as in the reference: no score tile dividing L raises StopIteration (kernels.py:110)
    block = block or next(size for size in SCORE_TILES if length % size == 0)
    if length % block:
        raise ValueError(f"attend block {block} does not divide L={length}")
    if dim != HEAD_DIM:
        raise ValueError(f"attend: head_dim {dim} unsupported (kernels are built for {HEAD_DIM})")
    for name, t in (("q", q), ("k", k), ("v", v)):
        _on_gpu(name, t)
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor shaped like q")
    _launch_attend(q, k, v, out, (heads * length * dim, length * dim, dim), splits)
    return out


def attend_merged(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                  out: torch.Tensor | None = None, splits: int | None = None) -> torch.Tensor:
    """``merge_heads(attend(q, k, v))`` (modules.py:63-65 after kernels.py:105-145) in one
    kernel: the attention epilogue writes o[b, t, h*D:(h+1)*D] directly, so the transposing
    copy of merge_heads disappears.  q, k, v (B, H, L, D) bf16 -> (B, L, H*D) bf16; ``out`` may
    be a (B, L, H*D) view whose rows are strided (e.g. columns of a wider buffer)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != 4:
            raise ValueError(f"{name} must be (B, H, L, D), got {tuple(t.shape)}")
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    batch, heads, length, dim = q.shape
    if dim != HEAD_DIM:
        raise ValueError(f"attend: head_dim {dim} unsupported (kernels are built for {HEAD_DIM})")
    for name, t in (("q", q), ("k", k), ("v", v)):
        _on_gpu(name, t)
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if out is None:
        out = torch.empty((batch, length, heads * dim), dtype=torch.bfloat16, device=q.device)
    elif (out.shape != (batch, length, heads * dim) or out.dtype != torch.bfloat16 or out.stride(2) != 1
          or out.stride(0) % 4 or out.stride(1) % 4 or out.data_ptr() % 8):
        raise ValueError(f"out must be a bf16 ({batch}, {length}, {heads * dim}) view with contiguous, "
                         "4-element aligned rows")
    _on_gpu("out", out)
    _launch_attend(q, k, v, out, (out.stride(0), dim, out.stride(1)), splits)
    return out


def attend_kernels(batch: int, heads: int, length: int) -> tuple[str, ...]:
    """Names of the kernels ``attend`` launches for a (batch, heads, length, 128) problem, in
    order, as kernel traces show them (for profiling; the choice is _launch_attend's)."""
    splits, _ = _lib.attend_plan(batch, heads, length)
    if splits > 1:
        return ("attend_kernel<true>", "attend_merge_kernel")
    if _lib.attend_balanced_plan(batch, heads, length)[0] > 0:
        return ("attend_balanced_kernel",)
    return (_lib.attend_kernel_name(batch, heads, length),)


def _launch_attend(q, k, v, out, o_strides, splits: int | None, balanced: bool | None = None) -> None:
    """O through strides (batch, head, row): with ``splits`` None the plan's choice -- the
    key-split path when the grid is small, the balanced path (flk_attend_balanced_to: one
    persistent block per CU, the last round's tiles cut by keys) when flk_attend_balanced_plan
    prefers it, else one block per tile.  An explicit ``splits`` forces that split count
    (1 = one block per tile, flk_attend_to); ``balanced=True`` forces the balanced launch."""
    batch, heads, length, dim = q.shape
    planned, _ = _lib.attend_plan(batch, heads, length)
    groups = max(1, -(-length // 256))
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), batch, heads, length, dim, *o_strides)
    if balanced is None:
        balanced = splits is None and planned == 1 and _lib.attend_balanced_plan(batch, heads, length)[0] > 0
    if balanced:
        if splits not in (None, 1):
            raise ValueError(f"the balanced launch takes no key split, got splits={splits}")
        _, nbytes, counters = _lib.attend_balanced_plan(batch, heads, length)
        stream = _lib.stream_of(q)
        ws = _lib.balanced_workspace(q.device, stream, nbytes, counters)
        _lib.run("flk_attend_balanced_to", (q, k, v, out, ws), *args, ws.data_ptr(), nbytes, stream)
        return
    splits = planned if splits is None else int(splits)
    if not 1 <= splits <= groups:
        raise ValueError(f"splits must be in [1, {groups}] for L={length}, got {splits}")
    if splits == 1:
        _lib.run("flk_attend_to", (q, k, v, out), *args, _lib.stream_of(q))
        return
    nbytes = splits * batch * heads * groups * 512 * 65 * 4
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    _lib.run("flk_attend_split_to", (q, k, v, out, workspace), *args, splits, workspace.data_ptr(), nbytes,
             _lib.stream_of(q))
