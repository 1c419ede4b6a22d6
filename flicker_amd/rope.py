"""RoPE position ids and tables (reference: src/flicker/rope.py, kernels.lane_pair).

Position ids are host numpy arrays, as in the reference (rope.py:33-45).  The tables
are built on the GPU by libflicker_hip.so:

  rope_freqs / embed_nd   rope.py:9-21     -> flk_rope_embed  ((..., L, P, 2, 2) rotation matrices)
  rope_lanes              embed_nd + kernels.lane_pair in one pass -> flk_rope_lanes
  position_ids            no table at all: qk_prep computes the lanes in-kernel -> flk_qk_prep_ids
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .config import Klein4B
from .kernels import Freqs, PositionIds

_KLEIN = Klein4B()


def img_ids(height: int, width: int, t: float = 0.0) -> np.ndarray:
    """rope.py:33-38 -- (1, h*w, 4) float32 ids (t, row, col, 0), row-major over the grid."""
    flat = np.arange(height * width)
    cols = [np.full(height * width, t), flat // width, flat % width, np.zeros(height * width)]
    return np.stack(cols, axis=-1).astype(np.float32)[None]


def txt_ids(length: int) -> np.ndarray:
    """rope.py:41-45 -- (1, n, 4) float32 ids (0, 0, 0, i)."""
    zeros = np.zeros(length)
    return np.stack([zeros, zeros, zeros, np.arange(length)], axis=-1).astype(np.float32)[None]


def sequence_ids(num_txt: int, height: int, width: int) -> np.ndarray:
    """dit.py:44-46 -- ids of the joint sequence, text first then image: (L, 4) float32."""
    return np.concatenate([txt_ids(num_txt)[0], img_ids(height, width)[0]], axis=0)


def _ids_on(ids, device) -> torch.Tensor:
    t = torch.as_tensor(ids, dtype=torch.float32)
    if device is not None:
        t = t.to(device)
    if t.device.type != "cuda":
        raise ValueError("RoPE tables are built on the GPU: pass ids on a cuda device or device='cuda'")
    return t.contiguous()


def embed_nd(ids, axes_dim=_KLEIN.axes_dim, theta: float = _KLEIN.theta, device=None) -> torch.Tensor:
    """rope.py:17-21 -- ids (L, A) or (B, L, A) -> pe (B, 1, L, sum(axes)/2, 2, 2) float32."""
    ids = _ids_on(ids, device)
    if ids.dim() == 2:
        ids = ids[None]
    batch, length, n_axes = ids.shape
    if n_axes != len(axes_dim):
        raise ValueError(f"ids have {n_axes} axes, axes_dim has {len(axes_dim)}")
    pairs = sum(axes_dim) // 2
    pe = torch.empty((batch, 1, length, pairs, 2, 2), dtype=torch.float32, device=ids.device)
    flat = ids.reshape(batch * length, n_axes)
    _lib.run("flk_rope_embed", (flat, pe), flat.data_ptr(), n_axes, batch * length, n_axes,
             _lib.int_array(axes_dim), float(theta), pe.data_ptr(), _lib.stream_of(pe))
    return pe


def rope_freqs(pos, dim: int, theta: float = _KLEIN.theta, device=None) -> torch.Tensor:
    """rope.py:9-14 -- positions (...) -> (..., dim/2, 2, 2) rotation matrices, one axis."""
    pos = _ids_on(pos, device)
    lead = pos.shape
    pe = embed_nd(pos.reshape(1, -1, 1), (dim,), theta)
    return pe.reshape(*lead, dim // 2, 2, 2)


def rope_lanes(ids, q_gain: float = 1.0, axes_dim=_KLEIN.axes_dim, theta: float = _KLEIN.theta,
               device=None) -> Freqs:
    """lane_pair(embed_nd(ids), q_gain) (kernels.py:28-31 over rope.py:17-21) in one kernel:
    ids (L, A) -> Freqs with (L, sum(axes)) float32 cos / sin lane tables."""
    ids = _ids_on(ids, device)
    if ids.dim() == 3:
        ids = ids[0]
    length, n_axes = ids.shape
    if n_axes != len(axes_dim):
        raise ValueError(f"ids have {n_axes} axes, axes_dim has {len(axes_dim)}")
    width = sum(axes_dim)
    cos = torch.empty((length, width), dtype=torch.float32, device=ids.device)
    sin = torch.empty_like(cos)
    _lib.run("flk_rope_lanes", (ids, cos, sin), ids.data_ptr(), n_axes, length, n_axes,
             _lib.int_array(axes_dim), float(theta), cos.data_ptr(), sin.data_ptr(), _lib.stream_of(cos))
    return Freqs(cos, sin, float(q_gain))


def position_ids(ids, q_gain: float = 1.0, axes_dim=_KLEIN.axes_dim, theta: float = _KLEIN.theta,
                 device=None) -> PositionIds:
    """The table-free RoPE source for qk_prep: ids (L, A) on the GPU plus the constants.
    qk_prep(..., position_ids(ids, g), ...) equals qk_prep(..., rope_lanes(ids, g), ...)
    bit for bit, without building or reading the two (L, sum(axes)) float32 tables."""
    ids = _ids_on(ids, device)
    if ids.dim() == 3:
        ids = ids[0]
    if ids.dim() != 2 or ids.shape[1] != len(axes_dim):
        raise ValueError(f"ids must be (L, {len(axes_dim)}), got {tuple(ids.shape)}")
    return PositionIds(ids, float(q_gain), tuple(int(a) for a in axes_dim), float(theta))
