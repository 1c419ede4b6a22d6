"""CPU restatement of flicker's DiT attention hot path (test infrastructure only).

Every function restates one reference function, cited as file:line into
kelechi-c/flicker's ``src/flicker/``.  Arrays are numpy; bf16 tensors are
represented as float32 arrays whose values are bf16-representable, and every
point where the reference rounds to bf16 is an explicit ``bf16_round``.

Arithmetic convention ("ideal float32"): where the reference reduces in
float32 with an order chosen by XLA or Mosaic (means, matmuls, softmax sums),
this restatement accumulates in float64 and rounds once to float32.  That is
the order-independent value every float32 order approximates; the HIP kernels
are compared to it with tolerances stated in the tests.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import numpy as np

from .numerics import bf16_round

F32 = np.float32
EPS = 1e-6                      # kernels.py:19, nn.py:24
ROW_TILES = (2304, 1536, 1152, 512, 256, 128, 64)   # kernels.py:20
SCORE_TILES = (2304, 1536, 1152, 512, 256, 128)     # kernels.py:94
EXP_LIMIT = 80.0                # kernels.py:95
AXES_DIM = (32, 32, 32, 32)     # config.py:35
THETA = 2000.0                  # config.py:36


# ----------------------------------------------------------------------------- RoPE tables
def rope_freqs(pos: np.ndarray, dim: int, theta: float = THETA) -> np.ndarray:
    """rope.py:9-14 -- (..., dim/2, 2, 2) rotation matrices [[cos, -sin], [sin, cos]]."""
    scale = np.arange(0, dim, 2, dtype=F32) / F32(dim)
    omega = F32(1.0) / np.power(F32(theta), scale, dtype=F32)
    angles = np.asarray(pos, dtype=F32)[..., None] * omega
    c, s = np.cos(angles, dtype=F32), np.sin(angles, dtype=F32)
    stacked = np.stack([c, -s, s, c], axis=-1)
    return stacked.reshape(*angles.shape, 2, 2)


def embed_nd(ids: np.ndarray, axes_dim=AXES_DIM, theta: float = THETA) -> np.ndarray:
    """rope.py:17-21 -- ids (B, L, n_axes) -> pe (B, 1, L, sum(axes)/2, 2, 2)."""
    ids = np.asarray(ids, dtype=F32)
    if ids.ndim == 2:
        ids = ids[None]
    per_axis = [rope_freqs(ids[..., i], axes_dim[i], theta) for i in range(len(axes_dim))]
    return np.concatenate(per_axis, axis=-3)[:, None]


def apply_rope(xq: np.ndarray, xk: np.ndarray, freqs: np.ndarray, out_bf16: bool = True):
    """rope.py:24-30 -- rotate (x[2j], x[2j+1]) pairs by the 2x2 matrices in f32, cast back."""
    def rotate(x):
        pairs = np.asarray(x, dtype=F32).reshape(*x.shape[:-1], -1, 1, 2)
        out = freqs[..., 0] * pairs[..., 0] + freqs[..., 1] * pairs[..., 1]
        out = out.reshape(*x.shape).astype(F32)
        return bf16_round(out) if out_bf16 else out
    return rotate(xq), rotate(xk)


def img_ids(height: int, width: int, t: float = 0.0) -> np.ndarray:
    """rope.py:33-38 -- (1, h*w, 4) ids (t, row, col, 0), row-major over the latent grid."""
    flat = np.arange(height * width)
    ids = np.stack([np.full(height * width, t), flat // width, flat % width,
                    np.zeros(height * width)], axis=-1).astype(F32)
    return ids[None]


def txt_ids(length: int) -> np.ndarray:
    """rope.py:41-45 -- (1, n, 4) ids (0, 0, 0, i)."""
    z = np.zeros(length)
    return np.stack([z, z, z, np.arange(length)], axis=-1).astype(F32)[None]


def sequence_ids(num_txt: int, height: int, width: int) -> np.ndarray:
    """dit.py:44-46 -- positions of the joint sequence: text ids then image ids, (L, 4)."""
    return np.concatenate([txt_ids(num_txt)[0], img_ids(height, width)[0]], axis=0)


class Freqs(NamedTuple):
    """kernels.py:12-16 -- lane tables for the fused kernel and the static query gain."""
    cos: np.ndarray
    sin: np.ndarray
    q_gain: float = 1.0


def lane_pair(pe: np.ndarray, q_gain: float = 1.0) -> Freqs:
    """kernels.py:28-31 -- (1,1,L,64,2,2) -> cos2/sin2 (L,128): cos2[2j]=cos2[2j+1]=cos_j,
    sin2[2j]=-sin_j, sin2[2j+1]=sin_j (batch 0, head-broadcast 0)."""
    cos, sin = pe[..., 0, 0][0, 0], pe[..., 1, 0][0, 0]
    lanes = np.stack([-sin, sin], axis=-1).reshape(*sin.shape[:-1], 2 * sin.shape[-1])
    return Freqs(np.repeat(cos, 2, axis=-1).astype(F32), lanes.astype(F32), q_gain)


def row_tile(length: int):
    """kernels.py:23-24."""
    return next((size for size in ROW_TILES if length % size == 0), None)


# ----------------------------------------------------------------------------- QK norm / heads
def _mean_square(x: np.ndarray) -> np.ndarray:
    """f32 mean of squares over the last axis, accumulated in f64 and rounded once."""
    x64 = x.astype(np.float64)
    return np.mean(x64 * x64, axis=-1, keepdims=True).astype(F32)


def _inv_rms(x: np.ndarray) -> np.ndarray:
    """lax.rsqrt(mean(x^2) + eps) as 1/sqrt in f32 (nn.py:26, kernels.py:44-45)."""
    return F32(1.0) / np.sqrt(_mean_square(x) + F32(EPS), dtype=F32)


def _scaled(normed_bf16: np.ndarray, scale: np.ndarray, scale_is_bf16: bool) -> np.ndarray:
    """bf16 x bf16 product rounds to bf16; a float32 scale promotes to float32 (nn.py:27)."""
    prod = (normed_bf16 * np.asarray(scale, dtype=F32)).astype(F32)
    return bf16_round(prod) if scale_is_bf16 else prod


def rms_norm(x: np.ndarray, scale: np.ndarray, scale_is_bf16: bool = True) -> np.ndarray:
    """nn.py:24-27 -- bf16(x * rsqrt(mean x^2 + 1e-6)) * scale."""
    xf = np.asarray(x, dtype=F32)
    normed = bf16_round(xf * _inv_rms(xf))
    return _scaled(normed, scale, scale_is_bf16)


def heads(qkv: np.ndarray, num_heads: int):
    """modules.py:56-60 -- (B, L, 3*H*D) -> three (B, H, L, D)."""
    b, length, _ = qkv.shape
    head_dim = qkv.shape[-1] // (3 * num_heads)
    split = qkv.reshape(b, length, 3, num_heads, head_dim).transpose(2, 0, 3, 1, 4)
    return split[0], split[1], split[2]


def merge_heads(x: np.ndarray) -> np.ndarray:
    """modules.py:63-65 -- (B, H, L, D) -> (B, L, H*D)."""
    b, h, n, d = x.shape
    return x.transpose(0, 2, 1, 3).reshape(b, n, h * d)


def qk_prep_plain(qkv, q_scale, k_scale, pe, num_heads, scale_is_bf16=True):
    """modules.py:78-80 (the plain-XLA branch of qkv_prep): heads -> qk_norm -> apply_rope."""
    q, k, v = heads(np.asarray(qkv, dtype=F32), num_heads)
    q = rms_norm(q, q_scale, scale_is_bf16)
    k = rms_norm(k, k_scale, scale_is_bf16)
    q, k = apply_rope(q, k, pe, out_bf16=scale_is_bf16)
    return q, k, v.copy()


def _pair_swap(x: np.ndarray) -> np.ndarray:
    """kernels.py:47 -- even lanes take x[i+1], odd lanes take x[i-1]."""
    out = np.empty_like(x)
    out[..., 0::2] = x[..., 1::2]
    out[..., 1::2] = x[..., 0::2]
    return out


def qk_prep_fused(qkv, q_scale, k_scale, freqs: Freqs, num_heads, scale_is_bf16=True,
                  return_normed: bool = False):
    """kernels.py:35-53,57-91 -- per (b, t, h): q,k <- bf16(gain * (cos2*y + sin2*swap(y))),
    y = f32(bf16(bf16(x * rsqrt(ms + EPS)) * scale)); v copied; outputs (B, H, L, D).
    The output is bf16 whatever the scale dtype (``.astype(value.dtype)``, kernels.py:49).
    With ``return_normed`` the pre-rotation y of q and k are returned as well."""
    q, k, v = heads(np.asarray(qkv, dtype=F32), num_heads)
    c = np.asarray(freqs.cos, dtype=F32)
    s = np.asarray(freqs.sin, dtype=F32)

    def prep(value, scale, gain):
        wide = _scaled(bf16_round(value * _inv_rms(value)), scale, scale_is_bf16)
        rotated = (c * wide + s * _pair_swap(wide)).astype(F32)
        if gain != 1.0:
            rotated = (F32(gain) * rotated).astype(F32)
        return bf16_round(rotated), wide

    (qo, qy), (ko, ky) = prep(q, q_scale, freqs.q_gain), prep(k, k_scale, 1.0)
    if return_normed:
        return qo, ko, v.copy(), qy, ky
    return qo, ko, v.copy()


def qkv_prep(qkv, q_scale, k_scale, pe, freqs: Freqs | None, num_heads, scale_is_bf16=True):
    """modules.py:68-80 -- the dispatch gate: the fused kernel (kernels.py:57-91, with
    ``freqs``' lanes and ``freqs.q_gain``) iff ``freqs`` is given and a row tile divides L
    (:76-77); otherwise the plain branch (:78-80), rotating by ``pe`` with no query gain."""
    if freqs is not None and row_tile(np.shape(qkv)[1]) is not None:
        return qk_prep_fused(qkv, q_scale, k_scale, freqs, num_heads, scale_is_bf16)
    return qk_prep_plain(qkv, q_scale, k_scale, pe, num_heads, scale_is_bf16)


# ----------------------------------------------------------------------------- attention
def _rows(length: int, chunk: int):
    for start in range(0, length, chunk):
        yield start, min(length, start + chunk)


def sdpa(q, k, v, chunk: int = 2048) -> np.ndarray:
    """nn.py:35-44 -- the plain-XLA attention: f32 logits * 1/sqrt(D), max-subtracted softmax,
    f32 weights @ V, cast to bf16.  Matmuls accumulate in f64 and round to f32."""
    q, k, v = (np.asarray(a, dtype=F32) for a in (q, k, v))
    batch, heads_, length, dim = q.shape
    scale = F32(1.0 / math.sqrt(dim))
    out = np.empty(q.shape, dtype=F32)
    for b in range(batch):
        for h in range(heads_):
            k64, v64 = k[b, h].astype(np.float64), v[b, h].astype(np.float64)
            for r0, r1 in _rows(length, chunk):
                logits = (q[b, h, r0:r1].astype(np.float64) @ k64.T).astype(F32) * scale
                shifted = (logits - logits.max(axis=-1, keepdims=True)).astype(F32)
                e = np.exp(shifted, dtype=F32)
                denom = e.astype(np.float64).sum(axis=-1, keepdims=True).astype(F32)
                w = (e / denom).astype(F32)
                out[b, h, r0:r1] = (w.astype(np.float64) @ v64).astype(F32)
    return bf16_round(out)


def attend_bounded(q, k, v, chunk: int = 2048, return_parts: bool = False):
    """kernels.py:105-145 -- bounded flash attention, q already scaled by 1/sqrt(D):
    S = q k^T (f32), P = bf16(exp S) with no max subtraction, l = sum f32(P),
    acc = P v (f32), O = bf16(acc / l)."""
    q, k, v = (np.asarray(a, dtype=F32) for a in (q, k, v))
    batch, heads_, length, dim = q.shape
    out = np.empty(q.shape, dtype=F32)
    acc_all = np.empty(q.shape, dtype=F32) if return_parts else None
    l_all = np.empty((batch, heads_, length), dtype=F32) if return_parts else None
    for b in range(batch):
        for h in range(heads_):
            k64, v64 = k[b, h].astype(np.float64), v[b, h].astype(np.float64)
            for r0, r1 in _rows(length, chunk):
                s = (q[b, h, r0:r1].astype(np.float64) @ k64.T).astype(F32)
                p = bf16_round(np.exp(s, dtype=F32))
                p64 = p.astype(np.float64)
                l_ = p64.sum(axis=-1, keepdims=True).astype(F32)
                acc = (p64 @ v64).astype(F32)
                out[b, h, r0:r1] = (acc / l_).astype(F32)
                if return_parts:
                    acc_all[b, h, r0:r1] = acc
                    l_all[b, h, r0:r1] = l_[:, 0]
    o = bf16_round(out)
    return (o, acc_all, l_all) if return_parts else o


def logit_bound(q_scale, k_scale) -> np.ndarray:
    """kernels.py:99-101 -- sqrt(D) * max|q_scale| * max|k_scale| (f32), over the last axis."""
    q_scale = np.asarray(q_scale, dtype=F32)
    k_scale = np.asarray(k_scale, dtype=F32)
    width = q_scale.shape[-1]
    return (F32(math.sqrt(width)) * np.max(np.abs(q_scale), -1)).astype(F32) * \
        np.max(np.abs(k_scale), -1).astype(F32)


def check_logit_bound(blocks) -> None:
    """loader.py:115-128 -- joint img/txt bound for double blocks, own bound for single blocks;
    ValueError if the worst bound reaches EXP_LIMIT."""
    double, single = blocks["double_blocks"], blocks["single_blocks"]

    def joint(name):
        return np.maximum(*(np.abs(np.asarray(double[f"{s}_attn.norm.{name}.scale"], F32))
                            for s in ("img", "txt")))

    bounds = (logit_bound(joint("query_norm"), joint("key_norm")),
              logit_bound(*(np.asarray(single[f"norm.{n}.scale"], F32)
                            for n in ("query_norm", "key_norm"))))
    worst = max(float(np.max(np.asarray(b))) for b in bounds)
    if worst >= EXP_LIMIT:
        raise ValueError(f"attention='bounded' needs logits under {EXP_LIMIT}; these weights allow "
                         f"{worst:.1f}. use attention='flash'")
