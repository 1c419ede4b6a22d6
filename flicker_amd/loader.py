"""Load-time guard of the bounded attention path (reference: src/flicker/loader.py:102-128).

``attend`` computes exp(S) without subtracting a running maximum, which is only safe
while every logit stays below EXP_LIMIT (exp(80) = 5.5e34 < float32 max).  The
QK-RMSNorm scales bound the logits (kernels.logit_bound); this check refuses weights
whose bound reaches the limit, exactly as the reference does before device_put.
"""

from __future__ import annotations

import math

import numpy as np

from .kernels import EXP_LIMIT


def _np(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().float().cpu().numpy()
    return np.asarray(x, dtype=np.float32)


def _bound(q_scale: np.ndarray, k_scale: np.ndarray) -> np.ndarray:
    width = q_scale.shape[-1]
    return (np.float32(math.sqrt(width)) * np.abs(q_scale).max(-1)).astype(np.float32) * \
        np.abs(k_scale).max(-1).astype(np.float32)


def check_logit_bound(blocks) -> None:
    """loader.py:115-128 -- ``blocks`` = {"double_blocks": {...}, "single_blocks": {...}} of
    stacked per-block norm scales.  Double blocks use the elementwise max of the image and
    text scales (text queries attend to image keys and vice versa); single blocks their own.
    Raises ValueError if the worst bound is >= EXP_LIMIT."""
    double, single = blocks["double_blocks"], blocks["single_blocks"]

    def joint(name: str) -> np.ndarray:
        img = np.abs(_np(double[f"img_attn.norm.{name}.scale"]))
        txt = np.abs(_np(double[f"txt_attn.norm.{name}.scale"]))
        return np.maximum(img, txt)

    bounds = (_bound(joint("query_norm"), joint("key_norm")),
              _bound(_np(single["norm.query_norm.scale"]), _np(single["norm.key_norm.scale"])))
    worst = max(float(np.max(b)) for b in bounds)
    if worst >= EXP_LIMIT:
        raise ValueError(f"attention='bounded' needs logits under {EXP_LIMIT}; these weights allow "
                         f"{worst:.1f}. use attention='flash'")


def sequence_margin(bound: float, length: int) -> float:
    """Headroom of the row sum l = sum_j exp(S_j) <= L * exp(bound) below float32 overflow
    (ln(FLT_MAX) = 88.72): positive means no key set of this length can overflow l."""
    return 88.72 - (bound + math.log(max(length, 1)))
