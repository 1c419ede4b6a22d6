"""SmoothQuant W8A8 for the QKV projection -- CPU restatement (test infrastructure only).

The reference has no quantisation: its QKV projection is the bf16 ``linear``
``x @ w`` (nn.py:13-14) called at modules.py:128,132,186.  The int8 path that
replaces it is defined here by an explicit formula, and the HIP kernels must
reproduce every integer and every float32 rounding of it bit for bit:

  calibration   s_j  = sqrt(max_t |X[t,j]|) / sqrt(max_o |W[j,o]|)   (alpha = 0.5;
                       s_j = 1 where either maximum is 0); inv_s_j = 1 / s_j
  weight        Wh[j,o] = f32(W[j,o]) * s_j
                w_o  = max_j |Wh[j,o]| / 127   (1 where the column is all zero)
                Wq[j,o] = clamp(rint(Wh[j,o] / w_o), -127, 127)        int8
  activation    Xh[t,j] = f32(X[t,j]) * inv_s_j
                a_t  = max_j |Xh[t,j]| / 127   (1 where the row is all zero)
                Xq[t,j] = clamp(rint(Xh[t,j] / a_t), -127, 127)        int8
  GEMM          acc[t,o] = sum_j Xq[t,j] * Wq[j,o]                        int32 exact
  rescale       Y[t,o] = bf16( (f32(acc[t,o]) * a_t) * w_o )
All float ops are single float32 operations with round-to-nearest-even
(division and sqrt correctly rounded), rint is ties-to-even.
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_round

F32 = np.float32
QMAX = 127


def smooth_factors(x_absmax, w_absmax) -> np.ndarray:
    """Per input channel j: sqrt(max|X_j|) / sqrt(max|W_j|) in f32 (1 where either is 0)."""
    xa = np.asarray(x_absmax, dtype=F32)
    wa = np.asarray(w_absmax, dtype=F32)
    ok = (xa > 0) & (wa > 0)
    s = np.where(ok, np.sqrt(np.where(ok, xa, F32(1)), dtype=F32) /
                 np.sqrt(np.where(ok, wa, F32(1)), dtype=F32), F32(1)).astype(F32)
    return s


def inverse(s) -> np.ndarray:
    """inv_s_j = 1 / s_j (f32, correctly rounded): the multiplier applied to activations."""
    return (F32(1) / np.asarray(s, dtype=F32)).astype(F32)


def _quantize(values: np.ndarray, scale: np.ndarray) -> np.ndarray:
    q = np.rint((values / scale).astype(F32))
    return np.clip(q, -QMAX, QMAX).astype(np.int8)


def _absmax_scale(amax: np.ndarray) -> np.ndarray:
    return np.where(amax > 0, (amax / F32(QMAX)).astype(F32), F32(1)).astype(F32)


def quantize_weight(w, s):
    """W (K, N) bf16-valued f32, s (K,) -> Wq (K, N) int8, w_scale (N,) f32."""
    wh = (np.asarray(w, dtype=F32) * np.asarray(s, dtype=F32)[:, None]).astype(F32)
    w_scale = _absmax_scale(np.max(np.abs(wh), axis=0))
    return _quantize(wh, w_scale[None, :]), w_scale


def quantize_act(x, inv_s):
    """X (M, K) bf16-valued f32, inv_s (K,) -> Xq (M, K) int8, a_scale (M,) f32."""
    xh = (np.asarray(x, dtype=F32) * np.asarray(inv_s, dtype=F32)[None, :]).astype(F32)
    a_scale = _absmax_scale(np.max(np.abs(xh), axis=1))
    return _quantize(xh, a_scale[:, None]), a_scale


def int_gemm(xq, wq) -> np.ndarray:
    """Exact int32 product of int8 operands.  |acc| <= K * 127^2 < 2^53, so a float64 BLAS
    matmul of the integer values is exact; the result is checked to fit in int32."""
    acc = np.asarray(xq, dtype=np.float64) @ np.asarray(wq, dtype=np.float64)
    assert np.all(np.abs(acc) < 2 ** 31)
    return acc.astype(np.int64).astype(np.int32)


def int_gemm_bruteforce(xq, wq) -> np.ndarray:
    """Independent integer loop (tiny shapes only): pins int_gemm."""
    m, k = xq.shape
    _, n = wq.shape
    out = np.zeros((m, n), dtype=np.int64)
    for i in range(m):
        for j in range(n):
            total = 0
            for t in range(k):
                total += int(xq[i, t]) * int(wq[t, j])
            out[i, j] = total
    return out.astype(np.int32)


def rescale(acc, a_scale, w_scale) -> np.ndarray:
    """Y = bf16((f32(acc) * a_t) * w_o)."""
    y = (np.asarray(acc).astype(F32) * np.asarray(a_scale, F32)[:, None]).astype(F32)
    y = (y * np.asarray(w_scale, F32)[None, :]).astype(F32)
    return bf16_round(y)


def w8a8_linear(x, inv_s, wq, w_scale):
    """Online half of the path: quantise X, exact GEMM, rescale to bf16."""
    xq, a_scale = quantize_act(x, inv_s)
    acc = int_gemm(xq, wq)
    return rescale(acc, a_scale, w_scale), acc, xq, a_scale


# --------------------------------------------------------- block input: LayerNorm + modulate
def layer_norm(x, eps: float = 1e-6) -> np.ndarray:
    """nn.py:17-21 -- bf16((x - mean) * rsqrt(var + eps)) over the last axis, with the mean and
    the variance each accumulated in f64 and rounded to f32 once (the order-free ideal of
    XLA's f32 reductions); x - mean, its square and the product are single f32 operations and
    rsqrt is 1/sqrt in f32, as for rms_norm (path.py)."""
    xf = np.asarray(x, dtype=F32)
    mean = np.mean(xf.astype(np.float64), axis=-1, keepdims=True).astype(F32)
    d = (xf - mean).astype(F32)
    sq = (d * d).astype(F32)
    var = np.mean(sq.astype(np.float64), axis=-1, keepdims=True).astype(F32)
    inv = F32(1.0) / np.sqrt(var + F32(eps), dtype=F32)
    return bf16_round((d * inv).astype(F32))


def modulate(x, shift, scale) -> np.ndarray:
    """modules.py:38-40 with norm=True -- (1 + scale) * layer_norm(x) + shift in bf16: each
    of the three bf16 operations rounds its f32 result to bf16.  x (B, L, K); shift, scale
    (B, K) (the reference's (B, 1, K) modulation rows)."""
    base = layer_norm(x)
    shift = np.asarray(shift, dtype=F32)[:, None, :]
    scale = np.asarray(scale, dtype=F32)[:, None, :]
    one_plus = bf16_round((F32(1.0) + scale).astype(F32))
    return bf16_round((bf16_round((one_plus * base).astype(F32)) + shift).astype(F32))
