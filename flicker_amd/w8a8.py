"""SmoothQuant W8A8 replacement of the bf16 QKV projection.

The reference projects with ``linear(x, w) = x @ w`` in bf16 (src/flicker/nn.py:13-14)
at the QKV projections of src/flicker/modules.py:128,132 (double blocks, img/txt) and
:186 (single blocks, the qkv part of linear1).  It has no quantisation; this module
defines the int8 replacement by an explicit formula (reproduced bit for bit by the HIP
kernels of libflicker_hip.so, see include/flicker_hip.h):

  offline   s_j = sqrt(max_t|X[t,j]|) / sqrt(max_o|W[j,o]|), inv_s_j = 1/s_j  (calibration)
            Wq = clamp(rint(W*s / w_o), +-127), w_o = max_j|W[j,o]*s_j| / 127   (per channel)
  online    Xq = clamp(rint(X*inv_s / a_t), +-127), a_t = max_j|X[t,j]*inv_s_j| / 127
            Y = bf16((f32(Xq . Wq) * a_t) * w_o)                                 (int32 GEMM)

Typical use::

    stats = absmax_cols(x_calib)                    # per input channel, over tokens
    qw = quantize_linear(w, stats)                  # once per weight
    y = linear(x, qw)                               # per forward: (..., K) -> (..., N) bf16
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib
from .kernels import _on_gpu


class QuantizedLinear(NamedTuple):
    """An int8 projection weight: ``wq_t`` (N, K) int8 is Wq transposed (k-contiguous
    rows), ``w_scale`` (N,) f32 the per-channel scales, ``smooth`` / ``inv_smooth`` (K,)
    f32 the SmoothQuant factors s and 1/s."""

    wq_t: torch.Tensor
    w_scale: torch.Tensor
    smooth: torch.Tensor
    inv_smooth: torch.Tensor

    @property
    def in_features(self) -> int:
        return self.wq_t.shape[1]

    @property
    def out_features(self) -> int:
        return self.wq_t.shape[0]


def _rows(name: str, t: torch.Tensor) -> torch.Tensor:
    """A 2-D bf16 view with a contiguous last axis and 16-byte aligned rows."""
    _on_gpu(name, t)
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    if t.dim() != 2:
        t = t.reshape(-1, t.shape[-1])
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _f32(name: str, t: torch.Tensor, n: int, device) -> torch.Tensor:
    _on_gpu(name, t)
    if t.shape != (n,):
        raise ValueError(f"{name} must have shape ({n},), got {tuple(t.shape)}")
    return t.to(device=device, dtype=torch.float32).contiguous()


def absmax_rows(w: torch.Tensor) -> torch.Tensor:
    """Per-row max |w| of a bf16 (K, N) weight: the max_o |W[j,o]| of the smoothing factor."""
    w = _rows("w", w)
    out = torch.empty(w.shape[0], dtype=torch.float32, device=w.device)
    _lib.run("flk_absmax_rows", (w, out), w.data_ptr(), w.shape[0], w.shape[1], w.stride(0), out.data_ptr(),
             _lib.stream_of(w))
    return out


def absmax_cols(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-channel max |x| over all tokens of a bf16 (..., K) activation.  With ``out``, the
    result is folded into it (running maximum over calibration batches)."""
    x = _rows("x", x)
    k = x.shape[1]
    accumulate = out is not None
    if out is None:
        out = torch.empty(k, dtype=torch.float32, device=x.device)
    elif out.shape != (k,) or out.dtype != torch.float32 or not out.is_contiguous() or out.device != x.device:
        raise ValueError(f"out must be a contiguous float32 ({k},) tensor on {x.device}")
    _lib.run("flk_absmax_cols", (x, out), x.data_ptr(), x.shape[0], k, x.stride(0), int(accumulate),
             out.data_ptr(), _lib.stream_of(x))
    return out


def smooth_factors(x_absmax: torch.Tensor, w_absmax: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(s, 1/s) with s_j = sqrt(x_absmax_j) / sqrt(w_absmax_j) (1 where either is 0)."""
    k = x_absmax.shape[0]
    xa = _f32("x_absmax", x_absmax, k, x_absmax.device)
    wa = _f32("w_absmax", w_absmax, k, xa.device)
    s = torch.empty_like(xa)
    inv = torch.empty_like(xa)
    _lib.run("flk_smooth_factors", (xa, wa, s, inv), xa.data_ptr(), wa.data_ptr(), k, s.data_ptr(),
             inv.data_ptr(), _lib.stream_of(xa))
    return s, inv


def quantize_weight(w: torch.Tensor, smooth: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (K, N) weight and smoothing factors -> (wq_t (N, K) int8, w_scale (N,) f32)."""
    w = _rows("w", w)
    k, n = w.shape
    s = _f32("smooth", smooth, k, w.device)
    wq_t = torch.empty((n, k), dtype=torch.int8, device=w.device)
    w_scale = torch.empty(n, dtype=torch.float32, device=w.device)
    _lib.run("flk_quantize_weight", (w, s, wq_t, w_scale), w.data_ptr(), w.stride(0), s.data_ptr(), k, n,
             wq_t.data_ptr(), w_scale.data_ptr(), _lib.stream_of(w))
    return wq_t, w_scale


def quantize_linear(w: torch.Tensor, x_absmax: torch.Tensor) -> QuantizedLinear:
    """Offline half: smoothing factors from calibration statistics, then the int8 weight."""
    s, inv = smooth_factors(x_absmax, absmax_rows(w))
    wq_t, w_scale = quantize_weight(w, s)
    return QuantizedLinear(wq_t, w_scale, s, inv)


def quantize_act(x: torch.Tensor, inv_smooth: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (..., K) activation -> (xq (M, K) int8, a_scale (M,) f32), M = prod(leading dims)."""
    x = _rows("x", x)
    m, k = x.shape
    inv = _f32("inv_smooth", inv_smooth, k, x.device)
    xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
    a_scale = torch.empty(m, dtype=torch.float32, device=x.device)
    _lib.run("flk_quantize_act", (x, inv, xq, a_scale), x.data_ptr(), x.stride(0), inv.data_ptr(), m, k,
             xq.data_ptr(), a_scale.data_ptr(), _lib.stream_of(x))
    return xq, a_scale


def quantize_act_modulated(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, inv_smooth: torch.Tensor,
                           *, x_mod: torch.Tensor | bool | None = None):
    """int8 activation of the modulated block input in one pass: X = modulate(x, shift, scale)
    (modules.py:38-40: (1 + scale) * layer_norm(x) + shift, bf16) then quantize_act(X).

    x (B, L, K) bf16 block input; shift, scale (B, K) bf16 modulation rows (the reference's
    (B, 1, K) ``ModTriple`` entries).  Returns (xq (B*L, K) int8, a_scale (B*L,) f32), plus X
    (B, L, K) bf16 when ``x_mod`` is True or a tensor to write it into."""
    xr, shift, scale, inv, xq, a_scale, out = _modulated_operands(x, shift, scale, inv_smooth, x_mod)
    batch, length, k = x.shape
    _lib.run("flk_quantize_act_modulated", (xr, shift, scale, inv, xq, a_scale, out),
             xr.data_ptr(), xr.stride(0), shift.data_ptr(), scale.data_ptr(), shift.stride(0), length,
             inv.data_ptr(), batch * length, k, xq.data_ptr(), a_scale.data_ptr(), _lib.ptr(out), k,
             _lib.stream_of(x))
    return (xq, a_scale) if out is None else (xq, a_scale, out)


def quantize_act_modulated_pair(x0, shift0, scale0, inv_smooth0, x1, shift1, scale1, inv_smooth1):
    """A double block's two modulated activations (text and image, each with its own
    modulation rows and smoothing factors, same width) in one launch.  Returns
    ((xq0, a_scale0), (xq1, a_scale1)), each exactly quantize_act_modulated of its stream."""
    o0 = _modulated_operands(x0, shift0, scale0, inv_smooth0, None)
    o1 = _modulated_operands(x1, shift1, scale1, inv_smooth1, None)
    if x0.shape[2] != x1.shape[2]:
        raise ValueError(f"both activations must have one width, got {x0.shape[2]} and {x1.shape[2]}")
    _lib.run("flk_quantize_act_modulated_pair", (*o0[:6], *o1[:6]),
             *_modulated_args(x0, *o0), *_modulated_args(x1, *o1), x0.shape[2], _lib.stream_of(x0))
    return (o0[4], o0[5]), (o1[4], o1[5])


def _modulated_args(x, xr, shift, scale, inv, xq, a_scale, out):
    """One stream's arguments of flk_quantize_act_modulated_pair (x .. x_mod_row_stride)."""
    batch, length, k = x.shape
    return (xr.data_ptr(), xr.stride(0), shift.data_ptr(), scale.data_ptr(), shift.stride(0), length,
            inv.data_ptr(), batch * length, xq.data_ptr(), a_scale.data_ptr(), _lib.ptr(out), k)


def _modulated_operands(x, shift, scale, inv_smooth, x_mod):
    """Checked device operands of one modulated activation: (x rows, shift, scale, 1/s, xq,
    a_scale, X or None)."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, K), got {tuple(x.shape)}")
    batch, length, k = x.shape
    shift = shift.reshape(batch, k) if shift.dim() == 3 else shift
    scale = scale.reshape(batch, k) if scale.dim() == 3 else scale
    for name, t in (("shift", shift), ("scale", scale)):
        _on_gpu(name, t)
        if t.dtype != torch.bfloat16 or t.shape != (batch, k):
            raise ValueError(f"{name} must be bfloat16 ({batch}, {k}) (or ({batch}, 1, {k}))")
    shift, scale = shift.contiguous(), scale.contiguous()
    xr = _rows("x", x)
    inv = _f32("inv_smooth", inv_smooth, k, x.device)
    m = batch * length
    xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
    a_scale = torch.empty(m, dtype=torch.float32, device=x.device)
    out = None
    if x_mod is True:
        out = torch.empty((batch, length, k), dtype=torch.bfloat16, device=x.device)
    elif isinstance(x_mod, torch.Tensor):
        out = x_mod
        if out.shape != (batch, length, k) or out.dtype != torch.bfloat16 or not out.is_contiguous():
            raise ValueError(f"x_mod must be a contiguous bfloat16 ({batch}, {length}, {k}) tensor")
    return xr, shift, scale, inv, xq, a_scale, out


def gemm(xq: torch.Tensor, a_scale: torch.Tensor, wq_t: torch.Tensor, w_scale: torch.Tensor, *,
         out: torch.Tensor | None = None, acc: torch.Tensor | None = None) -> torch.Tensor:
    """Y (M, N) bf16 = bf16((f32(xq . wq_t^T) * a_scale) * w_scale).  ``out`` may be a row-strided
    (M, N) view (e.g. the qkv columns of a wider buffer); ``acc`` (M, N) int32 receives the
    exact integer products when given."""
    for name, t in (("xq", xq), ("wq_t", wq_t)):
        _on_gpu(name, t)
        if t.dtype != torch.int8 or t.dim() != 2 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous 2-D int8 tensor")
    m, k = xq.shape
    n = wq_t.shape[0]
    if wq_t.shape[1] != k:
        raise ValueError(f"xq has {k} input channels but wq_t has {wq_t.shape[1]}")
    a = _f32("a_scale", a_scale, m, xq.device)
    ws = _f32("w_scale", w_scale, n, xq.device)
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=xq.device)
    elif out.shape != (m, n) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"out must be a bfloat16 ({m}, {n}) view with contiguous rows")
    if acc is not None and (acc.shape != (m, n) or acc.dtype != torch.int32 or not acc.is_contiguous()):
        raise ValueError(f"acc must be a contiguous int32 ({m}, {n}) tensor")
    _lib.run("flk_w8a8_gemm", (xq, wq_t, a, ws, out, acc), xq.data_ptr(), wq_t.data_ptr(), a.data_ptr(),
             ws.data_ptr(), m, k, n, out.data_ptr(), out.stride(0), _lib.ptr(acc), _lib.stream_of(xq))
    return out


def linear(x: torch.Tensor, qw: QuantizedLinear, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """int8 stand-in for ``linear(x, w)`` (nn.py:13-14): (..., K) bf16 -> (..., N) bf16."""
    lead = x.shape[:-1]
    xq, a_scale = quantize_act(x, qw.inv_smooth)
    y = gemm(xq, a_scale, qw.wq_t, qw.w_scale, out=None if out is None else out.view(-1, qw.out_features))
    return y.reshape(*lead, qw.out_features) if out is None else out


def _qk_stream(x, qw: QuantizedLinear, q_scale, k_scale, freqs, num_heads: int, modulation, quantized=None):
    """Checks and device operands of one fused projection + qk_prep stream: (xq, a_scale, cos,
    sin, q_scale, k_scale, q_gain), the activation quantised (modulated first when given)
    unless ``quantized`` already holds its (xq, a_scale)."""
    from .kernels import HEAD_DIM, Freqs, PositionIds

    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, K), got {tuple(x.shape)}")
    if isinstance(freqs, PositionIds):
        # The fused epilogue reads lane tables; build them from the ids with the same
        # arithmetic the in-kernel form uses, so the values are identical.
        from .rope import rope_lanes
        freqs = rope_lanes(freqs.ids, freqs.q_gain, freqs.axes_dim, freqs.theta)
    length = x.shape[1]
    if qw.out_features != 3 * num_heads * HEAD_DIM:
        raise ValueError(f"projection has {qw.out_features} outputs, not 3 * {num_heads} * {HEAD_DIM}")
    cos, sin, q_gain = Freqs(*freqs)
    for name, t in (("freqs.cos", cos), ("freqs.sin", sin), ("q_scale", q_scale), ("k_scale", k_scale)):
        _on_gpu(name, t)
    if cos.shape != (length, HEAD_DIM) or sin.shape != (length, HEAD_DIM) or cos.dtype != torch.float32 \
            or sin.dtype != torch.float32:
        raise ValueError(f"freqs tables must be float32 ({length}, {HEAD_DIM})")
    cos, sin = cos.contiguous(), sin.contiguous()
    if q_scale.dtype != k_scale.dtype or q_scale.dtype not in (torch.bfloat16, torch.float32) \
            or q_scale.numel() != HEAD_DIM or k_scale.numel() != HEAD_DIM:
        raise ValueError(f"q_scale / k_scale must be {HEAD_DIM} bfloat16 or float32 values of one dtype")
    q_scale, k_scale = q_scale.reshape(-1).contiguous(), k_scale.reshape(-1).contiguous()
    if quantized is not None:
        xq, a_scale = quantized
    elif modulation is None:
        xq, a_scale = quantize_act(x, qw.inv_smooth)
    else:
        xq, a_scale = quantize_act_modulated(x, modulation[0], modulation[1], qw.inv_smooth)
    return xq, a_scale, cos, sin, q_scale, k_scale, float(q_gain)


def qk_prep(x: torch.Tensor, qw: QuantizedLinear, q_scale: torch.Tensor, k_scale: torch.Tensor, freqs,
            num_heads: int, *, out=None, out_offset: int = 0, modulation=None):
    """``kernels.qk_prep(linear(x, qw), q_scale, k_scale, freqs, num_heads)`` in two launches
    instead of three: the activation quantisation, then one int8 GEMM whose epilogue applies
    QK-RMSNorm + RoPE (+ q_gain) to each finished head row and writes head-major q, k, v
    (kernels.py:57-91 after nn.py:13-14); the projected activation never reaches memory.
    Bit-identical to the unfused pair.  x (B, L, K) bf16 -> q, k, v (B, H, L, 128) bf16.

    With ``modulation=(shift, scale)`` x is the raw block input and the projection input is
    modulate(x, shift, scale) (modules.py:38-40), computed inside the activation quantisation:
    the whole ``qkv_prep(linear(modulate(x, mod1), w), ...)`` of a block (modules.py:128-133,
    186-190) is then two launches."""
    from .kernels import HEAD_DIM

    s = _qk_stream(x, qw, q_scale, k_scale, freqs, num_heads, modulation)
    batch, length, k = x.shape
    xq, a_scale, cos, sin, q_scale, k_scale, q_gain = s
    if out is None:
        if out_offset:
            raise ValueError("out_offset needs out=(q, k, v)")
        out = tuple(torch.empty((batch, num_heads, length, HEAD_DIM), dtype=torch.bfloat16, device=x.device)
                    for _ in range(3))
        out_length = length
    else:
        out = tuple(out)
        out_length = out[0].shape[2]
        for t in out:
            if (t.dtype != torch.bfloat16 or t.shape != (batch, num_heads, out_length, HEAD_DIM)
                    or not t.is_contiguous()):
                raise ValueError("out tensors must be contiguous bf16 (B, H, L_out, D) of one shape")
        if out_offset < 0 or out_offset + length > out_length:
            raise ValueError(f"out_offset {out_offset} + L {length} exceeds the output length {out_length}")
    _lib.run("flk_w8a8_qk_prep", (xq, qw.wq_t, a_scale, qw.w_scale, cos, sin, q_scale, k_scale, *out),
             xq.data_ptr(), qw.wq_t.data_ptr(), a_scale.data_ptr(), qw.w_scale.data_ptr(), k, cos.data_ptr(),
             sin.data_ptr(), cos.stride(0), q_scale.data_ptr(), k_scale.data_ptr(),
             int(q_scale.dtype == torch.float32), float(q_gain), batch, length, num_heads, HEAD_DIM,
             out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), out_length, out_offset, _lib.stream_of(x))
    return out


def qk_prep_pair(txt, img, num_heads: int, *, out=None, modulation=None):
    """A double block's two projections with their qk prep (modules.py:127-135: txt_attn.qkv
    and img_attn.qkv, each followed by qkv_prep) plus the text|image concatenations
    (modules.py:136-139), in one fused launch after one activation quantisation per stream.
    The text projection's 512 tokens run on the CUs the image projection leaves idle in its
    last round.

    ``txt`` and ``img`` are (x, qw, q_scale, k_scale, freqs): each stream's (B, L_i, K) input,
    quantised weight, norm scales and RoPE lanes of its own rows.  ``modulation`` is
    optionally ((shift_txt, scale_txt), (shift_img, scale_img)).  Returns the joint q, k, v
    (B, H, L_txt + L_img, 128), text first (or writes ``out``); each stream's rows are
    bit-identical to ``qk_prep`` of that stream alone."""
    from .kernels import HEAD_DIM

    if modulation is not None and modulation[0] is not None and modulation[1] is not None:
        (m0, m1) = modulation
        q0, q1 = quantize_act_modulated_pair(txt[0], m0[0], m0[1], txt[1].inv_smooth,
                                             img[0], m1[0], m1[1], img[1].inv_smooth)
        s0 = _qk_stream(*txt, num_heads, None, quantized=q0)
        s1 = _qk_stream(*img, num_heads, None, quantized=q1)
    else:
        mods = modulation if modulation is not None else (None, None)
        s0 = _qk_stream(*txt, num_heads, mods[0])
        s1 = _qk_stream(*img, num_heads, mods[1])
    x0, x1 = txt[0], img[0]
    if x0.shape[0] != x1.shape[0] or x0.shape[2] != x1.shape[2]:
        raise ValueError(f"text and image inputs must share batch and width, got {tuple(x0.shape)} "
                         f"and {tuple(x1.shape)}")
    if s0[6] != s1[6]:
        raise ValueError(f"both streams must share q_gain, got {s0[6]} and {s1[6]}")
    if s0[4].dtype != s1[4].dtype:
        raise ValueError("both streams' norm scales must share one dtype")
    batch, len0, k = x0.shape
    len1 = x1.shape[1]
    if out is None:
        out = tuple(torch.empty((batch, num_heads, len0 + len1, HEAD_DIM), dtype=torch.bfloat16,
                                device=x0.device) for _ in range(3))
    else:
        out = tuple(out)
        for t in out:
            if (t.dtype != torch.bfloat16 or t.shape != (batch, num_heads, len0 + len1, HEAD_DIM)
                    or not t.is_contiguous()):
                raise ValueError(f"out tensors must be contiguous bf16 ({batch}, {num_heads}, "
                                 f"{len0 + len1}, {HEAD_DIM})")

    def stream_args(st, qw, length, offset):
        xq, a_scale, cos, sin, q_scale, k_scale, _ = st
        return (xq.data_ptr(), qw.wq_t.data_ptr(), a_scale.data_ptr(), qw.w_scale.data_ptr(), cos.data_ptr(),
                sin.data_ptr(), q_scale.data_ptr(), k_scale.data_ptr(), length, offset)

    operands = (s0[0], txt[1].wq_t, s0[1], txt[1].w_scale, *s0[2:6],
                s1[0], img[1].wq_t, s1[1], img[1].w_scale, *s1[2:6], *out)
    _lib.run("flk_w8a8_qk_prep_pair", operands,
             *stream_args(s0, txt[1], len0, 0), *stream_args(s1, img[1], len1, len0),
             k, HEAD_DIM, int(s0[4].dtype == torch.float32), s0[6], batch, num_heads, HEAD_DIM,
             out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), len0 + len1, _lib.stream_of(x0))
    return out
