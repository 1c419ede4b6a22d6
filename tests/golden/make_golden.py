"""Generate the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference (kelechi-c/flicker) ships no tests, golden vectors or fixtures for this
path, and its JAX code cannot run here.  These fixtures are therefore computed by an
independent brute force written from the reference's formulas -- element-by-element
Python loops over Python floats, with float32 and bf16 rounding done arithmetically
(frexp + ties-to-even ``round``) rather than by the bit tricks the oracle uses -- so
that they pin the oracle (tests/test_golden.py) and, through it, the HIP kernels:

  rope.npz   embed_nd + lane_pair tables (rope.py:9-21, kernels.py:28-31)
  qk.npz     fused qk_prep, gain 1 and gain 1/sqrt(128) (kernels.py:35-53)
  attn.npz   plain sdpa (nn.py:35-44) and bounded attention (kernels.py:113-130)
  w8a8.npz   SmoothQuant W8A8 quantise / int32 GEMM / rescale (formula in oracle/w8a8.py)

Inputs are seeded; bf16 tensors are stored as uint16 bit patterns.
"""

from __future__ import annotations

import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


# ----------------------------------------------------------------------------- rounding
def round_bits(x: float, bits: int) -> float:
    """Nearest float with `bits` significant bits, ties to even (normal range only)."""
    if x == 0.0 or math.isinf(x) or math.isnan(x):
        return x
    m, e = math.frexp(x)            # x = m * 2^e, 0.5 <= |m| < 1
    q = round(m * (1 << bits))      # Python round(): ties to even
    return math.ldexp(q, e - bits)


def f32(x: float) -> float:
    return round_bits(x, 24)


def bf16(x: float) -> float:
    return round_bits(x, 8)


def bits16(values) -> np.ndarray:
    """bf16-representable floats -> uint16 patterns."""
    a = np.asarray(values, dtype=np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def from16(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- RoPE
AXES = (32, 32, 32, 32)
THETA = 2000.0


def omega(k: int, dim: int) -> float:
    scale = f32(float(2 * k) / float(dim))
    return f32(1.0 / f32(float(np.float32(THETA) ** np.float32(scale))))


def rope_tables(ids):
    """-> pe (L, 64, 2, 2), cos2 / sin2 (L, 128)."""
    length = len(ids)
    pe = np.zeros((length, 64, 2, 2), dtype=np.float64)
    cos2 = np.zeros((length, 128))
    sin2 = np.zeros((length, 128))
    for t in range(length):
        pair = 0
        for a, dim in enumerate(AXES):
            for k in range(dim // 2):
                ang = f32(float(ids[t][a]) * omega(k, dim))
                c, s = f32(math.cos(ang)), f32(math.sin(ang))
                pe[t, pair] = [[c, -s], [s, c]]
                cos2[t, 2 * pair] = cos2[t, 2 * pair + 1] = c
                sin2[t, 2 * pair], sin2[t, 2 * pair + 1] = -s, s
                pair += 1
    return pe, cos2, sin2


def make_rope(rng):
    ids = [[0, 0, 0, 0], [0, 0, 0, 7], [0, 0, 0, 511], [0, 3, 5, 0], [0, 63, 0, 0],
           [0, 0, 127, 0], [0, 12, 34, 0], [2, 1, 1, 9]]
    pe, cos2, sin2 = rope_tables(ids)
    np.savez(os.path.join(HERE, "rope.npz"), ids=np.asarray(ids, np.float32),
             pe=pe.astype(np.float32), cos=cos2.astype(np.float32), sin=sin2.astype(np.float32))


# ----------------------------------------------------------------------------- qk_prep
def qk_prep_bruteforce(qkv, qs, ks, cos2, sin2, heads, gain):
    """qkv (B, L, 3*H*D) floats -> q, k, v (B, H, L, D) floats, per kernels.py:35-53."""
    batch, length, width = qkv.shape
    dim = width // (3 * heads)
    out = np.zeros((3, batch, heads, length, dim))
    for b in range(batch):
        for t in range(length):
            for h in range(heads):
                for sec, scale, gn in ((0, qs, gain), (1, ks, 1.0)):
                    x = [float(qkv[b, t, (sec * heads + h) * dim + d]) for d in range(dim)]
                    ms = f32(math.fsum(v * v for v in x) / dim)          # exact mean, one rounding
                    inv = f32(1.0 / f32(math.sqrt(f32(ms + f32(1e-6)))))
                    y = [bf16(f32(bf16(f32(x[d] * inv)) * float(scale[d]))) for d in range(dim)]
                    for d in range(dim):
                        partner = d + 1 if d % 2 == 0 else d - 1
                        r = f32(f32(cos2[t, d] * y[d]) + f32(sin2[t, d] * y[partner]))
                        if gn != 1.0:
                            r = f32(f32(gn) * r)
                        out[sec, b, h, t, d] = bf16(r)
                for d in range(dim):
                    out[2, b, h, t, d] = float(qkv[b, t, (2 * heads + h) * dim + d])
    return out


def make_qk(rng):
    heads, length, dim = 2, 3, 128
    qkv = [bf16(float(v)) for v in rng.standard_normal(length * 3 * heads * dim)]
    qkv = np.asarray(qkv).reshape(1, length, 3 * heads * dim)
    qkv[0, 1, dim:2 * dim] = 0.0                     # one all-zero query head row
    qkv[0, 2, 3 * dim:4 * dim] *= 40.0                # one large-magnitude key head row
    qkv = np.vectorize(bf16)(qkv)
    qs = np.asarray([bf16(1.0 + 0.05 * float(v)) for v in rng.standard_normal(dim)])
    ks = np.asarray([bf16(1.0 + 0.05 * float(v)) for v in rng.standard_normal(dim)])
    ids = [[0, 0, 0, 5], [0, 7, 9, 0], [0, 0, 0, 300]]
    _, cos2, sin2 = rope_tables(ids)
    gain = 1.0 / math.sqrt(128)
    o1 = qk_prep_bruteforce(qkv, qs, ks, cos2, sin2, heads, 1.0)
    og = qk_prep_bruteforce(qkv, qs, ks, cos2, sin2, heads, gain)
    np.savez(os.path.join(HERE, "qk.npz"), qkv=bits16(qkv), q_scale=bits16(qs), k_scale=bits16(ks),
             ids=np.asarray(ids, np.float32), heads=heads, gain=gain,
             q1=bits16(o1[0]), k1=bits16(o1[1]), v1=bits16(o1[2]),
             qg=bits16(og[0]), kg=bits16(og[1]), vg=bits16(og[2]))


# ----------------------------------------------------------------------------- attention
def sdpa_exact(q, k, v):
    """Mathematical softmax attention (f64 throughout), scaled by 1/sqrt(D)."""
    heads, length, dim = q.shape
    out = np.zeros_like(q, dtype=np.float64)
    scale = 1.0 / math.sqrt(dim)
    for h in range(heads):
        for i in range(length):
            logits = [math.fsum(q[h, i, d] * k[h, j, d] for d in range(dim)) * scale for j in range(length)]
            top = max(logits)
            w = [math.exp(s - top) for s in logits]
            z = math.fsum(w)
            for d in range(dim):
                out[h, i, d] = math.fsum(w[j] * v[h, j, d] for j in range(length)) / z
    return out


def bounded_exact(q, k, v):
    """kernels.py:113-130 in exact arithmetic except its own rounding points:
    S = q.k (no scale, q is pre-scaled), P = bf16(f32(exp S)), o = sum P v / sum P."""
    heads, length, dim = q.shape
    out = np.zeros_like(q, dtype=np.float64)
    for h in range(heads):
        for i in range(length):
            p = [bf16(f32(math.exp(f32(math.fsum(q[h, i, d] * k[h, j, d] for d in range(dim))))))
                 for j in range(length)]
            z = math.fsum(p)
            for d in range(dim):
                out[h, i, d] = math.fsum(p[j] * v[h, j, d] for j in range(length)) / z
    return out


def make_attn(rng):
    heads, length, dim = 2, 24, 128
    x = rng.standard_normal((3, heads, length, dim))
    x[:2] /= np.sqrt((x[:2] ** 2).mean(-1, keepdims=True))          # unit-RMS q, k rows
    q_plain = np.vectorize(bf16)(x[0])
    k = np.vectorize(bf16)(x[1] * 1.3)
    v = np.vectorize(bf16)(rng.standard_normal((heads, length, dim)))
    q_pre = np.vectorize(bf16)(x[0] / math.sqrt(dim))
    np.savez(os.path.join(HERE, "attn.npz"), q_plain=bits16(q_plain), q_pre=bits16(q_pre), k=bits16(k),
             v=bits16(v), sdpa=sdpa_exact(q_plain, k, v).astype(np.float32),
             bounded=bounded_exact(q_pre, k, v).astype(np.float32))


# ----------------------------------------------------------------------------- W8A8
def quant(values, scale):
    r = round(f32(values / scale))                  # ties to even
    return int(max(-127, min(127, r)))


def make_w8a8(rng):
    m, kdim, n = 5, 16, 6
    x = rng.standard_normal((m, kdim))
    x[:, 3] *= 20.0                                  # outlier channel
    x[4] = 0.0                                       # all-zero token
    x = np.vectorize(bf16)(x)
    w = np.vectorize(bf16)(0.02 * rng.standard_normal((kdim, n)))
    xa = [max(abs(x[t, j]) for t in range(m)) for j in range(kdim)]
    wa = [max(abs(w[j, o]) for o in range(n)) for j in range(kdim)]
    s = [f32(f32(math.sqrt(xa[j])) / f32(math.sqrt(wa[j]))) if xa[j] > 0 and wa[j] > 0 else 1.0
         for j in range(kdim)]
    inv_s = [f32(1.0 / sj) for sj in s]
    wh = [[f32(w[j, o] * s[j]) for o in range(n)] for j in range(kdim)]
    w_scale = []
    for o in range(n):
        amax = max(abs(wh[j][o]) for j in range(kdim))
        w_scale.append(f32(amax / 127.0) if amax > 0 else 1.0)
    wq = [[quant(wh[j][o], w_scale[o]) for o in range(n)] for j in range(kdim)]
    a_scale, xq = [], []
    for t in range(m):
        xh = [f32(x[t, j] * inv_s[j]) for j in range(kdim)]
        amax = max(abs(v) for v in xh)
        a = f32(amax / 127.0) if amax > 0 else 1.0
        a_scale.append(a)
        xq.append([quant(v, a) for v in xh])
    acc = [[sum(xq[t][j] * wq[j][o] for j in range(kdim)) for o in range(n)] for t in range(m)]
    y = [[bf16(f32(f32(float(acc[t][o]) * a_scale[t]) * w_scale[o])) for o in range(n)] for t in range(m)]
    np.savez(os.path.join(HERE, "w8a8.npz"), x=bits16(x), w=bits16(w), smooth=np.asarray(s, np.float32),
             inv_smooth=np.asarray(inv_s, np.float32), wq=np.asarray(wq, np.int8),
             w_scale=np.asarray(w_scale, np.float32), xq=np.asarray(xq, np.int8),
             a_scale=np.asarray(a_scale, np.float32), acc=np.asarray(acc, np.int32), y=bits16(y))


def main():
    rng = np.random.default_rng(20261201)
    make_rope(rng)
    make_qk(rng)
    make_attn(rng)
    make_w8a8(rng)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
