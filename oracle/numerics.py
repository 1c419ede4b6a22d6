"""bf16 rounding on float32 numpy arrays (oracle helper, test infrastructure only).

The reference stores activations in bfloat16 and rounds float32 results to it
with ``.astype(jnp.bfloat16)`` (kernels.py:45,49; nn.py:27; rope.py:29), which
is IEEE round-to-nearest-even on the upper 16 bits of the float32 pattern.
"""

import numpy as np

_ROUND_BIAS = np.uint32(0x7FFF)
_HI_MASK = np.uint32(0xFFFF0000)
_QUIET = np.uint32(0x00400000)


def bf16_round(x) -> np.ndarray:
    """float32 -> nearest bf16 value (ties to even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    shape = x.shape
    x = np.ascontiguousarray(x).reshape(-1)
    u = x.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        r = (u + _ROUND_BIAS + lsb) & _HI_MASK
    r = np.where(np.isnan(x), (u | _QUIET) & _HI_MASK, r)
    return r.view(np.float32).reshape(shape)


def bf16_bits(x) -> np.ndarray:
    """float32 values (already bf16-representable or not) -> uint16 bf16 bit patterns."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint32) << np.uint32(16)).view(np.float32)


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (2^(e-7) for normal x), as float32."""
    x = np.abs(np.asarray(x, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(x, np.float32(2.0 ** -126))))
    return np.exp2(e - 7).astype(np.float32)
