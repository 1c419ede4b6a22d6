"""Seeded synthetic inputs for one Klein DiT attention op (no checkpoints or datasets).

A workload is one joint text|image sequence: ``num_txt`` text tokens followed by an
h x w grid of 2x2-patched latents (pipeline.py:27-28 of the reference), 24 heads of
128.  Inputs are generated on the CPU with torch.Generator (so every device sees the
same values) and then moved:

  qkv      (B, L, 9216) bf16 ~ N(0, 1)                              seed 0
  q_scale  (128,) bf16 = 1 + 0.05 N(0, 1)                             seed 1
  k_scale  (128,) bf16 = 1 + 0.05 N(0, 1)                             seed 2
  stress   a seeded 5% of the 9216 channels scaled by 8 (batch-4 case) seed 5
  ids      text (0, 0, 0, i) then image (0, row, col, 0)  (rope.py:33-45)

The int8 QKV projection workload (``Projection``) is X (M, 3072) bf16 ~ N(0, 1) with a
seeded 1% of the input channels scaled by 20 (activation outliers, the case SmoothQuant
targets; seeds 3 and 5) and W (3072, 9216) bf16 ~ N(0, 0.02) (seed 4).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from .config import Klein4B
from .rope import sequence_ids

KLEIN = Klein4B()


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    num_txt: int
    height: int
    width: int
    stress_fraction: float = 0.0   # fraction of QKV channels multiplied by 8
    num_heads: int = KLEIN.num_heads
    head_dim: int = KLEIN.head_dim

    @property
    def length(self) -> int:
        return self.num_txt + self.height * self.width

    @property
    def qkv_width(self) -> int:
        return 3 * self.num_heads * self.head_dim

    def qk_prep_bytes(self, tables: bool = True) -> int:
        """Algorithmic HBM bytes of one qk_prep: read QKV + write Q, K, V (bf16), the two bf16
        scale vectors, and either the float32 cos/sin tables (read once) or, for the variant
        that computes the lanes from position ids, the (L, 4) float32 ids."""
        act = self.batch * self.length * self.qkv_width * 2
        rope = 2 * self.length * self.head_dim * 4 if tables else self.length * 4 * 4
        return 2 * act + rope + 2 * self.head_dim * 2

    def attend_flops(self) -> int:
        """4 B H L^2 D: the QK^T and PV products of non-causal attention (exp and sums not counted)."""
        return 4 * self.batch * self.num_heads * self.length ** 2 * self.head_dim


WORKLOADS = {
    w.name: w
    for w in (
        Workload("klein_512", 1, 512, 32, 32),
        Workload("klein_1024", 1, 512, 64, 64),
        Workload("klein_1024_b4", 4, 512, 64, 64, stress_fraction=0.05),
        Workload("klein_2048", 1, 512, 128, 128),
        Workload("klein_1536x640", 1, 512, 96, 40),
    )
}


@dataclass(frozen=True)
class Projection:
    """One QKV projection: (tokens, hidden) x (hidden, 3 H D)."""

    name: str
    tokens: int
    hidden: int = KLEIN.hidden_size
    out_features: int = 3 * KLEIN.num_heads * KLEIN.head_dim
    outlier_fraction: float = 0.01
    outlier_gain: float = 20.0

    def gemm_bytes(self) -> int:
        """Algorithmic HBM bytes of one int8 GEMM: Xq (M, K) and WqT (N, K) int8 read once,
        Y (M, N) bf16 written (scales negligible)."""
        return self.tokens * self.hidden + self.hidden * self.out_features + 2 * self.tokens * self.out_features

    def gemm_ops(self) -> int:
        """2 M K N integer multiply-adds counted as two ops each."""
        return 2 * self.tokens * self.hidden * self.out_features


PROJECTIONS = {p.name: p for p in (Projection("qkv_1024", 4608), Projection("qkv_512", 1536))}


def _gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(seed)


def make_qkv(w: Workload, seed: int = 0) -> torch.Tensor:
    """(B, L, 3*H*D) bf16 ~ N(0,1) on the CPU, with the stress channels applied."""
    qkv = torch.randn((w.batch, w.length, w.qkv_width), generator=_gen(seed), dtype=torch.float32)
    if w.stress_fraction:
        count = int(round(w.stress_fraction * w.qkv_width))
        picks = torch.randperm(w.qkv_width, generator=_gen(5))[:count]
        qkv[..., picks] *= 8.0
    return qkv.to(torch.bfloat16)


def make_scales(w: Workload) -> tuple[torch.Tensor, torch.Tensor]:
    q_scale = (1.0 + 0.05 * torch.randn(w.head_dim, generator=_gen(1))).to(torch.bfloat16)
    k_scale = (1.0 + 0.05 * torch.randn(w.head_dim, generator=_gen(2))).to(torch.bfloat16)
    return q_scale, k_scale


def make_ids(w: Workload) -> np.ndarray:
    return sequence_ids(w.num_txt, w.height, w.width)


def q_gain(w: Workload) -> float:
    """dit.py:36 -- the bounded path pre-scales queries by 1/sqrt(head_dim)."""
    return 1.0 / math.sqrt(w.head_dim)


def make_projection(p: Projection) -> tuple[torch.Tensor, torch.Tensor]:
    """(X (M, K), W (K, N)) bf16 on the CPU: outlier channels in X, W ~ N(0, 0.02)."""
    x = torch.randn((p.tokens, p.hidden), generator=_gen(3), dtype=torch.float32)
    count = int(round(p.outlier_fraction * p.hidden))
    picks = torch.randperm(p.hidden, generator=_gen(5))[:count]
    x[:, picks] *= p.outlier_gain
    w = 0.02 * torch.randn((p.hidden, p.out_features), generator=_gen(4), dtype=torch.float32)
    return x.to(torch.bfloat16), w.to(torch.bfloat16)
