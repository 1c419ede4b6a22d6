"""torch-CPU float32 restatement of the reference's plain-XLA attention path -- the CPU
baseline that bench.py times beside the GPU numbers (test infrastructure only).

The reference's own CPU path is JAX on XLA:CPU, which cannot run here (no jax).  This
is the same computation in torch on the host cores, f32 compute from bf16 inputs:
  heads + rms_norm + apply_rope   modules.py:56-60,78-80; nn.py:24-27; rope.py:24-30
  sdpa                            nn.py:35-44
processed one head at a time (the arithmetic is per head, so chunking changes nothing).
"""

from __future__ import annotations

import math

import torch


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def rms_norm(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """nn.py:24-27 with bf16 activations and scale."""
    normed = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    return _bf16(_bf16(normed) * scale)


def apply_rope(x: torch.Tensor, pe: torch.Tensor) -> torch.Tensor:
    """rope.py:24-30 -- pe (L, P, 2, 2); x (..., L, 2P)."""
    pairs = x.reshape(*x.shape[:-1], -1, 1, 2)
    out = pe[..., 0] * pairs[..., 0] + pe[..., 1] * pairs[..., 1]
    return _bf16(out.reshape(x.shape))


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """nn.py:35-44 for one head: f32 logits * 1/sqrt(D), softmax, weights @ v, bf16."""
    logits = (q @ k.T) * (1.0 / math.sqrt(q.shape[-1]))
    return _bf16(torch.softmax(logits, dim=-1) @ v)


def plain_attention(qkv: torch.Tensor, q_scale: torch.Tensor, k_scale: torch.Tensor, pe: torch.Tensor,
                    num_heads: int, heads=None) -> torch.Tensor:
    """qkv (B, L, 3HD) bf16 (CPU), pe (L, P, 2, 2) f32 -> o (B, len(heads), L, D) bf16-valued f32."""
    batch, length, width = qkv.shape
    dim = width // (3 * num_heads)
    heads = list(range(num_heads)) if heads is None else list(heads)
    qs, ks = q_scale.float(), k_scale.float()
    out = torch.empty(batch, len(heads), length, dim)
    for b in range(batch):
        row = qkv[b].float()
        for j, h in enumerate(heads):
            q = row[:, h * dim:(h + 1) * dim]
            k = row[:, (num_heads + h) * dim:(num_heads + h + 1) * dim]
            v = row[:, (2 * num_heads + h) * dim:(2 * num_heads + h + 1) * dim]
            q = apply_rope(rms_norm(q, qs), pe)
            k = apply_rope(rms_norm(k, ks), pe)
            out[b, j] = sdpa(q, k, v)
    return out
