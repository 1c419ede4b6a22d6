"""Klein 4B DiT constants used by the attention path (reference: src/flicker/config.py:26-48)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Klein4B:
    """The hyper-parameters of FLUX.2 [klein] 4B that shape the attention hot path."""

    hidden_size: int = 3072
    num_heads: int = 24
    depth: int = 5                  # double-stream blocks
    depth_single_blocks: int = 20
    axes_dim: tuple = (32, 32, 32, 32)
    theta: int = 2000
    mlp_ratio: float = 3.0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def mlp_hidden(self) -> int:
        return int(self.hidden_size * self.mlp_ratio)
