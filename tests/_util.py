"""Shared helpers for the parity tests: tensor conversion and error statistics."""

from __future__ import annotations

import numpy as np
import torch

from oracle.numerics import bf16_ulp


def to_np(t: torch.Tensor) -> np.ndarray:
    """Any torch tensor (bf16 included) -> float32 numpy array on the host (exact for bf16)."""
    return t.detach().to("cpu", torch.float32).numpy()


def ulp_stats(got: np.ndarray, want: np.ndarray) -> dict:
    """Elementwise differences measured in bf16 ulps of the expected value."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ulps = diff / bf16_ulp(want).astype(np.float64)
    return {
        "max_ulps": float(ulps.max()) if ulps.size else 0.0,
        "mismatch": float(np.mean(diff > 0)) if diff.size else 0.0,
        "max_abs": float(diff.max()) if diff.size else 0.0,
    }


def abs_stats(got: np.ndarray, want: np.ndarray) -> dict:
    diff = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    return {"max_abs": float(diff.max()), "mean_abs": float(diff.mean())}


def describe(label: str, stats: dict) -> str:
    return label + " " + " ".join(f"{k}={v:.3g}" for k, v in stats.items())
