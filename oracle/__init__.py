"""CPU oracle for the DiT attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what kelechi-c/flicker computes on its
attention hot path, so that the HIP kernels in ``flicker_amd`` can be checked
against it.  It is never part of the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to compare results against it (or, for the baseline, as
the timed CPU restatement of the reference's plain-XLA path).

Modules
  numerics   bf16 round-to-nearest-even on float32 arrays
  path       RoPE tables, QK-RMSNorm + RoPE (both the plain-XLA form and the
             fused-kernel form), plain softmax attention, bounded attention,
             the logit bound and its load-time check
  w8a8       SmoothQuant W8A8 quantisation and the exact int32 GEMM

Pinning status (how each function is checked; see tests/test_oracle_*.py):
  rope_freqs / embed_nd / img_ids / txt_ids / lane_pair / apply_rope
      closed forms (omega_k = theta^(-2k/dim)), complex multiplication by
      e^{i angle}, identity at position 0, axis placement, f64 brute force.
  rms_norm / heads / merge_heads / qk_prep_plain / qk_prep_fused
      f64 brute-force loops on tiny shapes, constant-row known answers,
      norm preservation of the rotation, index round trips, and agreement
      of two independently written formulations (lanes vs 2x2 pairs).
  sdpa / attend_bounded
      f64 brute-force loops, uniform-key and dominant-key special cases,
      max-subtracted vs plain exponent identity.
  logit_bound / check_logit_bound
      Cauchy-Schwarz property on random normalised inputs; threshold at 80.
  w8a8 (not in the reference)
      brute-force integer loops; RNE tie cases; clamp; exactness of the
      float64 route for |acc| < 2^53.
  Parity unpinned: bit-level agreement with XLA's own rsqrt/exp/cos/sin and
  reduction order (jax is not installable here and the reference ships no
  golden vectors); all such differences are below one bf16 ulp per element.
"""

from . import numerics, path, w8a8  # noqa: F401
