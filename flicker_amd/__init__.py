"""flicker_amd -- MI355X (gfx950) implementation of kelechi-c/flicker's DiT attention hot path.

  kernels   Freqs, row_tile, lane_pair, qk_prep, logit_bound, attend   (src/flicker/kernels.py)
  rope      img_ids, txt_ids, embed_nd, rope_freqs, rope_lanes           (src/flicker/rope.py)
  modules   heads, merge_heads, qkv_prep, double/single block attention (src/flicker/modules.py)
  loader    check_logit_bound                                            (src/flicker/loader.py)
  workloads seeded synthetic Klein attention inputs

All compute runs in libflicker_hip.so (hand-written HIP for gfx950) through its C ABI.
"""

from .kernels import (EPS, EXP_LIMIT, ROW_TILES, SCORE_TILES, Freqs, attend, lane_pair,  # noqa: F401
                      logit_bound, qk_prep, row_tile)

__all__ = ["EPS", "EXP_LIMIT", "ROW_TILES", "SCORE_TILES", "Freqs", "attend", "lane_pair",
           "logit_bound", "qk_prep", "row_tile"]
