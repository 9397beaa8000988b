"""Random GGUF blocks with controlled f16 scale fields (shared by CPU and GPU tests)."""
from __future__ import annotations

import numpy as np

from oracle.oracle import BLOCK

# f16 fields per block type: (byte offset, lo, hi) magnitude ranges for the scales
F16_FIELDS = {6: [(0, 0.002, 0.05)], 7: [(0, 0.002, 0.05), (2, -0.1, 0.1)], 8: [(0, 0.0005, 0.01)],
              12: [(0, 0.0005, 0.01), (2, 0.0005, 0.01)], 13: [(0, 0.0005, 0.01), (2, 0.0005, 0.01)],
              14: [(208, 0.0001, 0.002)]}
TYPES = {"Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


def random_blocks(type_id: int, n_elems: int, rng: np.random.Generator, special: bool = False) -> np.ndarray:
    be, bb = BLOCK[type_id]
    raw = rng.integers(0, 256, size=(n_elems // be, bb), dtype=np.uint8)
    for off, lo, hi in F16_FIELDS[type_id]:
        vals = rng.uniform(lo, hi, size=raw.shape[0]) * rng.choice([-1.0, 1.0], size=raw.shape[0])
        if special:
            # zero, subnormal, tiny, large and negative-zero scales
            pool = np.array([0.0, 5.96e-8, 6.1e-5, -2.0, 1024.0, -0.0], dtype=np.float64)
            pick = rng.random(raw.shape[0]) < 0.3
            vals[pick] = rng.choice(pool, size=pick.sum())
        raw[:, off:off + 2] = vals.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)
