"""Seeded synthetic GGUF blocks and activations (numpy).

Inputs for every parity test and for bench.py, generated the same way on the
CPU container and on the GPU box:

* f16 scale fields (Q4_K/Q5_K d and dmin, Q6_K d, Q8_0/Q4_0/Q5_0 d) are
  f16(U[1e-3, 2e-2]);
* every other byte (6-bit scale/min packs, nibbles, high bits, Q6_K int8
  sub-block scales, Q8_0 int8 codes) is uniform over 0..255;
* F16 weights are f16(N(0,1) * 0.02) and F32 weights N(0,1) * 0.02 (finite);
* x is f32 N(0,1).

Field offsets inside a block follow src/quant.rs:106-292.
"""
from __future__ import annotations

import numpy as np

# (block elements, block bytes, byte offsets of f16 scale fields)
LAYOUT = {
    0: (1, 4, ()),           # F32
    1: (1, 2, ()),           # F16
    2: (32, 18, (0,)),       # Q4_0: d
    6: (32, 22, (0,)),       # Q5_0: d
    8: (32, 34, (0,)),       # Q8_0: d
    12: (256, 144, (0, 2)),  # Q4_K: d, dmin
    13: (256, 176, (0, 2)),  # Q5_K: d, dmin
    14: (256, 210, (208,)),  # Q6_K: d
}


def n_blocks(dtype: int, rows: int, cols: int) -> int:
    bs = LAYOUT[dtype][0]
    return -(-(rows * cols) // bs)


def gen_blocks(dtype: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Raw bytes of a rows x cols matrix of `dtype` (flat uint8 array)."""
    bs, bb, f16_offs = LAYOUT[dtype]
    nb = n_blocks(dtype, rows, cols)
    rng = np.random.default_rng(seed)
    if dtype == 0:
        return (rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)).view(np.uint8)
    if dtype == 1:
        w = (rng.standard_normal(nb, dtype=np.float32) * np.float32(0.02)).astype(np.float16)
        return w.view(np.uint8)
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    for off in f16_offs:
        d = rng.uniform(1e-3, 2e-2, size=nb).astype(np.float16)
        raw[:, off:off + 2] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def gen_x(n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed ^ 0x5A5A5A5A).standard_normal(n, dtype=np.float32)


def config_seed(index: int) -> int:
    """Seed of BASELINE.json config `index` (0-based)."""
    return 0x5EED0000 + index
