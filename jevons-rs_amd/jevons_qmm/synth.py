"""Seeded synthetic GGML weights and activations for the benchmark workloads.

All generators draw from numpy's PCG64 seeded with one integer, so a (seed, shape) pair always
gives the same bytes. Block contents follow the GGML layouts of
crates/jevons-formats/src/quant.rs:25-80:

  Q4_K  144 B: f16 d = |N(0,1)|*1e-3, f16 dmin = |N(0,1)|*1e-3, 12 uniform scale/min bytes
        (every byte pattern decodes to uniform 6-bit values), 128 uniform quant bytes.
  Q6_K  210 B: 128 uniform low-nibble bytes, 64 uniform high-bit bytes, 16 int8 scales uniform
        in [-32, 31], f16 d = |N(0,1)|*1e-3.
  Q8_0   34 B: f16 d = |N(0,1)|*0.02/127, 32 int8 quants uniform in [-127, 127].
  Q5_0   22 B: f16 d = |N(0,1)|*0.02/15, 4 uniform high-bit bytes, 16 uniform quant bytes.
"""
from __future__ import annotations

import numpy as np


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)


def q4k(rng: np.random.Generator, rows: int, k: int) -> np.ndarray:
    nb = rows * k // 256
    out = np.empty((nb, 144), np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
    out[:, 2:4] = _f16_bytes(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
    out[:, 4:144] = rng.integers(0, 256, size=(nb, 140), dtype=np.uint8)
    return out.reshape(-1)


def q6k(rng: np.random.Generator, rows: int, k: int) -> np.ndarray:
    nb = rows * k // 256
    out = np.empty((nb, 210), np.uint8)
    out[:, 0:192] = rng.integers(0, 256, size=(nb, 192), dtype=np.uint8)
    out[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
    out[:, 208:210] = _f16_bytes(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(1e-3))
    return out.reshape(-1)


def q8_0(rng: np.random.Generator, rows: int, k: int) -> np.ndarray:
    nb = rows * k // 32
    out = np.empty((nb, 34), np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(0.02 / 127))
    out[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    return out.reshape(-1)


def q5_0(rng: np.random.Generator, rows: int, k: int) -> np.ndarray:
    nb = rows * k // 32
    out = np.empty((nb, 22), np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(0.02 / 15))
    out[:, 2:22] = rng.integers(0, 256, size=(nb, 20), dtype=np.uint8)
    return out.reshape(-1)


def f16_weights(rng: np.random.Generator, rows: int, k: int, scale: float = 0.1) -> np.ndarray:
    w = (rng.random((rows, k), dtype=np.float32) * 2 - 1) * np.float32(scale)
    return w.astype(np.float16).view(np.uint8).reshape(-1)


GENERATORS = {12: q4k, 14: q6k, 8: q8_0, 6: q5_0, 1: f16_weights}


def weights(type_id: int, seed: int, rows: int, k: int) -> np.ndarray:
    return GENERATORS[type_id](np.random.default_rng(seed), rows, k)


def normal_rows(seed: int, m: int, k: int, outlier_frac: float = 0.0, outlier_scale: float = 20.0):
    """float32 N(0,1) [m, k]; a seeded `outlier_frac` of the columns scaled by `outlier_scale`."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    if outlier_frac > 0:
        cols = rng.choice(k, size=int(round(outlier_frac * k)), replace=False)
        x[:, cols] *= np.float32(outlier_scale)
    return x


def to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits (round to nearest even), as uint16."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
