"""Seeded synthetic GGUF blocks and activations for the benchmark configurations.

Every tensor is drawn from numpy's PCG64 generator seeded with the first 8 bytes of
SHA-256("<config>/<tensor name>"), so the GPU box regenerates bit-identical inputs.
f16 fields are drawn as f32 and rounded to f16 with round-to-nearest-even.

  Q4_K (256 values / 144 B): d, dmin ~ U[1e-3, 1e-2]; the 12 scale bytes and 128 quant
       bytes are uniform bytes, i.e. 6-bit scales/mins uniform in 0..63 and nibbles in 0..15.
  Q6_K (256 values / 210 B): ql, qh uniform bytes (6-bit quants uniform in 0..63), int8
       sub-scales ~ U{-64..64}, d ~ U[1e-3, 1e-2].
  Q8_0 (32 values / 34 B): d ~ U[1e-3, 4e-3], quants ~ U{-127..127}.
  activations: f32 N(0, 1).
"""
from __future__ import annotations

import hashlib

import numpy as np

from .engine import DType, row_bytes


def seed_of(config: str, name: str) -> int:
    return int.from_bytes(hashlib.sha256(f"{config}/{name}".encode()).digest()[:8], "little")


def rng(config: str, name: str) -> np.random.Generator:
    return np.random.default_rng(seed_of(config, name))


def _f16_bytes(g: np.random.Generator, n: int, lo: float, hi: float) -> np.ndarray:
    v = g.uniform(lo, hi, size=n).astype(np.float32).astype(np.float16)
    return v.view(np.uint8).reshape(n, 2)


def q4k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    b = g.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(g, n_blocks, 1e-3, 1e-2)
    b[:, 2:4] = _f16_bytes(g, n_blocks, 1e-3, 1e-2)
    return b


def q6k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    b = g.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
    b[:, 192:208] = g.integers(-64, 65, size=(n_blocks, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
    b[:, 208:210] = _f16_bytes(g, n_blocks, 1e-3, 1e-2)
    return b


def q8_0_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    b = np.empty((n_blocks, 34), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(g, n_blocks, 1e-3, 4e-3)
    b[:, 2:34] = g.integers(-127, 128, size=(n_blocks, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return b


def matrix(config: str, name: str, dtype: DType, n_in: int, n_out: int, n_expert: int = 1) -> np.ndarray:
    """Raw GGUF bytes of a [n_expert][n_out] x n_in matrix, flat uint8."""
    g = rng(config, name)
    n_blocks = n_expert * n_out * row_bytes(dtype, n_in) // {DType.Q4K: 144, DType.Q6K: 210, DType.Q8_0: 34}[dtype]
    maker = {DType.Q4K: q4k_blocks, DType.Q6K: q6k_blocks, DType.Q8_0: q8_0_blocks}[DType(dtype)]
    return maker(g, n_blocks).reshape(-1)


def activations(config: str, name: str, shape) -> np.ndarray:
    return rng(config, name).standard_normal(size=shape, dtype=np.float32)


def router(config: str, name: str, n_expert: int, n_embd: int) -> np.ndarray:
    return (rng(config, name).standard_normal(size=(n_expert, n_embd), dtype=np.float32) * np.float32(0.02))
