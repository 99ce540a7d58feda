"""Second, independent restatement of skyla-gguf/src/quant.rs in numpy (TEST INFRASTRUCTURE).

Vectorised over blocks; numpy float32 element-wise arithmetic rounds every operation
(no fusion), so the results must equal the C oracle bit for bit.  f16 -> f32 goes through
numpy.float16, an IEEE-754 implementation independent of the C one.
"""
from __future__ import annotations

import numpy as np


def _f16(b: np.ndarray) -> np.ndarray:
    """Little-endian f16 bytes [..., 2] -> f32."""
    return np.ascontiguousarray(b).view("<f2")[..., 0].astype(np.float32)


def scale_min_q4k(scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quant.rs:40-49 for all j at once: scales [n, 12] -> (sc [n, 8], m [n, 8])."""
    s = scales.astype(np.uint8)
    sc = np.empty((s.shape[0], 8), np.uint8)
    m = np.empty((s.shape[0], 8), np.uint8)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def dequant_q4k(blocks: np.ndarray) -> np.ndarray:
    """quant.rs:51-68: blocks [n, 144] -> [n, 256]."""
    b = blocks.reshape(-1, 144)
    d = _f16(b[:, 0:2].reshape(-1, 1, 2))
    dmin = _f16(b[:, 2:4].reshape(-1, 1, 2))
    sc, m = scale_min_q4k(b[:, 4:16])
    dsc = d * sc.astype(np.float32)          # [n, 8]   d * sc
    dm = dmin * m.astype(np.float32)         # [n, 8]   dmin * m
    qs = b[:, 16:144].reshape(-1, 4, 32)     # chunk, l
    lo = (qs & 0xF).astype(np.float32)       # sub-block 2c
    hi = (qs >> 4).astype(np.float32)        # sub-block 2c+1
    out = np.empty((b.shape[0], 4, 2, 32), np.float32)
    out[:, :, 0, :] = dsc[:, 0::2, None] * lo - dm[:, 0::2, None]
    out[:, :, 1, :] = dsc[:, 1::2, None] * hi - dm[:, 1::2, None]
    return out.reshape(-1, 256)


def dequant_q6k(blocks: np.ndarray) -> np.ndarray:
    """quant.rs:70-89: blocks [n, 210] -> [n, 256]."""
    b = blocks.reshape(-1, 210)
    d = _f16(b[:, 208:210].reshape(-1, 1, 2))[:, :, None]          # [n,1,1]
    out = np.empty((b.shape[0], 2, 4, 32), np.float32)
    for half in range(2):
        ql = b[:, half * 64: half * 64 + 64].astype(np.int32)
        qh = b[:, 128 + half * 32: 128 + half * 32 + 32].astype(np.int32)
        sc = b[:, 192 + half * 8: 192 + half * 8 + 8].view(np.int8).astype(np.float32)
        q = np.stack([
            (ql[:, :32] & 0xF) | ((qh & 3) << 4),
            (ql[:, 32:] & 0xF) | (((qh >> 2) & 3) << 4),
            (ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4),
            (ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4),
        ], axis=1) - 32                                                  # [n, 4, 32]
        is_ = np.arange(32) // 16
        s = sc[:, is_[None, :] + 2 * np.arange(4)[:, None]]              # [n, 4, 32]
        out[:, half] = (d * s) * q.astype(np.float32)
    return out.reshape(-1, 256)


def dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    """quant.rs:17-24: blocks [n, 34] -> [n, 32]."""
    b = blocks.reshape(-1, 34)
    d = _f16(b[:, 0:2].reshape(-1, 1, 2))
    return d * b[:, 2:].view(np.int8).astype(np.float32)


def dequantize(dtype: int, data: np.ndarray) -> np.ndarray:
    data = np.frombuffer(np.ascontiguousarray(data).tobytes(), np.uint8)
    if dtype == 12:
        return dequant_q4k(data).reshape(-1)
    if dtype == 14:
        return dequant_q6k(data).reshape(-1)
    if dtype == 8:
        return dequant_q8_0(data).reshape(-1)
    if dtype == 1:
        return data.view("<f2").astype(np.float32)
    if dtype == 0:
        return data.view("<f4").copy()
    raise ValueError(f"cannot dequantize ggml type {dtype}")
