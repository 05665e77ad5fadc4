"""Plain numpy encoders for Q4_0, Q4_1, Q5_1 and Q5_K blocks (test
infrastructure): valid GGML blocks that represent given weights to within a
code step, used to build test models whose matrices have these types.  They
are not llama.cpp's search-based encoders (the reference has none for these
types: src/quant.rs quantizes to Q4_K, Q5_0, Q8_0 and Q6_K only); the GPU
and the oracle read the same bytes, so any valid encoding serves.

Layouts (value_at, src/quant.rs:349-456):
  Q4_0  f16 d, 16 bytes: weight j < 16 = low nibble of byte j, 16 + j = high
        nibble; value d * (q - 8).
  Q4_1  f16 d, f16 m, 16 bytes as Q4_0; value d * q + m.
  Q5_1  f16 d, f16 m, 32 high bits (bit j = weight j), 16 bytes as Q4_0;
        value d * q + m, q = nibble | high bit << 4.
  Q5_K  f16 d, f16 dmin, 12 bytes of 6-bit scales/mins (scale_min_k4),
        32 bytes qh (bit g of byte l = high bit of weight l of group g),
        128 bytes qs (pair p: byte l = group 2p low nibble | group 2p+1
        high nibble); value d * sc_g * q - dmin * m_g, q in 0..31.
"""
from __future__ import annotations

import numpy as np


def _f16(v) -> np.ndarray:
    return np.asarray(v, np.float32).astype(np.float16)


def _nibbles(q: np.ndarray) -> np.ndarray:
    """[n, 32] codes -> [n, 16] bytes (low nibble = weight j, high = 16 + j)."""
    return ((q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)).astype(np.uint8)


def q4_0(x: np.ndarray) -> bytes:
    b = np.asarray(x, np.float32).reshape(-1, 32)
    idx = np.argmax(np.abs(b), axis=1)
    mx = b[np.arange(len(b)), idx]
    d = _f16(mx / -8.0)
    df = d.astype(np.float32)
    inv = np.where(df != 0, 1.0 / np.where(df != 0, df, 1), 0)
    q = np.clip(np.rint(b * inv[:, None] + 8), 0, 15).astype(np.int64)
    out = np.concatenate([d.view(np.uint8).reshape(-1, 2), _nibbles(q)], axis=1)
    return out.tobytes()


def _affine(b: np.ndarray, levels: int):
    lo, hi = b.min(axis=1), b.max(axis=1)
    d = _f16((hi - lo) / levels)
    m = _f16(lo)
    df, mf = d.astype(np.float32), m.astype(np.float32)
    inv = np.where(df != 0, 1.0 / np.where(df != 0, df, 1), 0)
    q = np.clip(np.rint((b - mf[:, None]) * inv[:, None]), 0, levels).astype(np.int64)
    return d, m, q


def q4_1(x: np.ndarray) -> bytes:
    b = np.asarray(x, np.float32).reshape(-1, 32)
    d, m, q = _affine(b, 15)
    out = np.concatenate([d.view(np.uint8).reshape(-1, 2), m.view(np.uint8).reshape(-1, 2),
                          _nibbles(q)], axis=1)
    return out.tobytes()


def q5_1(x: np.ndarray) -> bytes:
    b = np.asarray(x, np.float32).reshape(-1, 32)
    d, m, q = _affine(b, 31)
    qh = (((q >> 4) & 1) << np.arange(32)).sum(axis=1).astype(np.uint32)
    out = np.concatenate([d.view(np.uint8).reshape(-1, 2), m.view(np.uint8).reshape(-1, 2),
                          qh.view(np.uint8).reshape(-1, 4), _nibbles(q)], axis=1)
    return out.tobytes()


def _k4_pack(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """[n, 8] 6-bit scales and mins -> [n, 12] bytes (inverse of scale_min_k4)."""
    s = np.zeros((len(sc), 12), np.int64)
    s[:, 0:4] = sc[:, 0:4]
    s[:, 4:8] = mn[:, 0:4]
    s[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    s[:, 0:4] |= (sc[:, 4:8] >> 4) << 6
    s[:, 4:8] |= (mn[:, 4:8] >> 4) << 6
    return s.astype(np.uint8)


def q5_k(x: np.ndarray) -> bytes:
    b = np.asarray(x, np.float32).reshape(-1, 8, 32)
    lo = np.minimum(b.min(axis=2), 0.0)
    hi = b.max(axis=2)
    scale = (hi - lo) / 31.0                     # per group
    minv = -lo                                   # >= 0
    d = _f16(scale.max(axis=1) / 63.0)
    dm = _f16(minv.max(axis=1) / 63.0)
    df, dmf = d.astype(np.float32), dm.astype(np.float32)
    sc = np.clip(np.rint(scale / np.where(df != 0, df, 1)[:, None]), 0, 63).astype(np.int64)
    mn = np.clip(np.rint(minv / np.where(dmf != 0, dmf, 1)[:, None]), 0, 63).astype(np.int64)
    step = df[:, None] * sc                      # per group
    off = dmf[:, None] * mn
    q = np.where(step[:, :, None] != 0,
                 np.rint((b + off[:, :, None]) / np.where(step != 0, step, 1)[:, :, None]), 0)
    q = np.clip(q, 0, 31).astype(np.int64)       # [n, 8, 32]
    qh = np.zeros((len(b), 32), np.int64)
    for g in range(8):
        qh |= ((q[:, g] >> 4) & 1) << g
    qs = np.concatenate([(q[:, 2 * p] & 15) | ((q[:, 2 * p + 1] & 15) << 4) for p in range(4)], axis=1)
    out = np.concatenate([d.view(np.uint8).reshape(-1, 2), dm.view(np.uint8).reshape(-1, 2),
                          _k4_pack(sc, mn), qh.astype(np.uint8), qs.astype(np.uint8)], axis=1)
    return out.tobytes()


ENCODERS = {2: q4_0, 3: q4_1, 7: q5_1, 13: q5_k}  # GGML type id -> encoder
