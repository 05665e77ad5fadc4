"""Seeded random GGML weight blocks for the GEMV workloads.

Every block field is drawn uniformly from its format's valid range, scales
from |N(0, 0.02)| as f16:

  Q4_0 / Q5_0 / Q8_0   d = f16 |N(0,0.02)|; codes / qh uniform bytes
  Q4_1 / Q5_1          d = f16 |N(0,0.02)|, m = f16 N(0,0.02) (signed)
  Q4_K / Q5_K          d, dmin = f16 |N(0,0.02)|; the 12 packed 6-bit
                       scale/min bytes uniform (every 12-byte pattern decodes
                       validly through scale_min_k4, src/quant.rs:338-347),
                       codes / qh uniform bytes
  Q6_K                 d = f16 |N(0,0.02)| at byte 208; ql / qh uniform bytes;
                       16 int8 sub-block scales uniform
  F16 / BF16 / F32     N(0, 0.02) rounded to the format (never NaN/Inf)

Uniform code bytes make every nibble, high bit and 6-bit code uniform too.
"""
from __future__ import annotations

import numpy as np

from . import QuantType

# Offsets (bytes) of the f16 fields inside one block: (|d| fields, signed fields).
_F16_FIELDS = {
    QuantType.Q4_0: ([0], []), QuantType.Q5_0: ([0], []), QuantType.Q8_0: ([0], []),
    QuantType.Q4_1: ([0], [2]), QuantType.Q5_1: ([0], [2]),
    QuantType.Q4K: ([0, 2], []), QuantType.Q5K: ([0, 2], []),
    QuantType.Q6K: ([208], []),
}


def _f16_bits(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint16)


def _bf16_bits(values: np.ndarray) -> np.ndarray:
    # round-to-nearest-even truncation of f32 to its top 16 bits
    b = values.astype(np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def random_tensor_bytes(quant_type, rows: int, cols: int, seed: int, std: float = 0.02) -> bytes:
    """Native bytes of a [rows, cols] tensor of random valid blocks."""
    qt = QuantType(quant_type)
    rng = np.random.default_rng(seed)
    if qt == QuantType.F32:
        return (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(std)).tobytes()
    if qt in (QuantType.F16, QuantType.BF16):
        v = rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(std)
        return (_f16_bits(v) if qt == QuantType.F16 else _bf16_bits(v)).tobytes()
    bs, ts = qt.block_size(), qt.type_size()
    nblocks = rows * (cols // bs)
    raw = rng.integers(0, 256, size=(nblocks, ts), dtype=np.uint8)
    absf, signf = _F16_FIELDS[qt]
    for off in absf:
        v = np.abs(rng.standard_normal(nblocks, dtype=np.float32) * np.float32(std))
        raw[:, off:off + 2] = _f16_bits(v).view(np.uint8).reshape(nblocks, 2)
    for off in signf:
        v = rng.standard_normal(nblocks, dtype=np.float32) * np.float32(std)
        raw[:, off:off + 2] = _f16_bits(v).view(np.uint8).reshape(nblocks, 2)
    return raw.tobytes()


def random_activation(n: int, seed: int) -> np.ndarray:
    """An f32 activation vector drawn from N(0, 1)."""
    return np.random.default_rng(seed).standard_normal(n, dtype=np.float32)
