"""An independent, vectorised float32 decoder of the GGML block formats.

Written from the GGML block layouts (one whole block at a time, numpy
broadcasting), not from the oracle's per-element value_at.  Every product in
a dequantized value (f16 scale x <= 8-bit scale x <= 6-bit code) is exact in
float32, so this decoder and the oracle must agree bit-for-bit.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def _f16(raw: np.ndarray, off: int) -> np.ndarray:
    return raw[:, off:off + 2].copy().view(np.float16).astype(F32).reshape(-1)


def _scale_min_k4(sc12: np.ndarray):
    """6-bit scales and mins of the 8 sub-blocks of a K-quant super-block."""
    s = sc12.astype(np.int32)
    scale = np.empty((s.shape[0], 8), np.int32)
    mn = np.empty((s.shape[0], 8), np.int32)
    scale[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    scale[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return scale.astype(F32), mn.astype(F32)


def dequantize(data: bytes, ggml_type: int, rows: int, cols: int) -> np.ndarray:
    """Returns float32 [rows, cols]."""
    buf = np.frombuffer(data, dtype=np.uint8)
    if ggml_type == 0:
        return buf.view(F32).reshape(rows, cols).copy()
    if ggml_type == 1:
        return buf.view(np.float16).astype(F32).reshape(rows, cols)
    if ggml_type == 30:
        b = buf.view(np.uint16).astype(np.uint32) << 16
        nan = (buf.view(np.uint16) & 0x7FFF) > 0x7F80
        b[nan] |= 0x00400000
        return b.view(F32).reshape(rows, cols)
    size = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 12: 144, 13: 176, 14: 210}[ggml_type]
    raw = buf.reshape(-1, size)
    n = raw.shape[0]
    if ggml_type in (2, 3):  # Q4_0, Q4_1: low nibbles = first 16 values, high = last 16
        qo = 2 if ggml_type == 2 else 4
        qs = raw[:, qo:qo + 16]
        q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(F32)
        d = _f16(raw, 0)[:, None]
        out = d * (q - F32(8)) if ggml_type == 2 else d * q + _f16(raw, 2)[:, None]
    elif ggml_type in (6, 7):  # Q5_0, Q5_1: 32 high bits in a little-endian u32
        ho, qo = (2, 6) if ggml_type == 6 else (4, 8)
        qh = raw[:, ho:ho + 4].copy().view("<u4").reshape(-1).astype(np.uint64)
        bits = ((qh[:, None] >> np.arange(32, dtype=np.uint64)) & 1).astype(np.int32)
        qs = raw[:, qo:qo + 16].astype(np.int32)
        q = (np.concatenate([qs & 0xF, qs >> 4], axis=1) | (bits << 4)).astype(F32)
        d = _f16(raw, 0)[:, None]
        out = d * (q - F32(16)) if ggml_type == 6 else d * q + _f16(raw, 2)[:, None]
    elif ggml_type == 8:  # Q8_0
        out = _f16(raw, 0)[:, None] * raw[:, 2:34].view(np.int8).astype(F32)
    elif ggml_type in (12, 13):  # Q4_K, Q5_K: 4 pairs of sub-blocks share 32 code bytes
        d, dmin = _f16(raw, 0)[:, None], _f16(raw, 2)[:, None]
        sc, mn = _scale_min_k4(raw[:, 4:16])
        qo = 16 if ggml_type == 12 else 48
        qs = raw[:, qo:qo + 128].reshape(n, 4, 32).astype(np.int32)
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(n, 8, 32)  # sub-block 2p, 2p+1
        if ggml_type == 13:
            qh = raw[:, 16:48].astype(np.int32)  # bit g of byte l: sub-block g, element l
            hb = (qh[:, None, :] >> np.arange(8)[None, :, None]) & 1
            q = q + hb * 16
        out = (d[:, :, None] * sc[:, :, None] * q.astype(F32) -
               dmin[:, :, None] * mn[:, :, None]).reshape(n, 256)
    elif ggml_type == 14:  # Q6_K: [ql 128][qh 64][scales 16 x i8][d]
        d = _f16(raw, 208)
        out = np.empty((n, 256), F32)
        for half in range(2):
            ql = raw[:, 64 * half:64 * half + 64].astype(np.int32)
            qh = raw[:, 128 + 32 * half:128 + 32 * half + 32].astype(np.int32)
            sc = raw[:, 192 + 8 * half:200 + 8 * half].view(np.int8).astype(F32)
            quarters = [
                (ql[:, :32] & 0xF) | ((qh & 3) << 4),
                (ql[:, 32:] & 0xF) | (((qh >> 2) & 3) << 4),
                (ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4),
                (ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4),
            ]
            for k, q in enumerate(quarters):
                scale = np.repeat(sc[:, 2 * k:2 * k + 2], 16, axis=1)  # elements 0-15 / 16-31
                out[:, 128 * half + 32 * k:128 * half + 32 * k + 32] = (
                    d[:, None] * scale * (q - 32).astype(F32))
    else:
        raise ValueError(ggml_type)
    return out.astype(F32).reshape(rows, cols)
