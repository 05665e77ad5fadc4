"""GGUF reader/writer (host logic, CPU only): the product's C++ reader and the
oracle's C reader against the reference's minimal v3 file (src/gguf.rs:382-418)
and the reader's error paths (src/gguf.rs:84-101, 147-167, 231-248, 274-279,
332, 352-358, 367)."""
from __future__ import annotations

import struct

import numpy as np
import pytest


def put_string(out: bytearray, s: str):
    out += struct.pack("<Q", len(s)) + s.encode()


def minimal_v3(alignment=4, version=3, tensor_type=0, data=(1.0, 2.0, 3.0, 4.0)) -> bytes:
    """The bytes of parses_a_minimal_v3_file (src/gguf.rs:383-403)."""
    b = bytearray(b"GGUF")
    b += struct.pack("<I", version) + struct.pack("<Q", 1) + struct.pack("<Q", 1)
    put_string(b, "general.alignment")
    b += struct.pack("<I", 4) + struct.pack("<I", alignment)
    put_string(b, "x")
    b += struct.pack("<I", 2) + struct.pack("<Q", 2) + struct.pack("<Q", 2)
    b += struct.pack("<I", tensor_type) + struct.pack("<Q", 0)
    while len(b) % 4:
        b += b"\0"
    for v in data:
        b += struct.pack("<f", v)
    return bytes(b)


def test_minimal_v3_file_product_reader(llrs, tmp_path):
    p = tmp_path / "m.gguf"
    p.write_bytes(minimal_v3())
    ver, t = llrs.gguf_read_tensor(p, "x")
    assert ver == 3 and t.shape == (2, 2) and t.quant_type == llrs.QuantType.F32
    assert np.frombuffer(t.data, np.float32).tolist() == [1.0, 2.0, 3.0, 4.0]


def test_minimal_v3_file_oracle_reader(oracle, tmp_path):
    p = tmp_path / "m.gguf"
    p.write_bytes(minimal_v3())
    ver, v = oracle.gguf_read_f32(p, "x")
    assert ver == 3 and v.shape == (2, 2) and v.reshape(-1).tolist() == [1.0, 2.0, 3.0, 4.0]


def _variants():
    good = minimal_v3()
    yield "bad magic", b"GGUX" + good[4:]
    yield "version 1", minimal_v3(version=1)
    yield "version 4", minimal_v3(version=4)
    yield "truncated header", good[:20]
    yield "truncated data", good[:-3]
    yield "unknown tensor type", minimal_v3(tensor_type=99)
    yield "alignment not a power of two", minimal_v3(alignment=3)
    yield "alignment too large", minimal_v3(alignment=1 << 21)
    huge = bytearray(good)
    huge[8:16] = struct.pack("<Q", 2_000_000)
    yield "unreasonable counts", bytes(huge)
    nd = bytearray(good)
    i = nd.index(b"x", 40) + 1
    nd[i:i + 4] = struct.pack("<I", 5)
    yield "invalid dimension count", bytes(nd)
    off = bytearray(good)
    off[i + 4 + 16 + 4:i + 4 + 16 + 12] = struct.pack("<Q", 1 << 40)
    yield "tensor outside file", bytes(off)
    bad_meta = bytearray(good)
    j = good.index(b"general.alignment") + len("general.alignment")
    bad_meta[j:j + 4] = struct.pack("<I", 13)
    yield "unknown metadata type", bytes(bad_meta)


@pytest.mark.parametrize("name,data", list(_variants()), ids=[n for n, _ in _variants()])
def test_malformed_files_are_rejected(llrs, oracle, tmp_path, name, data):
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    with pytest.raises(llrs.LlrsError):
        llrs.gguf_read_tensor(p, "x")
    with pytest.raises(RuntimeError):
        oracle.gguf_read_f32(p, "x")


def test_version_2_accepted(llrs, oracle, tmp_path):
    p = tmp_path / "v2.gguf"
    p.write_bytes(minimal_v3(version=2))
    assert llrs.gguf_read_tensor(p, "x")[0] == 2
    assert oracle.gguf_read_f32(p, "x")[0] == 2


def test_synthetic_gguf_roundtrip_through_both_readers(llrs, oracle, tmp_path):
    cfg = llrs.SynthConfig(hidden_size=64, intermediate_size=256, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=1, vocab_size=128,
                           tie_word_embeddings=False, recipe=llrs.LoadQuantization.Q4KM, seed=5)
    p = tmp_path / "s.gguf"
    cfg.write_gguf(p)
    QT = llrs.QuantType
    want = {"token_embd.weight": QT.Q8_0, "output.weight": QT.Q8_0,
            "blk.0.attn_q.weight": QT.Q5_0,  # 64 columns: Q4_K falls back to Q5_0
            "blk.0.attn_v.weight": QT.Q8_0, "blk.0.ffn_down.weight": QT.Q6K,
            "blk.0.attn_norm.weight": QT.F32, "blk.0.attn_q.bias": QT.F32}
    for name, qt in want.items():
        _, t = llrs.gguf_read_tensor(p, name)
        assert t.quant_type == qt, name
        _, v = oracle.gguf_read_f32(p, name)
        assert v.shape == t.shape
    _, g = oracle.gguf_read_f32(p, "blk.0.attn_norm.weight")
    assert abs(float(g.mean()) - 1.0) < 0.02  # gains are 1 + N(0, 0.02)
    _, w = oracle.gguf_read_f32(p, "blk.0.ffn_down.weight")
    assert 0.015 < float(w.std()) < 0.025  # N(0, 0.02) after Q6_K
    # Deterministic from the seed.
    p2 = tmp_path / "s2.gguf"
    cfg.write_gguf(p2)
    assert p.read_bytes() == p2.read_bytes()
