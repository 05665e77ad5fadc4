"""A minimal GGUF v3 writer for tests: rewrites a model file with some
tensors replaced (planted LM-head rows, edited weight types), so that a test
can build a Qwen2 model whose outputs it knows in advance.

Format (the GGUF spec; the reference's reader is src/gguf.rs:77-258): magic
"GGUF", u32 version, u64 tensor count, u64 metadata count, metadata
(string key, u32 value type, value), tensor infos (string name, u32 n_dims,
u64 dims innermost first, u32 ggml type, u64 offset from the data section),
then the data section aligned to `general.alignment`.  Strings are a u64
length and UTF-8 bytes.
"""
from __future__ import annotations

import struct

GGUF_UINT32, GGUF_FLOAT32, GGUF_STRING = 4, 6, 8


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def qwen2_metadata(cfg) -> list[tuple[str, int, object]]:
    """The metadata keys GgufLoader::load reads (src/loader.rs:246-278) for `cfg`
    (a SynthConfig or anything with the same fields)."""
    return [
        ("general.architecture", GGUF_STRING, "qwen2"),
        ("general.alignment", GGUF_UINT32, 32),
        ("qwen2.embedding_length", GGUF_UINT32, cfg.hidden_size),
        ("qwen2.feed_forward_length", GGUF_UINT32, cfg.intermediate_size),
        ("qwen2.attention.head_count", GGUF_UINT32, cfg.num_attention_heads),
        ("qwen2.attention.head_count_kv", GGUF_UINT32, cfg.num_key_value_heads),
        ("qwen2.block_count", GGUF_UINT32, cfg.num_hidden_layers),
        ("qwen2.context_length", GGUF_UINT32, cfg.max_position_embeddings),
        ("qwen2.attention.layer_norm_rms_epsilon", GGUF_FLOAT32, cfg.rms_norm_eps),
        ("qwen2.rope.freq_base", GGUF_FLOAT32, cfg.rope_theta),
    ]


def write_gguf(path, metadata, tensors, alignment: int = 32) -> None:
    """tensors: list of (name, ggml_type, rows, cols, data bytes); a vector has
    rows == 1 and is written with one dimension."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", 3, len(tensors), len(metadata))
    for key, ty, value in metadata:
        out += _string(key) + struct.pack("<I", ty)
        if ty == GGUF_STRING:
            out += _string(value)
        elif ty == GGUF_UINT32:
            out += struct.pack("<I", int(value))
        elif ty == GGUF_FLOAT32:
            out += struct.pack("<f", float(value))
        else:
            raise ValueError(f"metadata type {ty} not supported here")
    offsets, off = [], 0
    for name, ty, rows, cols, data in tensors:
        offsets.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, ty, rows, cols, data), o in zip(tensors, offsets):
        dims = [cols] if rows == 1 and name.endswith((".bias", "norm.weight")) else [cols, rows]
        out += _string(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, o)
    out += b"\0" * ((-len(out)) % alignment)
    for (name, ty, rows, cols, data), o in zip(tensors, offsets):
        out += data
        out += b"\0" * ((-len(data)) % alignment)
    with open(path, "wb") as f:
        f.write(bytes(out))


def rewrite(llrs, src, dst, cfg, names, replace=None) -> None:
    """Copies the tensors `names` of GGUF file `src` to `dst`, replacing those in
    `replace` (name -> (ggml_type, rows, cols, bytes))."""
    replace = replace or {}
    tensors = []
    for name in names:
        if name in replace:
            tensors.append((name,) + tuple(replace[name]))
            continue
        _, t = llrs.gguf_read_tensor(src, name)
        rows, cols = t.shape if len(t.shape) == 2 else (1, t.shape[0])
        tensors.append((name, int(t.quant_type), rows, cols, bytes(t.data)))
    write_gguf(dst, qwen2_metadata(cfg), tensors)
