"""SafeTensors loader: SafetensorsLoader::load, SafetensorStore and
LlamaConfig::from_json (src/loader.rs:44-228, 536-645; src/config.rs:17-90).

The reader is pinned against the `safetensors` Python package (a separate
implementation of the format): every file it writes reads back byte for
byte, and each malformed header below is rejected by both.  The GPU tests
then check that a checkpoint loads into exactly the device tensors the GGUF
path builds from the same values (bit-exact, unquantized and through the
load-time quantizers) and decodes the oracle's greedy tokens.
"""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from hf_checkpoint import write_checkpoint

E_INVALID, E_UNSUPPORTED, E_FORMAT = -1, -2, -6


def _pkg_rejects(path) -> bool:
    import safetensors.numpy
    try:
        safetensors.numpy.load_file(str(path))
    except Exception:
        return True
    return False


def raw_file(header, data: bytes = b"", n: int | None = None) -> bytes:
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    return struct.pack("<Q", len(h) if n is None else n) + h + data


# -------------------------------------------------------------- the reader

def test_reader_matches_safetensors_package(llrs, tmp_path):
    import safetensors.torch
    import torch
    rng = np.random.default_rng(3)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float16)
    c = torch.from_numpy(rng.standard_normal((4, 6)).astype(np.float32)).to(torch.bfloat16)
    safetensors.torch.save_file({"a": torch.from_numpy(a), "b": torch.from_numpy(b), "c": c},
                                str(tmp_path / "model.safetensors"), metadata={"format": "pt"})
    ty, shape, data = llrs.safetensors_read_tensor(tmp_path, "a")
    assert (ty, shape, data) == (llrs.QuantType.F32, (3, 5), a.tobytes())
    ty, shape, data = llrs.safetensors_read_tensor(tmp_path, "b")
    assert (ty, shape, data) == (llrs.QuantType.F16, (8,), b.tobytes())
    ty, shape, data = llrs.safetensors_read_tensor(tmp_path, "c")
    assert (ty, shape) == (llrs.QuantType.BF16, (4, 6))
    assert data == c.view(torch.int16).numpy().tobytes()
    with pytest.raises(llrs.LlrsError, match="missing safetensors tensor"):
        llrs.safetensors_read_tensor(tmp_path, "d")


def test_index_shards_and_duplicates(llrs, tmp_path):
    import safetensors.numpy
    x, y = np.arange(4, dtype=np.float32), np.arange(6, dtype=np.float32).reshape(2, 3)
    safetensors.numpy.save_file({"x": x}, str(tmp_path / "s1.safetensors"))
    safetensors.numpy.save_file({"y": y}, str(tmp_path / "s2.safetensors"))
    # No index: every .safetensors file of the directory.
    assert llrs.safetensors_read_tensor(tmp_path, "y")[2] == y.tobytes()
    safetensors.numpy.save_file({"x": x * 2}, str(tmp_path / "s3.safetensors"))
    with pytest.raises(llrs.LlrsError, match="duplicate safetensors tensor x"):
        llrs.safetensors_read_tensor(tmp_path, "y")
    # An index names the shard of each tensor; other files are not read.
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"x": "s3.safetensors", "y": "s2.safetensors",
                                   "z": "s1.safetensors"}}))
    assert llrs.safetensors_read_tensor(tmp_path, "x")[2] == (x * 2).tobytes()
    with pytest.raises(llrs.LlrsError, match="not in"):
        llrs.safetensors_read_tensor(tmp_path, "z")
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weights": {}}))
    with pytest.raises(llrs.LlrsError) as e:
        llrs.safetensors_read_tensor(tmp_path, "x")
    assert e.value.code == E_FORMAT
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(llrs.LlrsError, match="no .safetensors files"):
        llrs.safetensors_read_tensor(empty, "x")


def _malformed():
    f4 = struct.pack("<4f", 1, 2, 3, 4)
    ok = {"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}
    yield "too_small", b"\x01\x00\x00"
    yield "header_too_large", raw_file(b"{}", n=100_000_001)
    yield "length_past_end", raw_file(json.dumps(ok).encode(), f4, n=1000)
    yield "not_utf8", raw_file(b'{"t\xff": 1}', f4)
    yield "not_an_object", raw_file(b'[1, 2]')
    yield "bad_json", raw_file(b'{"t": {"dtype": "F32",', f4)
    yield "unknown_dtype", raw_file({"t": {"dtype": "F3", "shape": [4], "data_offsets": [0, 16]}}, f4)
    yield "gap", raw_file({"t": {"dtype": "F32", "shape": [4], "data_offsets": [4, 20]}}, f4 + f4)
    yield "size_mismatch", raw_file({"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, f4)
    yield "trailing_bytes", raw_file(ok, f4 + b"\0" * 4)
    yield "short_data", raw_file(ok, f4[:12])
    yield "overlap", raw_file({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]},
                               "u": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]}}, f4)
    yield "three_offsets", raw_file({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16, 16]}}, f4)
    yield "negative_dim", raw_file({"t": {"dtype": "F32", "shape": [-4], "data_offsets": [0, 16]}}, f4)
    yield "float_dim", raw_file({"t": {"dtype": "F32", "shape": [4.0], "data_offsets": [0, 16]}}, f4)
    yield "metadata_not_strings", raw_file({"__metadata__": {"a": 1}, **ok}, f4)


@pytest.mark.parametrize("name,data", list(_malformed()), ids=[n for n, _ in _malformed()])
def test_malformed_headers_rejected_like_the_package(llrs, tmp_path, name, data):
    path = tmp_path / "model.safetensors"
    path.write_bytes(data)
    assert _pkg_rejects(path), name  # the independent implementation rejects it too
    with pytest.raises(llrs.LlrsError) as e:
        llrs.safetensors_read_tensor(tmp_path, "t")
    assert e.value.code == E_FORMAT, (name, str(e.value))


def test_valid_edge_files_accepted_like_the_package(llrs, tmp_path):
    """Whitespace around the JSON, __metadata__, an empty tensor and tensors
    listed out of offset order are all valid."""
    f4 = struct.pack("<4f", 1, 2, 3, 4)
    hdr = json.dumps({"u": {"dtype": "F16", "shape": [2], "data_offsets": [16, 20]},
                      "__metadata__": {"format": "pt"},
                      "e": {"dtype": "F32", "shape": [0, 3], "data_offsets": [16, 16]},
                      "t": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}).encode()
    hdr = b" \n" + hdr + b" " * (-len(hdr) % 8)
    path = tmp_path / "model.safetensors"
    path.write_bytes(raw_file(hdr, f4 + np.array([1.5, -2], np.float16).tobytes()))
    assert not _pkg_rejects(path)
    assert llrs.safetensors_read_tensor(tmp_path, "t") == (llrs.QuantType.F32, (2, 2), f4)
    ty, shape, data = llrs.safetensors_read_tensor(tmp_path, "u")
    assert np.frombuffer(data, np.float16).tolist() == [1.5, -2.0]


def test_unsupported_dtypes_and_ranks(llrs, tmp_path):
    import safetensors.numpy
    safetensors.numpy.save_file({"i": np.arange(4, dtype=np.int32),
                                 "d": np.zeros(2, np.float64),
                                 "cube": np.zeros((2, 2, 2), np.float32),
                                 "s": np.zeros((), np.float32)}, str(tmp_path / "model.safetensors"))
    for name in ("i", "d"):
        with pytest.raises(llrs.LlrsError, match="unsupported safetensors dtype") as e:
            llrs.safetensors_read_tensor(tmp_path, name)
        assert e.value.code == E_UNSUPPORTED
    for name in ("cube", "s"):
        with pytest.raises(llrs.LlrsError, match="only 1D and 2D"):
            llrs.safetensors_read_tensor(tmp_path, name)


# ------------------------------------------------------------- config.json

QWEN25_7B = {  # the fields of Qwen2.5-7B-Instruct's config.json
    "architectures": ["Qwen2ForCausalLM"], "attention_dropout": 0.0, "bos_token_id": 151643,
    "eos_token_id": 151645, "hidden_act": "silu", "hidden_size": 3584, "initializer_range": 0.02,
    "intermediate_size": 18944, "max_position_embeddings": 32768, "max_window_layers": 28,
    "model_type": "qwen2", "num_attention_heads": 28, "num_hidden_layers": 28,
    "num_key_value_heads": 4, "rms_norm_eps": 1e-06, "rope_theta": 1000000.0,
    "sliding_window": 131072, "tie_word_embeddings": False, "torch_dtype": "bfloat16",
    "transformers_version": "4.43.1", "use_cache": True, "use_sliding_window": False,
    "vocab_size": 152064,
}


def _cfg(llrs, tmp_path, d):
    p = tmp_path / "config.json"
    p.write_text(json.dumps(d) if isinstance(d, dict) else d)
    return llrs.hf_config(p)


def test_config_qwen25_7b(llrs, tmp_path):
    c = _cfg(llrs, tmp_path, QWEN25_7B)
    assert (c.hidden_size, c.intermediate_size, c.num_attention_heads, c.num_key_value_heads,
            c.num_hidden_layers, c.vocab_size, c.max_position_embeddings) == \
        (3584, 18944, 28, 4, 28, 152064, 32768)
    assert (c.head_dim, c.kv_width, c.tie_word_embeddings) == (128, 512, False)
    assert c.rms_norm_eps == np.float32(1e-6) and c.rope_theta == 1e6


def test_config_defaults_and_optional_fields(llrs, tmp_path):
    """src/config.rs:4-14, 24-38: rms_norm_eps 1e-6, rope_theta 10000,
    max_position_embeddings 32768, tie_word_embeddings false, head_dim
    hidden / heads; integers are accepted for float fields."""
    base = {k: QWEN25_7B[k] for k in ("model_type", "hidden_size", "intermediate_size",
                                      "num_attention_heads", "num_key_value_heads",
                                      "num_hidden_layers", "vocab_size")}
    c = _cfg(llrs, tmp_path, base)
    assert (c.rms_norm_eps, c.rope_theta, c.max_position_embeddings, c.tie_word_embeddings,
            c.head_dim) == (np.float32(1e-6), 10000.0, 32768, False, 128)
    c = _cfg(llrs, tmp_path, {**base, "head_dim": 128, "rms_norm_eps": 1, "tie_word_embeddings": True,
                              "head_dim_unused": None})
    assert (c.head_dim, c.rms_norm_eps, c.tie_word_embeddings) == (128, 1.0, True)
    assert _cfg(llrs, tmp_path, {**base, "head_dim": None}).head_dim == 128


@pytest.mark.parametrize("patch,match,code", [
    ({"model_type": "llama"}, "unsupported Hugging Face model_type", E_UNSUPPORTED),
    ({"model_type": None}, "missing model_type", E_INVALID),
    ({"hidden_size": None}, "hidden_size", E_FORMAT),
    ({"hidden_size": 3584.0}, "hidden_size", E_FORMAT),
    ({"num_key_value_heads": -4}, "num_key_value_heads", E_FORMAT),
    ({"rms_norm_eps": "1e-6"}, "rms_norm_eps", E_FORMAT),
    ({"tie_word_embeddings": 0}, "tie_word_embeddings", E_FORMAT),
    ({"vocab_size": 0}, "non-zero", E_INVALID),
    ({"num_key_value_heads": 3}, "divisible by num_key_value_heads", E_INVALID),
    ({"hidden_size": 3585}, "divisible by num_attention_heads", E_INVALID),
    ({"head_dim": 64}, "must equal hidden_size", E_INVALID),
    ({"hidden_size": 28 * 7, "head_dim": 7}, "even head_dim", E_INVALID),
    ({"rms_norm_eps": 0}, "rms_norm_eps", E_INVALID),
    ({"rope_theta": -1}, "rope_theta", E_INVALID),
    ({"rope_theta": 1e39}, "rope_theta", E_INVALID),  # f32 overflow: not finite
])
def test_config_errors(llrs, tmp_path, patch, match, code):
    d = {**QWEN25_7B, **patch}
    d = {k: v for k, v in d.items() if not (k in ("model_type", "hidden_size") and v is None)}
    with pytest.raises(llrs.LlrsError, match=match) as e:
        _cfg(llrs, tmp_path, d)
    assert e.value.code == code


def test_config_not_json(llrs, tmp_path):
    with pytest.raises(llrs.LlrsError) as e:
        _cfg(llrs, tmp_path, '{"model_type": "qwen2",}')
    assert e.value.code == E_FORMAT
    with pytest.raises(llrs.LlrsError, match="failed to read"):
        llrs.hf_config(tmp_path / "absent.json")


# -------------------------------------------------------- format detection

def test_format_detection(llrs, tmp_path):
    """ModelLoader::load (src/loader.rs:44-77)."""
    g = tmp_path / "a.gguf"
    g.write_bytes(b"GGUF")
    assert llrs.model_format(g) == ("gguf", str(g))
    st = tmp_path / "ckpt"
    st.mkdir()
    (st / "model-00001-of-00002.safetensors").write_bytes(b"")
    assert llrs.model_format(st / "model-00001-of-00002.safetensors") == ("safetensors", str(st))
    with pytest.raises(llrs.LlrsError, match="cannot detect model format"):
        llrs.model_format(st)  # shards without model.safetensors or an index
    (st / "model.safetensors.index.json").write_text("{}")
    assert llrs.model_format(st) == ("safetensors", str(st))
    (st / "x.gguf").write_bytes(b"GGUF")
    assert llrs.model_format(st) == ("safetensors", str(st))  # a checkpoint wins over GGUF
    d = tmp_path / "one"
    d.mkdir()
    (d / "m.gguf").write_bytes(b"GGUF")
    assert llrs.model_format(d) == ("gguf", str(d / "m.gguf"))
    (d / "n.gguf").write_bytes(b"GGUF")
    with pytest.raises(llrs.LlrsError, match="multiple GGUF files"):
        llrs.model_format(d)
    with pytest.raises(llrs.LlrsError, match="cannot detect model format"):
        llrs.model_format(tmp_path / "missing")
    (tmp_path / "w.bin").write_bytes(b"")
    with pytest.raises(llrs.LlrsError, match="cannot detect model format"):
        llrs.model_format(tmp_path / "w.bin")


def test_checkpoint_writer_round_trip(llrs, tmp_path):
    """The test checkpoints read back through the reader as written."""
    cfg = llrs.SynthConfig(hidden_size=64, intermediate_size=128, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=2, vocab_size=96,
                           max_position_embeddings=64, seed=5, tie_word_embeddings=False)
    stored = write_checkpoint(llrs, cfg, tmp_path / "ck", "BF16", shards=2)
    c = llrs.hf_config(tmp_path / "ck" / "config.json")
    assert (c.hidden_size, c.num_hidden_layers, c.vocab_size, c.tie_word_embeddings) == (64, 2, 96, False)
    assert len(stored) == 3 + 2 * 12
    for name in ("model.embed_tokens.weight", "model.layers.1.self_attn.k_proj.bias",
                 "model.layers.0.mlp.down_proj.weight"):
        ty, shape, data = llrs.safetensors_read_tensor(tmp_path / "ck", name)
        assert ty == llrs.QuantType.BF16 and shape == stored[name].shape
        widened = (np.frombuffer(data, np.uint16).astype(np.uint32) << 16).view(np.float32)
        np.testing.assert_array_equal(widened, stored[name].reshape(-1))


# ------------------------------------------------------------------- GPU

HF_RECIPE = {"embed_tokens": 8, "lm_head": 8, "v_proj": 8, "down_proj": 14}  # Q8_0 / Q6_K; else Q4_K


def _requested(name):
    for key, ty in HF_RECIPE.items():
        if key in name:
            return ty
    return 12


def _gguf_of(name):
    from hf_checkpoint import HF_LAYER, HF_NAMES
    inv = {v: k for k, v in HF_NAMES.items()}
    if name in inv:
        return inv[name]
    _, _, layer, rest = name.split(".", 3)
    return f"blk.{layer}." + {v: k for k, v in HF_LAYER.items()}[rest]


def _tiny(llrs, **kw):
    base = dict(hidden_size=256, intermediate_size=768, num_attention_heads=4, num_key_value_heads=2,
                num_hidden_layers=2, vocab_size=1000, max_position_embeddings=512, seed=23,
                tie_word_embeddings=False)
    base.update(kw)
    return llrs.SynthConfig(**base)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,shards", [("BF16", 1), ("F16", 3), ("F32", 1)])
def test_unquantized_load_keeps_the_bytes(llrs, backend, tmp_path, dtype, shards):
    cfg = _tiny(llrs)
    stored = write_checkpoint(llrs, cfg, tmp_path / "ck", dtype, shards=shards)
    model = llrs.ModelLoader.load(tmp_path / "ck", backend)
    print(f"[st] {dtype} x{shards} loaded", flush=True)
    assert model.config().tie_word_embeddings is False
    model.export_gguf(tmp_path / "out.gguf")
    for name, vals in stored.items():
        _, qt = llrs.gguf_read_tensor(tmp_path / "out.gguf", _gguf_of(name))
        if vals.ndim == 1:  # norms and biases: f32 on the device
            np.testing.assert_array_equal(np.frombuffer(qt.data, np.float32), vals, err_msg=name)
        else:
            assert qt.quant_type == llrs.QuantType[dtype]
            _, _, raw = llrs.safetensors_read_tensor(tmp_path / "ck", name)
            assert qt.data == raw, name


@pytest.mark.gpu
@pytest.mark.parametrize("recipe", ["Q4KM", "Q4K"])
def test_load_time_quantization_matches_host_quantizers(llrs, backend, tmp_path, recipe):
    cfg = _tiny(llrs, tie_word_embeddings=True)
    stored = write_checkpoint(llrs, cfg, tmp_path / "ck", "BF16",
                              drop=("model.layers.1.self_attn.k_proj.bias",))
    q = getattr(llrs.LoadQuantization, recipe)
    model = llrs.SafetensorsLoader.load(tmp_path / "ck", backend, q)
    assert model.config().tie_word_embeddings is True  # no lm_head.weight in the checkpoint
    model.export_gguf(tmp_path / "out.gguf")
    for name, vals in stored.items():
        _, qt = llrs.gguf_read_tensor(tmp_path / "out.gguf", _gguf_of(name))
        if vals.ndim == 1:
            np.testing.assert_array_equal(np.frombuffer(qt.data, np.float32), vals, err_msg=name)
            continue
        want_ty = _requested(name) if recipe == "Q4KM" else 12
        host = llrs.QuantTensor.quantize(want_ty, vals, *vals.shape)
        assert qt.quant_type == host.quant_type, name
        assert qt.data == host.data, name
    _, qt = llrs.gguf_read_tensor(tmp_path / "out.gguf", "blk.1.attn_k.bias")
    assert not np.frombuffer(qt.data, np.float32).any()  # a missing bias is zeros


@pytest.mark.gpu
def test_safetensors_model_greedy_parity(llrs, backend, oracle, tmp_path):
    """A BF16 checkpoint quantized at load (q4km) decodes the oracle's greedy
    tokens; the oracle reads the loaded tensors back from a GGUF export."""
    cfg = _tiny(llrs, num_hidden_layers=3, seed=29)
    write_checkpoint(llrs, cfg, tmp_path / "ck", "BF16", shards=2)
    model = llrs.ModelLoader.load(tmp_path / "ck" / "model-00001-of-00002.safetensors", backend,
                                  llrs.LoadQuantization.Q4KM)
    model.export_gguf(tmp_path / "out.gguf")
    om = oracle.load(tmp_path / "out.gguf")
    ctx = 96
    om.new_state(ctx)
    kv = llrs.KVCache(model, ctx)
    prompt = np.array([5, 77, 901, 13, 2, 640, 31, 8], np.uint32)
    model.prefill(prompt, 0, kv)
    om.prefill(prompt, 0)
    err = float(np.abs(kv.logits() - om.logits()).max())
    print(f"[st] prefill logits max-abs err {err:.3e}", flush=True)
    assert err <= 2e-2
    got = model.decode_greedy(len(prompt), 32, kv)
    want = om.decode_greedy(len(prompt), 32)
    np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
def test_safetensors_load_errors(llrs, backend, tmp_path):
    cfg = _tiny(llrs, num_hidden_layers=1)
    write_checkpoint(llrs, cfg, tmp_path / "a", "BF16", drop=("model.layers.0.mlp.up_proj.weight",))
    with pytest.raises(llrs.LlrsError, match="missing safetensors tensor model.layers.0.mlp.up_proj.weight"):
        llrs.ModelLoader.load(tmp_path / "a", backend)
    write_checkpoint(llrs, cfg, tmp_path / "b", "BF16")
    d = json.loads((tmp_path / "b" / "config.json").read_text())
    (tmp_path / "b" / "config.json").write_text(json.dumps({**d, "intermediate_size": 512}))
    with pytest.raises(llrs.LlrsError, match=r"mlp.gate_proj.weight has shape \[768, 256\], expected \[512, 256\]"):
        llrs.ModelLoader.load(tmp_path / "b", backend)
    with pytest.raises(llrs.LlrsError, match="unknown quantization"):
        llrs.SafetensorsLoader.load(tmp_path / "b", backend, 7)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["BF16", "F16"])
def test_gguf_half_matrices_quantize_like_safetensors(llrs, backend, tmp_path, dtype):
    """GgufLoader's maybe_quantize on F16/BF16 matrices (src/loader.rs:406-447)
    takes the same device path (raw upload, widen, encode): a GGUF file with
    the checkpoint's half-precision matrices, loaded with q4km, holds the
    same bytes as the checkpoint loaded with q4km."""
    cfg = _tiny(llrs, num_hidden_layers=1, seed=31)
    write_checkpoint(llrs, cfg, tmp_path / "ck", dtype)
    half = llrs.SafetensorsLoader.load(tmp_path / "ck", backend)
    half.export_gguf(tmp_path / "half.gguf")  # F16/BF16 matrices, f32 vectors
    _, qt = llrs.gguf_read_tensor(tmp_path / "half.gguf", "blk.0.ffn_up.weight")
    assert qt.quant_type == llrs.QuantType[dtype]
    a = llrs.GgufLoader.load(tmp_path / "half.gguf", backend, llrs.LoadQuantization.Q4KM)
    b = llrs.SafetensorsLoader.load(tmp_path / "ck", backend, llrs.LoadQuantization.Q4KM)
    a.export_gguf(tmp_path / "a.gguf")
    b.export_gguf(tmp_path / "b.gguf")
    for g in ("token_embd.weight", "output.weight", "blk.0.attn_q.weight", "blk.0.attn_v.weight",
              "blk.0.ffn_down.weight", "blk.0.ffn_gate.weight", "blk.0.attn_norm.weight"):
        _, x = llrs.gguf_read_tensor(tmp_path / "a.gguf", g)
        _, y = llrs.gguf_read_tensor(tmp_path / "b.gguf", g)
        assert (x.quant_type, x.data) == (y.quant_type, y.data), g


def test_header_json_escapes_and_nesting(llrs, tmp_path):
    """The header's JSON strings decode escapes (\\u, surrogate pairs) to the
    UTF-8 names they stand for, as the package reads them; nesting beyond
    the parser's limit is rejected by both."""
    f4 = struct.pack("<4f", 1, 2, 3, 4)
    hdr = b'{"t\\u00e9\\ud83d\\ude00\\n": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}'
    path = tmp_path / "model.safetensors"
    path.write_bytes(raw_file(hdr, f4))
    import safetensors.numpy
    assert list(safetensors.numpy.load_file(str(path))) == ["té\U0001F600\n"]
    assert llrs.safetensors_read_tensor(tmp_path, "té\U0001F600\n")[2] == f4
    deep = b'{"__metadata__": {"a": "b"}, "x": ' + b"[" * 200 + b"]" * 200 + b"}"
    path.write_bytes(raw_file(deep))
    assert _pkg_rejects(path)
    with pytest.raises(llrs.LlrsError) as e:
        llrs.safetensors_read_tensor(tmp_path, "x")
    assert e.value.code == E_FORMAT
