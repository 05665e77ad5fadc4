"""Decode of models whose every matrix has one of the block types outside the
q4km/q4k recipes (Q4_0, Q4_1, Q5_1, Q5_K), against the oracle: these types
run the tuned digit GEMV in every fused form the decode step uses (Q/K/V as
one three-segment launch with bias, gate/up with SiLU*up, o and down with the
residual, the LM head with the argmax), on the launch-per-phase path.

The GGUF files hold the synthetic F32 model's weights encoded by
tests/simple_quant.py (GgufLoader keeps quantized tensors as they are,
src/loader.rs:437-441).  Bars: logits <= 2e-2 max-abs after the prefill and
after 16 greedy steps, identical tokens; and the generic wave-per-row GEMV
(LLRS_GENERIC_GEMV=1) decodes the same tokens, its logits differing from the
tuned path's (a different kernel ran) by less than the bar.
"""
from __future__ import annotations

import numpy as np
import pytest

import simple_quant

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
TYPES = {"Q4_0": 2, "Q4_1": 3, "Q5_1": 7, "Q5_K": 13}


def write_typed_model(llrs, tmp_path, cfg, ty):
    from gguf_write import qwen2_metadata, write_gguf
    from hf_checkpoint import gguf_names
    f32 = tmp_path / "f32.gguf"
    llrs.SynthConfig(**{**cfg.__dict__, "recipe": llrs.LoadQuantization.NONE}).write_gguf(f32)
    tensors = []
    for name in gguf_names(cfg.num_hidden_layers, tied=False):
        _, t = llrs.gguf_read_tensor(f32, name)
        rows, cols = t.shape if len(t.shape) == 2 else (1, t.shape[0])
        vals = np.frombuffer(t.data, np.float32)
        if name.endswith(".weight") and rows > 1:
            tensors.append((name, ty, rows, cols, simple_quant.ENCODERS[ty](vals)))
        else:
            tensors.append((name, 0, rows, cols, bytes(t.data)))
    path = tmp_path / f"typed_{ty}.gguf"
    write_gguf(path, qwen2_metadata(cfg), tensors)
    return path


@pytest.mark.parametrize("name", list(TYPES))
def test_decode_with_type(llrs, backend, oracle, tmp_path, monkeypatch, name):
    ty = TYPES[name]
    cfg = llrs.SynthConfig(hidden_size=256, intermediate_size=768, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=2, vocab_size=1024,
                           max_position_embeddings=512, recipe=llrs.LoadQuantization.NONE,
                           seed=71 + ty, tie_word_embeddings=False)
    path = write_typed_model(llrs, tmp_path, cfg, ty)
    assert int(llrs.gguf_read_tensor(path, "blk.0.ffn_gate.weight")[1].quant_type) == ty
    model = llrs.ModelLoader.load_dynamic(path, backend)
    om = oracle.load(path)
    prompt = np.random.default_rng(ty).integers(0, cfg.vocab_size, 20).astype(np.uint32)
    ctx = 64
    kv = llrs.KVCache(model, ctx)
    assert not kv.persistent  # no persistent instantiation for these types
    om.new_state(ctx)
    model.prefill(prompt, 0, kv)
    om.prefill(prompt, 0)
    err = float(np.abs(kv.logits() - om.logits()).max())
    print(f"[types] {name} prefill logits err {err:.2e}", flush=True)
    assert err <= LOGIT_TOL
    got = model.decode_greedy(len(prompt), 16, kv)
    want = om.decode_greedy(len(prompt), 16)
    np.testing.assert_array_equal(got, want)
    tuned = kv.logits().copy()
    err = float(np.abs(tuned - om.logits()).max())
    print(f"[types] {name} tokens {got[:6].tolist()} logits err {err:.2e}", flush=True)
    assert err <= LOGIT_TOL

    monkeypatch.setenv("LLRS_GENERIC_GEMV", "1")
    kv_g = llrs.KVCache(model, ctx)
    model.prefill(prompt, 0, kv_g)
    np.testing.assert_array_equal(model.decode_greedy(len(prompt), 16, kv_g), got)
    diff = float(np.abs(kv_g.logits() - tuned).max())
    print(f"[types] {name} generic vs tuned logits diff {diff:.2e}", flush=True)
    assert 0 < diff <= LOGIT_TOL
