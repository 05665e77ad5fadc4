"""GPU-side generation and load-time quantization produce the host's bytes (MI355X).

The encoders (src/quant.rs:650-967 restated) and the synthetic RNG are shared
host/device code built without FP contraction; these tests hold the two
builds to bit-identical output.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def small_cfg(llrs, recipe, **kw):
    base = dict(hidden_size=512, intermediate_size=1280, num_attention_heads=8,
                num_key_value_heads=2, num_hidden_layers=2, vocab_size=700,
                max_position_embeddings=256, recipe=recipe, seed=21, tie_word_embeddings=False)
    base.update(kw)
    return llrs.SynthConfig(**base)


@pytest.mark.parametrize("recipe", ["Q4KM", "Q4K", "NONE"])
def test_gpu_synthetic_model_equals_host_gguf(llrs, backend, tmp_path, recipe):
    cfg = small_cfg(llrs, getattr(llrs.LoadQuantization, recipe))
    host = tmp_path / "host.gguf"
    cfg.write_gguf(host)
    model = llrs.HipQwen2Model.synthetic(backend, cfg)
    dev = tmp_path / "dev.gguf"
    model.export_gguf(dev)
    names = ["token_embd.weight", "output.weight", "output_norm.weight"]
    for i in range(cfg.num_hidden_layers):
        names += [f"blk.{i}.{n}" for n in ("attn_norm.weight", "attn_q.weight", "attn_q.bias",
                                           "attn_k.weight", "attn_k.bias", "attn_v.weight",
                                           "attn_v.bias", "attn_output.weight", "ffn_norm.weight",
                                           "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight")]
    for name in names:
        _, a = llrs.gguf_read_tensor(host, name)
        _, b = llrs.gguf_read_tensor(dev, name)
        assert a.quant_type == b.quant_type and a.shape == b.shape, name
        assert a.data == b.data, name


def test_gpu_load_time_quantization_matches_host_quantizer(llrs, backend, oracle, tmp_path):
    """maybe_quantize (src/loader.rs:406-447) on an F32 GGUF: the GPU encoders emit
    exactly the host quantizer's blocks for every recipe type."""
    cfg = small_cfg(llrs, llrs.LoadQuantization.NONE, hidden_size=768, intermediate_size=1536,
                    num_attention_heads=6)
    f32 = tmp_path / "f32.gguf"
    cfg.write_gguf(f32)
    QT = llrs.QuantType
    for quant, expect in ((llrs.LoadQuantization.Q4KM,
                           {"blk.0.attn_q.weight": QT.Q4K, "blk.0.attn_v.weight": QT.Q8_0,
                            "blk.1.ffn_down.weight": QT.Q6K, "token_embd.weight": QT.Q8_0}),
                          (llrs.LoadQuantization.Q4K,
                           {"blk.0.ffn_up.weight": QT.Q4K, "output.weight": QT.Q4K})):
        model = llrs.ModelLoader.load_dynamic(f32, backend, quant)
        out = tmp_path / f"q{int(quant)}.gguf"
        model.export_gguf(out)
        for name, qt in expect.items():
            _, src = llrs.gguf_read_tensor(f32, name)
            vals = np.frombuffer(src.data, np.float32)
            want = llrs.QuantTensor.quantize(qt, vals, src.shape[0], src.shape[1])
            _, got = llrs.gguf_read_tensor(out, name)
            assert got.quant_type == want.quant_type == qt, name
            assert got.data == want.data, name


def test_q5_0_fallback_rows_on_gpu(llrs, backend, tmp_path):
    """Rows of 896 (not a multiple of 256) fall back to Q5_0 in the GPU encoder too."""
    cfg = small_cfg(llrs, llrs.LoadQuantization.NONE, hidden_size=896, num_attention_heads=14,
                    intermediate_size=1024, num_hidden_layers=1)
    f32 = tmp_path / "f.gguf"
    cfg.write_gguf(f32)
    model = llrs.ModelLoader.load_dynamic(f32, backend, llrs.LoadQuantization.Q4K)
    out = tmp_path / "o.gguf"
    model.export_gguf(out)
    _, src = llrs.gguf_read_tensor(f32, "blk.0.ffn_gate.weight")
    want = llrs.QuantTensor.quantize(llrs.QuantType.Q4K, np.frombuffer(src.data, np.float32),
                                     src.shape[0], src.shape[1])
    _, got = llrs.gguf_read_tensor(out, "blk.0.ffn_gate.weight")
    assert want.quant_type == got.quant_type == llrs.QuantType.Q5_0
    assert got.data == want.data
