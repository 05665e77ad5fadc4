"""Hugging Face Qwen2 checkpoint directories for the SafeTensors loader tests.

A synthetic model is written as an F32 GGUF file (llrs_synth_write_gguf with
recipe NONE), its tensors are renamed to the Hugging Face names that
SafetensorsLoader::load reads (src/loader.rs:102-213), cast to the requested
dtype and written with the `safetensors` package, an implementation of the
format independent of the one under test.
"""
from __future__ import annotations

import json
import pathlib

import numpy as np

HF_NAMES = {
    "token_embd.weight": "model.embed_tokens.weight",
    "output_norm.weight": "model.norm.weight",
    "output.weight": "lm_head.weight",
}
HF_LAYER = {
    "attn_norm.weight": "input_layernorm.weight",
    "ffn_norm.weight": "post_attention_layernorm.weight",
    "attn_q.weight": "self_attn.q_proj.weight",
    "attn_q.bias": "self_attn.q_proj.bias",
    "attn_k.weight": "self_attn.k_proj.weight",
    "attn_k.bias": "self_attn.k_proj.bias",
    "attn_v.weight": "self_attn.v_proj.weight",
    "attn_v.bias": "self_attn.v_proj.bias",
    "attn_output.weight": "self_attn.o_proj.weight",
    "ffn_gate.weight": "mlp.gate_proj.weight",
    "ffn_up.weight": "mlp.up_proj.weight",
    "ffn_down.weight": "mlp.down_proj.weight",
}


def gguf_names(n_layers: int, tied: bool) -> list[str]:
    names = ["token_embd.weight", "output_norm.weight"] + ([] if tied else ["output.weight"])
    for i in range(n_layers):
        names += [f"blk.{i}.{k}" for k in HF_LAYER]
    return names


def hf_name(g: str) -> str:
    if g in HF_NAMES:
        return HF_NAMES[g]
    _, layer, rest = g.split(".", 2)
    return f"model.layers.{layer}.{HF_LAYER[rest]}"


def to_dtype(values: np.ndarray, dtype: str):
    """(array for safetensors.numpy / torch tensor, f32 values the file holds)."""
    if dtype == "F32":
        return values.astype(np.float32), values.astype(np.float32)
    if dtype == "F16":
        h = values.astype(np.float16)
        return h, h.astype(np.float32)
    import torch
    t = torch.from_numpy(values.astype(np.float32)).to(torch.bfloat16)
    back = t.to(torch.float32).numpy()
    return t, back


def write_checkpoint(llrs, cfg, out_dir: pathlib.Path, dtype: str = "BF16", shards: int = 1,
                     drop: tuple = ()) -> dict:
    """Writes config.json + safetensors shard(s) for SynthConfig `cfg`; returns
    {hf name: f32 values as stored (after the dtype cast)}."""
    import safetensors.numpy
    import safetensors.torch

    out_dir = pathlib.Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    src = out_dir.parent / (out_dir.name + "_src.gguf")
    f32cfg = type(cfg)(**{**cfg.__dict__, "recipe": llrs.LoadQuantization.NONE})
    f32cfg.write_gguf(src)
    stored, tensors = {}, {}
    for g in gguf_names(cfg.num_hidden_layers, cfg.tie_word_embeddings):
        _, qt = llrs.gguf_read_tensor(src, g)
        v = np.frombuffer(qt.data, dtype=np.float32)
        shape = qt.shape if not g.endswith(("norm.weight", ".bias")) else (qt.shape[-1],)
        arr, back = to_dtype(v.reshape(shape), dtype)
        name = hf_name(g)
        if name in drop:
            continue
        tensors[name] = arr
        stored[name] = back
    src.unlink()
    save = safetensors.torch.save_file if dtype == "BF16" else safetensors.numpy.save_file
    if shards == 1:
        save(tensors, str(out_dir / "model.safetensors"), metadata={"format": "pt"})
    else:
        names = sorted(tensors)
        weight_map = {}
        for s in range(shards):
            part = names[s::shards]
            fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            save({n: tensors[n] for n in part}, str(out_dir / fname), metadata={"format": "pt"})
            weight_map.update({n: fname for n in part})
        (out_dir / "model.safetensors.index.json").write_text(
            json.dumps({"metadata": {"total_size": 0}, "weight_map": weight_map}))
    config = {
        "architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2",
        "hidden_size": cfg.hidden_size, "intermediate_size": cfg.intermediate_size,
        "num_attention_heads": cfg.num_attention_heads,
        "num_key_value_heads": cfg.num_key_value_heads,
        "num_hidden_layers": cfg.num_hidden_layers, "vocab_size": cfg.vocab_size,
        "max_position_embeddings": cfg.max_position_embeddings,
        "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
        "tie_word_embeddings": cfg.tie_word_embeddings, "torch_dtype": "bfloat16",
    }
    (out_dir / "config.json").write_text(json.dumps(config, indent=2))
    return stored
