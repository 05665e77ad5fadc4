"""Model-level mirror of the reference's CausalModel boundary over the C ABI.

    ModelLoader.load_dynamic(path, LoadOptions)   src/loader.rs:37-77
    GgufLoader / SafetensorsLoader .load          src/loader.rs:80-399
    HipQwen2Model.forward_token / prefill         src/architecture.rs:47-77
    KVCache (device-resident, + InferenceBuffers) src/cache.rs:4-101
    InferenceEngine.benchmark_tokens              src/engine.rs:189-223
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field

import numpy as np

from . import (F32P, HipBackend, LlrsError, LoadQuantization, LogitsMode, _check, _f32, _Generation,
               _ModelConfig, _Sampling, _SynthConfig, lib, P, SZ, U32P)


@dataclass
class SamplingOptions:
    """EngineOptions' sampling fields and their defaults (src/engine.rs:14-31)."""
    temperature: float = 0.7
    top_p: float = 0.9
    top_k: int = 40
    repetition_penalty: float = 1.1


class Sampler:
    """The engine's sampling state (src/engine.rs:36-90, 243-251): the options
    and the window of the last `repeat_last_n` tokens the penalty applies to."""

    def __init__(self, opts: SamplingOptions | None = None, repeat_last_n: int = 64):
        self.opts = opts or SamplingOptions()
        self.max_repeat_window = repeat_last_n
        self.recent_tokens: list[int] = []

    def remember(self, token: int) -> None:
        if self.max_repeat_window == 0:
            return
        self.recent_tokens.append(int(token))
        if len(self.recent_tokens) > self.max_repeat_window:
            self.recent_tokens.pop(0)

    def sample(self, kv: "KVCache", uniform: float) -> int:
        return kv.sample(self.opts, uniform, self.recent_tokens)


@dataclass
class LlamaConfig:
    """config::LlamaConfig (src/config.rs:18-55) as loaded onto the device."""
    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    num_hidden_layers: int
    vocab_size: int
    max_position_embeddings: int
    head_dim: int
    kv_width: int
    rms_norm_eps: float
    rope_theta: float
    tie_word_embeddings: bool


def _config_from_c(c: _ModelConfig) -> LlamaConfig:
    return LlamaConfig(c.hidden_size, c.intermediate_size, c.num_attention_heads,
                       c.num_key_value_heads, c.num_hidden_layers, c.vocab_size,
                       c.max_position_embeddings, c.head_dim, c.kv_width, c.rms_norm_eps,
                       c.rope_theta, bool(c.tie_word_embeddings))


def hf_config(config_json_path) -> LlamaConfig:
    """LlamaConfig::from_json + validate (src/config.rs:17-90) of a Qwen2
    config.json (model_type checked as src/loader.rs:85-97 does)."""
    c = _ModelConfig()
    _check(lib().llrs_hf_config_read(str(config_json_path).encode(), C.byref(c)))
    return _config_from_c(c)


@dataclass
class SynthConfig:
    """A synthetic Qwen2 model: shape, recipe and seed (llrs_synth_config)."""
    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    num_hidden_layers: int
    vocab_size: int
    max_position_embeddings: int = 32768
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = True
    recipe: LoadQuantization = LoadQuantization.Q4KM
    seed: int = 0
    weight_std: float = 0.02
    threads: int = 0

    def _c(self) -> _SynthConfig:
        return _SynthConfig(self.hidden_size, self.intermediate_size, self.num_attention_heads,
                            self.num_key_value_heads, self.num_hidden_layers, self.vocab_size,
                            self.max_position_embeddings, self.rms_norm_eps, self.rope_theta,
                            int(self.tie_word_embeddings), int(self.recipe), self.seed,
                            self.weight_std, self.threads)

    def write_gguf(self, path: str) -> None:
        """Writes the model as a pre-quantized GGUF v3 file."""
        _check(lib().llrs_synth_write_gguf(C.byref(self._c()), str(path).encode()))


class HipQwen2Model:
    """architecture::CausalModel for Qwen2 on the GPU."""

    def __init__(self, backend: HipBackend, handle):
        self._backend = backend
        self.handle = handle
        self._free = lib().llrs_model_free
        c = _ModelConfig()
        _check(lib().llrs_model_config_get(handle, C.byref(c)))
        self._config = _config_from_c(c)

    @classmethod
    def synthetic(cls, backend: HipBackend, cfg: SynthConfig) -> "HipQwen2Model":
        h = P()
        _check(lib().llrs_model_synthetic(backend.handle, C.byref(cfg._c()), C.byref(h)))
        return cls(backend, h)

    def architecture(self) -> str:
        return "qwen2"

    def config(self) -> LlamaConfig:
        return self._config

    def backend(self) -> HipBackend:
        return self._backend

    def export_gguf(self, path) -> None:
        """Writes the device model to a GGUF v3 file (native block bytes)."""
        _check(lib().llrs_model_export_gguf(self.handle, str(path).encode()))

    def weight_bytes(self) -> int:
        return int(lib().llrs_model_weight_bytes(self.handle))

    def forward_token(self, token_id: int, pos: int, kv_cache: "KVCache",
                      logits: LogitsMode = LogitsMode.COMPUTE) -> None:
        _check(lib().llrs_forward_token(self.handle, kv_cache.handle, token_id, pos, int(logits)))

    def prefill(self, tokens, start_pos: int, kv_cache: "KVCache") -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        _check(lib().llrs_prefill(self.handle, kv_cache.handle, t.ctypes.data_as(U32P), t.size,
                                  start_pos))

    def decode_greedy(self, start_pos: int, n_steps: int, kv_cache: "KVCache") -> np.ndarray:
        out = np.zeros(max(n_steps, 1), dtype=np.uint32)
        _check(lib().llrs_decode_greedy(self.handle, kv_cache.handle, start_pos, n_steps,
                                        out.ctypes.data_as(U32P)))
        return out[:n_steps]

    # Launch groups of the decode step: fused Q/K/V (+RMSNorm), O (+residual),
    # gate/up (+RMSNorm, SiLU*up), down (+residual), LM head (+RMSNorm, argmax).
    PROJECTIONS = ("qkv", "o", "gate_up", "down", "lm_head")

    def profile_projection(self, kv_cache: "KVCache", which: str, iters: int = 10):
        """(mean launch time in us, bytes per launch) of one projection's decode-step
        launch, timed with HIP events on the backend's stream."""
        us, nb = C.c_double(), SZ()
        _check(lib().llrs_profile_projection(self.handle, kv_cache.handle,
                                             self.PROJECTIONS.index(which), iters, C.byref(us),
                                             C.byref(nb)))
        return us.value, nb.value

    def profile_layers(self, kv_cache: "KVCache", iters: int = 10):
        """(mean time in us, weight bytes) of every layer of one decode step: the
        persistent kernel when kv_cache.persistent, else the per-phase launches."""
        us, nb = C.c_double(), SZ()
        _check(lib().llrs_profile_projection(self.handle, kv_cache.handle, len(self.PROJECTIONS),
                                             iters, C.byref(us), C.byref(nb)))
        return us.value, nb.value

    def __del__(self):
        # Caches hold their own reference to the model on the C side, so the
        # finalizers may run in any order (at interpreter shutdown too).
        h, free = getattr(self, "handle", None), getattr(self, "_free", None)
        if h and free is not None:
            free(h)
            self.handle = None


class KVCache:
    """cache::KVCache + InferenceBuffers, resident in HBM."""

    def __init__(self, model: HipQwen2Model, max_seq_len: int):
        h = P()
        _check(lib().llrs_kv_create(model.handle, max_seq_len, C.byref(h)))
        self.handle = h
        self._free = lib().llrs_kv_free
        self.model = model
        self.max_seq_len = max_seq_len

    def reset(self) -> None:
        _check(lib().llrs_kv_reset(self.handle))

    @property
    def persistent(self) -> bool:
        """Whether decode steps run as one persistent launch for all layers."""
        return lib().llrs_kv_decode_path(self.handle) == 1

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.config().vocab_size, dtype=np.float32)
        _check(lib().llrs_read_logits(self.handle, _f32(out), out.size))
        return out

    def argmax(self) -> int:
        t = C.c_uint32()
        _check(lib().llrs_argmax(self.handle, C.byref(t)))
        return int(t.value)

    def sample(self, opts: "SamplingOptions", uniform: float, recent=()) -> int:
        """sample_current_logits (src/engine.rs:253-325) on the device with the
        caller's uniform draw in [0, 1); `recent` is the repeat window."""
        r = np.ascontiguousarray(np.asarray(recent, dtype=np.uint32))
        o = _Sampling(opts.temperature, opts.top_p, opts.top_k, opts.repetition_penalty)
        t = C.c_uint32()
        _check(lib().llrs_sample(self.handle, C.byref(o), r.ctypes.data_as(P) if r.size else None,
                                 r.size, float(uniform), C.byref(t)))
        return int(t.value)

    def tokens(self, start: int, n: int) -> np.ndarray:
        """The device's token ids for positions [start, start + n) (position
        p + 1 holds the greedy token of the logits computed at p)."""
        out = np.zeros(max(n, 1), dtype=np.uint32)
        _check(lib().llrs_read_tokens(self.handle, start, n, out.ctypes.data_as(U32P)))
        return out[:n]

    def layer(self, layer: int, which: str, n_pos: int) -> np.ndarray:
        cfg = self.model.config()
        out = np.empty(n_pos * cfg.kv_width, dtype=np.float32)
        _check(lib().llrs_read_kv(self.handle, layer, 0 if which == "k" else 1, _f32(out),
                                  out.size))
        return out.reshape(n_pos, cfg.kv_width)

    def __del__(self):
        h, free = getattr(self, "handle", None), getattr(self, "_free", None)
        if h and free is not None:
            free(h)
            self.handle = None


class ModelLoader:
    """loader::ModelLoader (src/loader.rs:33-78): a .gguf file, a .safetensors
    file (its directory), or a directory with a Hugging Face checkpoint or
    exactly one .gguf file."""

    @staticmethod
    def load(path, backend: HipBackend,
             quantization: LoadQuantization = LoadQuantization.NONE) -> HipQwen2Model:
        h = P()
        _check(lib().llrs_model_load(backend.handle, str(path).encode(), int(quantization),
                                     C.byref(h)))
        return HipQwen2Model(backend, h)

    load_dynamic = load


class GgufLoader:
    """loader::GgufLoader (src/loader.rs:230-399)."""

    @staticmethod
    def load(path, backend: HipBackend,
             quantization: LoadQuantization = LoadQuantization.NONE) -> HipQwen2Model:
        h = P()
        _check(lib().llrs_model_load_gguf(backend.handle, str(path).encode(), int(quantization),
                                          C.byref(h)))
        return HipQwen2Model(backend, h)


class SafetensorsLoader:
    """loader::SafetensorsLoader (src/loader.rs:80-228): config.json plus
    model.safetensors or the shards named by model.safetensors.index.json."""

    @staticmethod
    def load(model_dir, backend: HipBackend,
             quantization: LoadQuantization = LoadQuantization.NONE) -> HipQwen2Model:
        h = P()
        _check(lib().llrs_model_load_safetensors(backend.handle, str(model_dir).encode(),
                                                 int(quantization), C.byref(h)))
        return HipQwen2Model(backend, h)


@dataclass
class InferenceMetrics:
    """benchmark::InferenceMetrics (src/benchmark.rs:3-34)."""
    prompt_tokens: int = 0
    generated_tokens: int = 0
    prefill_s: float = 0.0
    decode_s: float = 0.0
    tokens: list = field(default_factory=list)

    def prefill_tokens_per_second(self) -> float:
        return self.prompt_tokens / self.prefill_s if self.prefill_s > 0 else 0.0

    def decode_tokens_per_second(self) -> float:
        return self.generated_tokens / self.decode_s if self.decode_s > 0 else 0.0


def find_eos_tokens(model_path) -> list[int]:
    """find_eos_tokens (src/engine.rs:340-387): generation_config.json's
    eos_token_id and the ids of <|im_end|> / <|endoftext|> in tokenizer.json."""
    n = SZ()
    _check(lib().llrs_find_eos_tokens(str(model_path).encode(), None, 0, C.byref(n)))
    out = np.zeros(max(n.value, 1), dtype=np.uint32)
    _check(lib().llrs_find_eos_tokens(str(model_path).encode(), out.ctypes.data_as(U32P), out.size,
                                      C.byref(n)))
    return [int(t) for t in out[:n.value]]


@dataclass
class GenerationOutput:
    """benchmark::GenerationOutput without the text (src/benchmark.rs): the
    generated ids and the metrics."""
    token_ids: list
    metrics: InferenceMetrics
    stopped_on_eos: bool


class InferenceEngine:
    """engine::InferenceEngine on token ids (src/engine.rs:36-241): the
    benchmark loop and the generation loop; the tokenizer stays with the
    caller (pass its ids, and the EOS ids from find_eos_tokens)."""

    def __init__(self, model: HipQwen2Model, context_length: int = 4096,
                 sampling: "SamplingOptions | None" = None, repeat_last_n: int = 64,
                 eos_token_ids=()):
        ctx = min(context_length, model.config().max_position_embeddings)
        if ctx <= 0:
            raise LlrsError(-1, "context length must be positive")
        self.model = model
        self.kv_cache = KVCache(model, ctx)
        self.sampling = sampling or SamplingOptions()
        self.max_repeat_window = repeat_last_n
        self.eos_token_ids = [int(t) for t in eos_token_ids]

    def generate_with_metrics(self, prompt_tokens, max_new_tokens: int, uniforms=None) -> GenerationOutput:
        """generate_with_metrics (src/engine.rs:115-186) on ids: `uniforms` are
        the sampler's draws in [0, 1), one per generated token (the reference
        takes them from rand::thread_rng); None draws them with numpy."""
        prompt = np.ascontiguousarray(prompt_tokens, dtype=np.uint32)
        if uniforms is None:
            # float32 draws in [0, 1): a float64 draw above 1 - 2^-25 would
            # round to 1.0f, which the sampler rejects.
            uniforms = np.random.default_rng().random(max(max_new_tokens, 1), dtype=np.float32)
        u = np.ascontiguousarray(uniforms, dtype=np.float32)
        if u.size < max_new_tokens:
            raise LlrsError(-1, "one uniform draw per generated token is needed")
        eos = np.ascontiguousarray(self.eos_token_ids, dtype=np.uint32)
        out = np.zeros(max(max_new_tokens, 1), dtype=np.uint32)
        o = self.sampling
        opts = _Sampling(o.temperature, o.top_p, o.top_k, o.repetition_penalty)
        res = _Generation()
        _check(lib().llrs_generate(self.model.handle, self.kv_cache.handle,
                                   prompt.ctypes.data_as(U32P) if prompt.size else None, prompt.size,
                                   C.byref(opts), self.max_repeat_window,
                                   eos.ctypes.data_as(U32P) if eos.size else None, eos.size,
                                   max_new_tokens, u.ctypes.data_as(F32P), out.ctypes.data_as(U32P),
                                   C.byref(res)))
        toks = [int(t) for t in out[:res.generated_tokens]]
        m = InferenceMetrics(res.prompt_tokens, res.generated_tokens, res.prefill_ms / 1e3,
                             res.decode_ms / 1e3, toks)
        return GenerationOutput(toks, m, bool(res.stopped_on_eos))

    def benchmark_tokens(self, prompt_tokens, decode_tokens: int) -> InferenceMetrics:
        prompt = np.ascontiguousarray(prompt_tokens, dtype=np.uint32)
        if prompt.size == 0:
            raise LlrsError(-1, "benchmark prompt is empty")
        if prompt.size + decode_tokens > self.kv_cache.max_seq_len:
            raise LlrsError(-1, "benchmark token counts exceed context")
        self.kv_cache.reset()
        t0 = time.perf_counter()
        self.model.prefill(prompt, 0, self.kv_cache)
        t1 = time.perf_counter()
        toks = self.model.decode_greedy(prompt.size, decode_tokens, self.kv_cache)
        t2 = time.perf_counter()
        return InferenceMetrics(prompt.size, decode_tokens, t1 - t0, t2 - t1, list(toks))
