"""Python mirror of llama.rs's kernel and model boundaries over the HIP C ABI.

The product is libllrs_hip.so (HIP kernels for gfx950 + C++ host code behind
include/llrs.h).  This module binds it with ctypes and mirrors the
reference's Rust interface names so callers and tests read like the
reference's own code:

    KernelBackend / HipBackend   backend::KernelBackend (src/backend.rs:67-73)
    QuantType, QuantTensor       quant::{QuantType, QuantTensor} (src/quant.rs:10-324)
    LlamaConfig                  config::LlamaConfig (src/config.rs:18-55)
    HipQwen2Model                architecture::CausalModel for Qwen2
                                 (src/architecture.rs:42-78, src/model.rs:276-296)
    KVCache                      cache::KVCache + InferenceBuffers (src/cache.rs)
    ModelLoader.load_dynamic     loader::ModelLoader::load_dynamic (src/loader.rs:37-42)

Errors raise LlrsError (the reference returns anyhow::Error).  There is no CPU
fallback: if the library is missing or the GPU is absent, calls fail loudly.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
import pathlib
from dataclasses import dataclass

import numpy as np

PKG_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libllrs_hip.so"
HEADER = PKG_DIR.parent / "include" / "llrs.h"


class LlrsError(RuntimeError):
    """A failed call into libllrs_hip.so (negative status + message)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"llrs error {code}: {message}")
        self.code = code


_lib = None


def lib() -> C.CDLL:
    """Loads libllrs_hip.so (built by build.py); raises if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python llama.rs_amd/build.py` "
                "(there is no CPU fallback)")
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


class _BackendConfig(C.Structure):
    _fields_ = [("device", C.c_int), ("flags", C.c_uint32)]


class _ModelConfig(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in (
        "hidden_size", "intermediate_size", "num_attention_heads", "num_key_value_heads",
        "num_hidden_layers", "vocab_size", "max_position_embeddings", "head_dim", "kv_width")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("tie_word_embeddings", C.c_int)]


class _Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("repetition_penalty", C.c_float)]


class _Generation(C.Structure):
    _fields_ = [("prompt_tokens", C.c_size_t), ("generated_tokens", C.c_size_t),
                ("prefill_ms", C.c_double), ("decode_ms", C.c_double), ("stopped_on_eos", C.c_int)]


class _SynthConfig(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in (
        "hidden_size", "intermediate_size", "num_attention_heads", "num_key_value_heads",
        "num_hidden_layers", "vocab_size", "max_position_embeddings")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("tie_word_embeddings", C.c_int),
        ("recipe", C.c_int), ("seed", C.c_uint64), ("weight_std", C.c_float),
        ("threads", C.c_int)]


P = C.c_void_p
SZ = C.c_size_t
F32P = C.POINTER(C.c_float)
U32P = C.POINTER(C.c_uint32)

# (name, restype, argtypes) for every entry point in include/llrs.h.
SIGNATURES = [
    ("llrs_last_error", C.c_char_p, []),
    ("llrs_backend_create", C.c_int, [C.POINTER(_BackendConfig), C.POINTER(P)]),
    ("llrs_backend_destroy", None, [P]),
    ("llrs_backend_name", C.c_char_p, [P]),
    ("llrs_backend_threads", SZ, [P]),
    ("llrs_backend_synchronize", C.c_int, [P]),
    ("llrs_tensor_upload", C.c_int, [P, P, SZ, C.c_uint32, SZ, SZ, C.POINTER(P)]),
    ("llrs_tensor_free", None, [P]),
    ("llrs_tensor_info", C.c_int, [P, U32P, C.POINTER(SZ), C.POINTER(SZ), C.POINTER(SZ)]),
    ("llrs_tensor_download", C.c_int, [P, P, SZ]),
    ("llrs_matvec", C.c_int, [P, P, F32P, SZ, F32P, SZ]),
    ("llrs_matvec_dev", C.c_int, [P, P, P, P]),
    ("llrs_dequant_row", C.c_int, [P, P, SZ, F32P, SZ]),
    ("llrs_device_alloc", C.c_int, [P, SZ, C.POINTER(P)]),
    ("llrs_device_free", C.c_int, [P, P]),
    ("llrs_copy_h2d", C.c_int, [P, P, P, SZ]),
    ("llrs_copy_d2h", C.c_int, [P, P, P, SZ]),
    ("llrs_device_copy", C.c_int, [P, P, P, SZ]),
    ("llrs_quantize", C.c_int, [C.c_uint32, F32P, SZ, SZ, P, SZ, C.POINTER(SZ), U32P]),
    ("llrs_gguf_read_tensor", C.c_int, [C.c_char_p, C.c_char_p, U32P, U32P, C.POINTER(SZ),
                                        C.POINTER(SZ), P, SZ, C.POINTER(SZ)]),
    ("llrs_model_load_gguf", C.c_int, [P, C.c_char_p, C.c_int, C.POINTER(P)]),
    ("llrs_model_load_safetensors", C.c_int, [P, C.c_char_p, C.c_int, C.POINTER(P)]),
    ("llrs_model_load", C.c_int, [P, C.c_char_p, C.c_int, C.POINTER(P)]),
    ("llrs_model_format", C.c_int, [C.c_char_p, C.POINTER(C.c_int), C.c_char_p, SZ]),
    ("llrs_hf_config_read", C.c_int, [C.c_char_p, C.POINTER(_ModelConfig)]),
    ("llrs_safetensors_read_tensor", C.c_int, [C.c_char_p, C.c_char_p, U32P, C.POINTER(SZ),
                                               C.POINTER(SZ), P, SZ, C.POINTER(SZ)]),
    ("llrs_model_free", None, [P]),
    ("llrs_model_config_get", C.c_int, [P, C.POINTER(_ModelConfig)]),
    ("llrs_model_weight_bytes", SZ, [P]),
    ("llrs_synth_write_gguf", C.c_int, [C.POINTER(_SynthConfig), C.c_char_p]),
    ("llrs_model_synthetic", C.c_int, [P, C.POINTER(_SynthConfig), C.POINTER(P)]),
    ("llrs_model_export_gguf", C.c_int, [P, C.c_char_p]),
    ("llrs_kv_create", C.c_int, [P, SZ, C.POINTER(P)]),
    ("llrs_kv_free", None, [P]),
    ("llrs_kv_reset", C.c_int, [P]),
    ("llrs_kv_decode_path", C.c_int, [P]),
    ("llrs_kv_debug_set_wait_flag", C.c_int, [P, C.c_int]),
    ("llrs_debug_lds_probe", C.c_int, [P, C.c_int, C.c_int, C.c_int]),
    ("llrs_forward_token", C.c_int, [P, P, C.c_uint32, SZ, C.c_int]),
    ("llrs_prefill", C.c_int, [P, P, U32P, SZ, SZ]),
    ("llrs_decode_greedy", C.c_int, [P, P, SZ, SZ, U32P]),
    ("llrs_argmax", C.c_int, [P, U32P]),
    ("llrs_sample", C.c_int, [P, P, P, SZ, C.c_float, U32P]),
    ("llrs_sample_noalloc", C.c_int, [P, P, P, SZ, C.c_float, U32P]),
    ("llrs_generate", C.c_int, [P, P, U32P, SZ, P, SZ, U32P, SZ, SZ, F32P, U32P, P]),
    ("llrs_find_eos_tokens", C.c_int, [C.c_char_p, U32P, SZ, C.POINTER(SZ)]),
    ("llrs_read_logits", C.c_int, [P, F32P, SZ]),
    ("llrs_read_kv", C.c_int, [P, SZ, C.c_int, F32P, SZ]),
    ("llrs_read_tokens", C.c_int, [P, SZ, SZ, U32P]),
    ("llrs_profile_projection", C.c_int, [P, P, C.c_int, C.c_int, C.POINTER(C.c_double),
                                          C.POINTER(SZ)]),
]


def _declare(l: C.CDLL) -> None:
    for name, res, args in SIGNATURES:
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def _check(code: int) -> None:
    if code != 0:
        msg = lib().llrs_last_error()
        raise LlrsError(code, msg.decode() if msg else "")


def _f32(a: np.ndarray) -> C.POINTER(C.c_float):
    return a.ctypes.data_as(F32P)


# --------------------------------------------------------------------------- types


class QuantType(enum.IntEnum):
    """quant::QuantType with its GGML type ids (src/quant.rs:10-44)."""
    F32 = 0  # `QuantType::None` in the reference
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q4K = 12
    Q5K = 13
    Q6K = 14
    BF16 = 30

    @classmethod
    def from_ggml_type(cls, value: int) -> "QuantType":
        try:
            return cls(value)
        except ValueError:
            raise LlrsError(-2, f"unsupported GGML tensor type {value}") from None

    def block_size(self) -> int:
        if self in (QuantType.F32, QuantType.F16, QuantType.BF16):
            return 1
        if self in (QuantType.Q4K, QuantType.Q5K, QuantType.Q6K):
            return 256
        return 32

    def type_size(self) -> int:
        return {QuantType.F32: 4, QuantType.F16: 2, QuantType.BF16: 2, QuantType.Q4_0: 18,
                QuantType.Q4_1: 20, QuantType.Q5_0: 22, QuantType.Q5_1: 24, QuantType.Q8_0: 34,
                QuantType.Q4K: 144, QuantType.Q5K: 176, QuantType.Q6K: 210}[self]

    def row_bytes(self, cols: int) -> int:
        return cols // self.block_size() * self.type_size()


class LoadQuantization(enum.IntEnum):
    """loader::LoadQuantization (src/loader.rs:16-25)."""
    NONE = 0
    Q4K = 1
    Q4KM = 2


class LogitsMode(enum.IntEnum):
    """architecture::LogitsMode (src/architecture.rs:35-39)."""
    SKIP = 0
    COMPUTE = 1


@dataclass
class QuantTensor:
    """Host-side quant::QuantTensor: native GGUF block bytes, shape [rows, cols]."""
    data: bytes
    shape: tuple
    quant_type: QuantType

    @classmethod
    def from_owned(cls, data, shape, quant_type) -> "QuantTensor":
        qt = QuantType(quant_type)
        shape = tuple(int(s) for s in shape)
        if not 1 <= len(shape) <= 2:
            raise LlrsError(-1, "only 1D and 2D tensors are supported")
        cols = shape[-1]
        if cols % qt.block_size():
            raise LlrsError(-1, f"last dimension {cols} is not divisible by {qt.block_size()}")
        expected = int(np.prod(shape)) // qt.block_size() * qt.type_size()
        data = bytes(data)
        if len(data) != expected:
            raise LlrsError(-1, f"bad tensor byte length: got {len(data)}, expected {expected}")
        return cls(data, shape, qt)

    @classmethod
    def quantize(cls, quant_type, values: np.ndarray, rows: int, cols: int) -> "QuantTensor":
        """QuantTensor::quantize_{q4k,q5_0,q8_0,q6k} (src/quant.rs:187-259) on the host."""
        v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        if v.size != rows * cols:
            raise LlrsError(-1, "quantization shape/data mismatch")
        need, ty = SZ(), C.c_uint32()
        _check(lib().llrs_quantize(int(quant_type), _f32(v), rows, cols, None, 0, C.byref(need),
                                   C.byref(ty)))
        out = np.empty(need.value, dtype=np.uint8)
        _check(lib().llrs_quantize(int(quant_type), _f32(v), rows, cols, out.ctypes.data, out.size,
                                   C.byref(need), C.byref(ty)))
        return cls(out.tobytes(), (rows, cols), QuantType(ty.value))

    def rows(self) -> int:
        return 1 if len(self.shape) == 1 else self.shape[0]

    def cols(self) -> int:
        return self.shape[-1]

    def row_bytes(self) -> int:
        return self.quant_type.row_bytes(self.cols())


# ------------------------------------------------------------------------ backend


class KernelBackend:
    """backend::KernelBackend (src/backend.rs:67-73)."""

    def name(self) -> str:
        raise NotImplementedError

    def threads(self) -> int:
        raise NotImplementedError

    def matvec(self, weight, input: np.ndarray, output: np.ndarray) -> None:
        raise NotImplementedError


class DeviceTensor:
    """A QuantTensor resident in HBM (llrs_tensor_upload)."""

    def __init__(self, backend: "HipBackend", tensor: QuantTensor):
        self.backend = backend
        self.quant_type = tensor.quant_type
        self.shape = (tensor.rows(), tensor.cols()) if len(tensor.shape) == 2 else tensor.shape
        h = P()
        buf = np.frombuffer(tensor.data, dtype=np.uint8)
        _check(lib().llrs_tensor_upload(backend.handle, buf.ctypes.data if buf.size else None,
                                        buf.size, int(tensor.quant_type), tensor.rows(),
                                        tensor.cols(), C.byref(h)))
        self.handle = h
        self._free = lib().llrs_tensor_free  # bound now: usable at interpreter shutdown
        self.nbytes = buf.size

    def rows(self) -> int:
        return self.shape[0] if len(self.shape) == 2 else 1

    def cols(self) -> int:
        return self.shape[-1]

    def download(self) -> bytes:
        out = np.empty(self.nbytes, dtype=np.uint8)
        _check(lib().llrs_tensor_download(self.handle, out.ctypes.data, out.size))
        return out.tobytes()

    def row_into(self, row: int, output: np.ndarray) -> None:
        """QuantTensor::row_into (src/quant.rs:261-272), dequantized on the GPU."""
        _check(lib().llrs_dequant_row(self.backend.handle, self.handle, row, _f32(output),
                                      output.size))

    def __del__(self):
        # The C side counts references (a tensor keeps its backend alive), so
        # finalizers may run in any order, at interpreter shutdown too.
        h, free = getattr(self, "handle", None), getattr(self, "_free", None)
        if h and free is not None:
            free(h)
            self.handle = None


class HipBackend(KernelBackend):
    """The MI355X KernelBackend: one HIP device + stream (CpuBackend's counterpart)."""

    def __init__(self, device: int = 0):
        cfg = _BackendConfig(device, 0)
        h = P()
        _check(lib().llrs_backend_create(C.byref(cfg), C.byref(h)))
        self.handle = h
        self._free = lib().llrs_backend_destroy

    def name(self) -> str:
        return lib().llrs_backend_name(self.handle).decode()

    def threads(self) -> int:
        return int(lib().llrs_backend_threads(self.handle))

    def upload(self, tensor: QuantTensor) -> DeviceTensor:
        return DeviceTensor(self, tensor)

    def matvec(self, weight, input: np.ndarray, output: np.ndarray) -> None:
        """KernelBackend::matvec: output[r] = sum_c weight[r, c] * input[c]."""
        if isinstance(weight, QuantTensor):
            weight = self.upload(weight)
        x = np.ascontiguousarray(input, dtype=np.float32)
        if output.dtype != np.float32 or not output.flags.c_contiguous:
            raise LlrsError(-1, "output must be a contiguous float32 array")
        _check(lib().llrs_matvec(self.handle, weight.handle, _f32(x), x.size, _f32(output),
                                 output.size))

    def synchronize(self) -> None:
        _check(lib().llrs_backend_synchronize(self.handle))

    def __del__(self):
        # Releases this handle only: models, caches and tensors made from the
        # backend hold their own references to it (any finalization order).
        h, free = getattr(self, "handle", None), getattr(self, "_free", None)
        if h and free is not None:
            free(h)
            self.handle = None


def gguf_read_tensor(path, name: str):
    """GgufFile::open(path).tensor(name) (src/gguf.rs:78-215): (version, QuantTensor)."""
    ver, ty, rows, cols, nb = C.c_uint32(), C.c_uint32(), SZ(), SZ(), SZ()
    p, n = str(path).encode(), name.encode()
    _check(lib().llrs_gguf_read_tensor(p, n, C.byref(ver), C.byref(ty), C.byref(rows),
                                       C.byref(cols), None, 0, C.byref(nb)))
    buf = np.empty(nb.value, dtype=np.uint8)
    _check(lib().llrs_gguf_read_tensor(p, n, C.byref(ver), C.byref(ty), C.byref(rows),
                                       C.byref(cols), buf.ctypes.data if buf.size else None,
                                       buf.size, C.byref(nb)))
    shape = (rows.value, cols.value)
    return ver.value, QuantTensor(buf.tobytes(), shape, QuantType(ty.value))


def safetensors_read_tensor(model_dir, name: str):
    """SafetensorStore::open(model_dir).tensor(name) (src/loader.rs:543-645):
    (QuantType, shape, raw bytes)."""
    ty, nd, nb = C.c_uint32(), SZ(), SZ()
    shape = (SZ * 2)()
    d, n = str(model_dir).encode(), name.encode()
    _check(lib().llrs_safetensors_read_tensor(d, n, C.byref(ty), shape, C.byref(nd), None, 0,
                                              C.byref(nb)))
    buf = np.empty(nb.value, dtype=np.uint8)
    _check(lib().llrs_safetensors_read_tensor(d, n, C.byref(ty), shape, C.byref(nd),
                                              buf.ctypes.data if buf.size else None, buf.size,
                                              C.byref(nb)))
    return QuantType(ty.value), tuple(shape[i] for i in range(nd.value)), buf.tobytes()


def model_format(path):
    """ModelLoader::load's format choice (src/loader.rs:44-77): ("gguf", file)
    or ("safetensors", directory)."""
    fmt = C.c_int()
    buf = C.create_string_buffer(4096)
    _check(lib().llrs_model_format(str(path).encode(), C.byref(fmt), buf, len(buf)))
    return ("gguf" if fmt.value == 1 else "safetensors"), buf.value.decode()


__all__ = ["gguf_read_tensor", "safetensors_read_tensor", "model_format", "LlrsError", "QuantType", "QuantTensor", "LoadQuantization", "LogitsMode",
           "KernelBackend", "HipBackend", "DeviceTensor", "lib", "LIB_PATH", "HEADER"]

from . import blocks  # noqa: E402
from .model import (LlamaConfig, KVCache, HipQwen2Model, ModelLoader,  # noqa: E402
                    GgufLoader, SafetensorsLoader, hf_config, SynthConfig, InferenceEngine,
                    Sampler, SamplingOptions, find_eos_tokens, GenerationOutput)

__all__ += ["LlamaConfig", "KVCache", "HipQwen2Model", "ModelLoader", "GgufLoader",
            "SafetensorsLoader", "hf_config", "SynthConfig", "InferenceEngine", "Sampler",
            "SamplingOptions", "find_eos_tokens", "GenerationOutput"]
