"""ctypes bindings to the CPU oracle (oracle/liboracle.so) -- test infrastructure.

The oracle is the checker for the HIP path, never the thing measured or
shipped.  It is built from oracle/*.c with oracle/Makefile.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIB = ROOT / "oracle" / "liboracle.so"

F32P = C.POINTER(C.c_float)
U8P = C.c_void_p
U32P = C.POINTER(C.c_uint32)


class OqConfig(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in (
        "hidden_size", "intermediate_size", "num_attention_heads", "num_key_value_heads",
        "num_hidden_layers", "vocab_size", "max_position_embeddings", "head_dim", "kv_width")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("tie_word_embeddings", C.c_int)]


SCALAR, AVX2 = 0, 1


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


class Oracle:
    def __init__(self):
        if not LIB.exists():
            build()
        l = C.CDLL(str(LIB))
        sig = {
            "oq_block_size": (C.c_int, [C.c_uint32]),
            "oq_type_size": (C.c_int, [C.c_uint32]),
            "oq_row_bytes": (C.c_size_t, [C.c_uint32, C.c_size_t]),
            "oq_f16_to_f32": (C.c_float, [C.c_uint16]),
            "oq_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "oq_value_at": (C.c_float, [U8P, C.c_uint32, C.c_size_t]),
            "oq_dequant_row": (None, [U8P, C.c_uint32, C.c_size_t, F32P]),
            "oq_dot_row_scalar": (C.c_float, [U8P, C.c_uint32, F32P, C.c_size_t]),
            "oq_dot_row_avx2": (C.c_float, [U8P, C.c_uint32, F32P, C.c_size_t]),
            "oq_cpu_has_avx2_fma": (C.c_int, []),
            "oq_matvec": (C.c_int, [U8P, C.c_uint32, C.c_size_t, C.c_size_t, F32P, F32P, C.c_int,
                                    C.c_int, C.c_size_t]),
            "oq_model_load_gguf": (C.c_void_p, [C.c_char_p, C.c_int, C.c_int]),
            "oq_model_free": (None, [C.c_void_p]),
            "oq_last_error": (C.c_char_p, []),
            "oq_model_config": (None, [C.c_void_p, C.POINTER(OqConfig)]),
            "oq_state_new": (C.c_void_p, [C.c_void_p, C.c_size_t]),
            "oq_state_free": (None, [C.c_void_p]),
            "oq_forward_token": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_size_t, C.c_int]),
            "oq_prefill": (C.c_int, [C.c_void_p, C.c_void_p, U32P, C.c_size_t, C.c_size_t]),
            "oq_argmax": (C.c_uint32, [F32P, C.c_size_t]),
            "oq_sample": (C.c_uint32, [F32P, C.c_size_t, C.c_float, C.c_size_t, C.c_float, C.c_float,
                                       U32P, C.c_size_t, C.c_float]),
            "oq_decode_greedy": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, U32P]),
            "oq_gguf_read_f32": (C.c_int, [C.c_char_p, C.c_char_p, U32P, C.POINTER(C.c_size_t),
                                           C.POINTER(C.c_size_t), F32P, C.c_size_t]),
            "oq_state_logits": (F32P, [C.c_void_p]),
            "oq_state_residual": (F32P, [C.c_void_p]),
            "oq_state_k_cache": (F32P, [C.c_void_p, C.c_size_t]),
            "oq_state_v_cache": (F32P, [C.c_void_p, C.c_size_t]),
            "oq_state_load": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t, F32P, C.c_size_t]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(l, name)
            fn.restype, fn.argtypes = res, args
        self.lib = l

    # ------------------------------------------------------------- block-level
    def row_bytes(self, ty: int, cols: int) -> int:
        return int(self.lib.oq_row_bytes(ty, cols))

    def dequant_row(self, data: bytes, ty: int, row: int, cols: int) -> np.ndarray:
        rb = self.row_bytes(ty, cols)
        buf = np.frombuffer(data, dtype=np.uint8)[row * rb:(row + 1) * rb]
        buf = np.ascontiguousarray(buf)
        out = np.empty(cols, dtype=np.float32)
        self.lib.oq_dequant_row(buf.ctypes.data, ty, cols, out.ctypes.data_as(F32P))
        return out

    def dot(self, row_bytes: bytes, ty: int, x: np.ndarray, kernel: int = SCALAR) -> float:
        buf = np.frombuffer(row_bytes, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        f = self.lib.oq_dot_row_avx2 if kernel == AVX2 else self.lib.oq_dot_row_scalar
        return float(f(buf.ctypes.data, ty, x.ctypes.data_as(F32P), x.size))

    def matvec(self, data: bytes, ty: int, rows: int, cols: int, x: np.ndarray,
               kernel: int = SCALAR, threads: int = 0, threshold: int = 128 * 1024) -> np.ndarray:
        buf = np.frombuffer(data, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        rc = self.lib.oq_matvec(buf.ctypes.data, ty, rows, cols, x.ctypes.data_as(F32P),
                                y.ctypes.data_as(F32P), kernel, threads, threshold)
        assert rc == 0
        return y

    def sample(self, logits: np.ndarray, temperature: float, top_k: int, top_p: float,
               repetition_penalty: float, recent, uniform: float) -> int:
        """sample_current_logits (src/engine.rs:253-325) with the given uniform draw."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        r = np.ascontiguousarray(np.asarray(recent, dtype=np.uint32))
        return int(self.lib.oq_sample(lg.ctypes.data_as(F32P), lg.size, temperature, top_k, top_p,
                                      repetition_penalty, r.ctypes.data_as(U32P) if r.size else None,
                                      r.size, uniform))

    def gguf_read_f32(self, path, name: str):
        """(version, values[rows, cols]) via the oracle's GGUF reader; raises on error."""
        ver, rows, cols = C.c_uint32(), C.c_size_t(), C.c_size_t()
        if self.lib.oq_gguf_read_f32(str(path).encode(), name.encode(), C.byref(ver),
                                     C.byref(rows), C.byref(cols), None, 0):
            raise RuntimeError(self.lib.oq_last_error().decode())
        out = np.empty(rows.value * cols.value, np.float32)
        if self.lib.oq_gguf_read_f32(str(path).encode(), name.encode(), C.byref(ver),
                                     C.byref(rows), C.byref(cols), out.ctypes.data_as(F32P),
                                     out.size):
            raise RuntimeError(self.lib.oq_last_error().decode())
        return ver.value, out.reshape(rows.value, cols.value)

    def has_avx2(self) -> bool:
        return bool(self.lib.oq_cpu_has_avx2_fma())

    # ------------------------------------------------------------------ model
    def load(self, path, kernel: int = SCALAR, threads: int = 0) -> "OracleModel":
        h = self.lib.oq_model_load_gguf(str(path).encode(), kernel, threads)
        if not h:
            raise RuntimeError(self.lib.oq_last_error().decode())
        return OracleModel(self, h)


class OracleModel:
    def __init__(self, o: Oracle, h):
        self.o, self.h = o, h
        c = OqConfig()
        o.lib.oq_model_config(h, C.byref(c))
        self.cfg = c
        self.state = None

    def new_state(self, max_seq_len: int) -> None:
        if self.state:
            self.o.lib.oq_state_free(self.state)
        self.state = self.o.lib.oq_state_new(self.h, max_seq_len)
        if not self.state:
            raise RuntimeError(self.o.lib.oq_last_error().decode())

    def forward_token(self, token: int, pos: int, compute: bool = True) -> None:
        if self.o.lib.oq_forward_token(self.h, self.state, token, pos, int(compute)):
            raise RuntimeError(self.o.lib.oq_last_error().decode())

    def prefill(self, tokens, start: int = 0) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        if self.o.lib.oq_prefill(self.h, self.state, t.ctypes.data_as(U32P), t.size, start):
            raise RuntimeError(self.o.lib.oq_last_error().decode())

    def decode_greedy(self, start: int, n: int) -> np.ndarray:
        out = np.zeros(max(n, 1), dtype=np.uint32)
        if self.o.lib.oq_decode_greedy(self.h, self.state, start, n, out.ctypes.data_as(U32P)):
            raise RuntimeError(self.o.lib.oq_last_error().decode())
        return out[:n]

    def logits(self) -> np.ndarray:
        p = self.o.lib.oq_state_logits(self.state)
        return np.ctypeslib.as_array(p, shape=(self.cfg.vocab_size,)).copy()

    def kv(self, layer: int, which: str, n_pos: int) -> np.ndarray:
        f = self.o.lib.oq_state_k_cache if which == "k" else self.o.lib.oq_state_v_cache
        p = f(self.state, layer)
        return np.ctypeslib.as_array(p, shape=(n_pos * self.cfg.kv_width,)).copy().reshape(
            n_pos, self.cfg.kv_width)

    def load_kv(self, layer: int, which: str, rows: np.ndarray) -> None:
        """Seeds the cache rows of `layer` from position 0 (e.g. with the GPU's)."""
        r = np.ascontiguousarray(rows, dtype=np.float32).ravel()
        if self.o.lib.oq_state_load(self.state, 0 if which == "k" else 1, layer,
                                    r.ctypes.data_as(F32P), r.size):
            raise RuntimeError(self.o.lib.oq_last_error().decode())

    def load_logits(self, logits: np.ndarray) -> None:
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        if self.o.lib.oq_state_load(self.state, 2, 0, lg.ctypes.data_as(F32P), lg.size):
            raise RuntimeError(self.o.lib.oq_last_error().decode())

    def argmax(self) -> int:
        lg = self.logits()
        return int(self.o.lib.oq_argmax(lg.ctypes.data_as(F32P), lg.size))

    def __del__(self):
        if getattr(self, "state", None):
            self.o.lib.oq_state_free(self.state)
        if getattr(self, "h", None):
            self.o.lib.oq_model_free(self.h)
            self.h = None
