"""The host parsers under AddressSanitizer and UndefinedBehaviorSanitizer, fed
malformed files by hypothesis (CPU only).

The product library's host-only sources (error.cpp, json.cpp, gguf.cpp,
safetensors.cpp, engine.cpp, quantize_host.cpp with the encoders of
quant_encode.h) are compiled with g++ -fsanitize=address,undefined,
float-cast-overflow and -fno-sanitize-recover into a driver
(tests/fuzz/fuzz_host.cpp) that runs one parser on each file given.  Inputs
are valid files mutated by hypothesis: byte flips and overwrites (lengths,
counts, offsets, type ids set to extremes), truncations, appended bytes,
and for JSON generated documents with deep nesting, odd numbers and escapes.
Every run must end normally, each file accepted or rejected with an error
message; a sanitizer report fails the test and hypothesis stops at the first
failing input (derandomized, so the runs are reproducible).  The files that
untrusted input reaches at load time are these: GGUF (src/gguf.rs), the
SafeTensors header and config.json (src/loader.rs:80-228, src/config.rs),
tokenizer.json / generation_config.json (src/engine.rs:340-387).
"""
from __future__ import annotations

import json
import os
import pathlib
import shutil
import struct
import subprocess

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from conftest import ROOT
from test_gguf import minimal_v3

CSRC = ROOT / "llama.rs_amd" / "csrc"
SOURCES = ["error.cpp", "json.cpp", "gguf.cpp", "safetensors.cpp", "engine.cpp", "quantize_host.cpp"]
SAN = ["-fsanitize=address,undefined,float-cast-overflow", "-fno-sanitize-recover=all",
       "-fno-omit-frame-pointer"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
SETTINGS = settings(max_examples=40, deadline=None, derandomize=True,
                    suppress_health_check=[HealthCheck.function_scoped_fixture,
                                           HealthCheck.too_slow])


@pytest.fixture(scope="session")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ is not available")
    out = tmp_path_factory.mktemp("fuzz") / "fuzz_host"
    cmd = [gxx, "-std=c++17", "-O1", "-g", *SAN, "-ffp-contract=off", "-D__HIP_PLATFORM_AMD__",
           "-I/opt/rocm/include", f"-I{CSRC}", f"-I{ROOT / 'include'}",
           *[str(CSRC / s) for s in SOURCES], str(ROOT / "tests" / "fuzz" / "fuzz_host.cpp"),
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out


def run(driver, mode, paths):
    res = subprocess.run([str(driver), mode, *map(str, paths)], capture_output=True, text=True,
                         env=ENV, timeout=120)
    report = res.stdout[-3000:] + res.stderr[-6000:]
    assert res.returncode == 0, report
    assert "Sanitizer" not in res.stderr and "runtime error" not in res.stderr, report
    lines = [l for l in res.stdout.splitlines() if not l.startswith("== ")]
    assert len(lines) == len(paths), report
    return lines


def mutate(data: bytes, draw) -> bytes:
    """A few random edits of `data`: flips, 1/4/8-byte overwrites with extreme
    values, a truncation or appended bytes."""
    b = bytearray(data)
    for _ in range(draw(st.integers(1, 6))):
        kind = draw(st.sampled_from(["flip", "u32", "u64", "cut", "append", "byte"]))
        at = draw(st.integers(0, max(0, len(b) - 1)))
        if kind == "flip" and b:
            b[at] ^= 1 << draw(st.integers(0, 7))
        elif kind == "byte" and b:
            b[at] = draw(st.integers(0, 255))
        elif kind in ("u32", "u64") and len(b) >= 8:
            n = 4 if kind == "u32" else 8
            at = min(at, len(b) - n)
            v = draw(st.sampled_from([0, 1, 2 ** 31 - 1, 2 ** 32 - 1, 2 ** 63 - 1, 2 ** 64 - 1,
                                      len(data), len(data) + 1]))
            b[at:at + n] = (v % (1 << (8 * n))).to_bytes(n, "little")
        elif kind == "cut":
            del b[at:]
        elif kind == "append":
            b += draw(st.binary(min_size=1, max_size=64))
    return bytes(b)


# ------------------------------------------------------------------- GGUF
def gguf_bases(llrs, tmp) -> list[bytes]:
    cfg = llrs.SynthConfig(hidden_size=64, intermediate_size=128, num_attention_heads=2,
                           num_key_value_heads=1, num_hidden_layers=1, vocab_size=32,
                           max_position_embeddings=64, recipe=llrs.LoadQuantization.Q4KM, seed=3)
    cfg.write_gguf(tmp / "base.gguf")
    return [minimal_v3(), minimal_v3(version=2), minimal_v3(tensor_type=8, data=(0.0,) * 9),
            (tmp / "base.gguf").read_bytes()]


@SETTINGS
@given(data=st.data())
def test_gguf_reader_on_mutated_files(llrs, driver, tmp_path, data):
    bases = gguf_bases(llrs, tmp_path)
    paths = []
    for i, base in enumerate(bases):
        for j in range(3):
            p = tmp_path / f"m{i}_{j}.gguf"
            p.write_bytes(mutate(base, data.draw))
            paths.append(p)
    run(driver, "gguf", paths)


# ------------------------------------------------------------- SafeTensors
def st_base(tmp) -> bytes:
    header = {"__metadata__": {"format": "pt"},
              "w": {"dtype": "BF16", "shape": [4, 8], "data_offsets": [0, 64]},
              "b": {"dtype": "F32", "shape": [8], "data_offsets": [64, 96]}}
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    return struct.pack("<Q", len(h)) + h + bytes(range(96))


CONFIG = {"model_type": "qwen2", "hidden_size": 8, "intermediate_size": 16, "num_attention_heads": 2,
          "num_key_value_heads": 1, "num_hidden_layers": 1, "vocab_size": 4,
          "max_position_embeddings": 64, "rms_norm_eps": 1e-6, "rope_theta": 1e6}


@SETTINGS
@given(data=st.data())
def test_safetensors_and_config_on_mutated_files(driver, tmp_path, data):
    base = st_base(tmp_path)
    cfg = json.dumps(CONFIG).encode()
    dirs, cfgs = [], []
    for j in range(6):
        d = tmp_path / f"ck{j}"
        d.mkdir(exist_ok=True)
        # Mutate either the 8-byte length, the JSON header, or anywhere.
        (d / "model.safetensors").write_bytes(mutate(base, data.draw))
        (d / "config.json").write_bytes(mutate(cfg, data.draw) if j % 2 else cfg)
        dirs.append(d)
        cfgs.append(d / "config.json")
    run(driver, "safetensors", dirs)
    run(driver, "config", cfgs)


# ------------------------------------------------------------------- JSON
json_values = st.recursive(
    st.none() | st.booleans() | st.integers(-2 ** 70, 2 ** 70) | st.floats(allow_nan=False)
    | st.text(max_size=20),
    lambda kids: st.lists(kids, max_size=5) | st.dictionaries(st.text(max_size=8), kids, max_size=5),
    max_leaves=30)


@SETTINGS
@given(data=st.data())
def test_json_reader_on_generated_and_mutated_documents(driver, tmp_path, data):
    paths = []
    for j in range(8):
        doc = json.dumps(data.draw(json_values), ensure_ascii=bool(j % 2)).encode()
        if j >= 4:
            doc = mutate(doc, data.draw)
        p = tmp_path / f"d{j}.json"
        p.write_bytes(doc)
        paths.append(p)
    deep = tmp_path / "deep.json"
    deep.write_bytes(b"[" * 200 + b"]" * 200)
    esc = tmp_path / "esc.json"
    esc.write_bytes(b'"\\ud800\\udc00 \\uD83D \\u00zz \\\\"')
    lines = run(driver, "json", paths + [deep, esc])
    assert "rejected" in lines[-2] and "rejected" in lines[-1]  # nesting limit, bad escape


# ----------------------------------------------------------------- EOS ids
@SETTINGS
@given(data=st.data())
def test_eos_discovery_on_mutated_files(driver, tmp_path, data):
    tok = json.dumps({"added_tokens": [{"id": 5, "content": "<|im_end|>"}],
                      "model": {"type": "BPE", "vocab": {"a": 0, "<|endoftext|>": 3}}}).encode()
    gen = json.dumps({"eos_token_id": [5, 7]}).encode()
    dirs = []
    for j in range(4):
        d = tmp_path / f"e{j}"
        d.mkdir(exist_ok=True)
        (d / "tokenizer.json").write_bytes(mutate(tok, data.draw))
        (d / "generation_config.json").write_bytes(mutate(gen, data.draw) if j % 2 else gen)
        dirs.append(d)
    run(driver, "eos", dirs)


# --------------------------------------------------------------- encoders
special = st.sampled_from([0.0, -0.0, float("nan"), float("inf"), float("-inf"), 1e-45, -1e-45,
                           3.4e38, -3.4e38, 1.0, 65504.0, 65520.0, 1e-8])


@SETTINGS
@given(vals=st.lists(st.floats(width=32) | special, min_size=256, max_size=1024))
def test_encoders_on_arbitrary_floats(driver, tmp_path, vals):
    p = tmp_path / "v.bin"
    np.array(vals, np.float32).tofile(p)
    assert run(driver, "quantize", [p]) == [f"{p}: ok"]
