"""Handle ownership: a model holds a counted reference to its backend and a KV
cache one to its model, as Qwen2Model holds an Arc<dyn KernelBackend>
(src/model.rs:117; src/loader.rs:99, 242), so the handles may be released in
any order.  Each case runs in a child process (one at a time) and must exit 0.
"""
from __future__ import annotations

import subprocess
import sys
import textwrap

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

PRELUDE = textwrap.dedent(f"""
    import ctypes as C, sys
    sys.path.insert(0, {str(ROOT / 'tests')!r})
    from conftest import load_package
    llrs = load_package()
    from llama_rs_amd.model import HipQwen2Model, KVCache, SynthConfig
    cfg = SynthConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                      num_key_value_heads=2, num_hidden_layers=2, vocab_size=512,
                      max_position_embeddings=256, seed=11)
""")


def run_child(body: str) -> subprocess.CompletedProcess:
    src = PRELUDE + textwrap.dedent(body)
    print(f"[ownership] child: {body.strip().splitlines()[0]}", flush=True)
    return subprocess.run([sys.executable, "-c", src], capture_output=True, text=True, timeout=180)


def test_backend_destroyed_before_model_and_cache():
    """The C handles released backend first, model second: the cache still
    decodes, and freeing it last releases everything."""
    r = run_child("""
        lib = llrs.lib()
        b = llrs.HipBackend(0)
        model = HipQwen2Model.synthetic(b, cfg)
        kv = KVCache(model, 64)
        prompt = [3, 7, 11, 13]
        model.prefill(prompt, 0, kv)
        first = model.decode_greedy(len(prompt), 6, kv).tolist()
        # Release the raw handles in the order that used to fault: backend, model, cache.
        bh, mh, kh = b.handle, model.handle, kv.handle
        b.handle = model.handle = kv.handle = None
        lib.llrs_backend_destroy(bh)
        lib.llrs_model_free(mh)
        # The cache still owns the model and the backend: decode again from the start.
        kv.handle = kh
        model.handle = mh  # a borrowed pointer, kept alive by the cache
        model._free = None
        model.prefill(prompt, 0, kv)
        again = model.decode_greedy(len(prompt), 6, kv).tolist()
        assert again == first, (first, again)
        kv.handle = None
        lib.llrs_kv_free(kh)
        print("ok", flush=True)
    """)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")


def test_finalizers_at_interpreter_shutdown():
    """Objects still alive at exit (held by a reference cycle and by a failed
    test's traceback, as in pytest) are finalized in arbitrary order."""
    r = run_child("""
        b = llrs.HipBackend(0)
        model = HipQwen2Model.synthetic(b, cfg)
        kv = KVCache(model, 64)
        model.prefill([1, 2, 3], 0, kv)
        cycle = {"kv": kv, "model": model, "backend": b}
        cycle["self"] = cycle
        try:
            raise RuntimeError("keep the frame")
        except RuntimeError as e:
            sys.last_exc = e  # the traceback holds this frame's objects
        del b
        print("ok", flush=True)
    """)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")
