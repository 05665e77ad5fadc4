"""llrs_sample_noalloc: the sampler with its scratch in a file-scope device
array (no allocation on any call) against llrs_sample (scratch allocated on
first use), through the C ABI.

Two calls in a row on the same GPU share that array: a 152,064-token
vocabulary first, then a 1,000-token one (a smaller input, whose call must
not see anything the larger one left).  Each call's token must equal
llrs_sample's for the same options, window and uniform draw.

The property itself is probed with hipMemGetInfo: on a fresh cache the
device's free bytes are unchanged by the first llrs_sample_noalloc calls,
and the same probe sees llrs_sample's first call allocate its scratch.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def noalloc(llrs, kv, opts, recent, u):
    f = llrs.lib().llrs_sample_noalloc  # bound from include/llrs.h's signature
    r = np.ascontiguousarray(np.asarray(recent, dtype=np.uint32))
    o = llrs._Sampling(opts.temperature, opts.top_p, opts.top_k, opts.repetition_penalty)
    t = C.c_uint32()
    rc = f(kv.handle, C.byref(o), r.ctypes.data_as(C.c_void_p) if r.size else None, r.size, float(u),
           C.byref(t))
    if rc != 0:
        raise llrs.LlrsError(rc, llrs.lib().llrs_last_error().decode())
    return int(t.value)


def model_kv(llrs, backend, vocab, seed):
    cfg = llrs.SynthConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=1, vocab_size=vocab,
                           max_position_embeddings=256, recipe=llrs.LoadQuantization.Q4KM,
                           seed=seed, tie_word_embeddings=False)
    model = llrs.HipQwen2Model.synthetic(backend, cfg)
    kv = llrs.KVCache(model, 64)
    model.prefill(np.arange(1, 9, dtype=np.uint32) * 37 % vocab, 0, kv)
    return model, kv


def test_sample_noalloc_matches_sample(llrs, backend):
    rng = np.random.default_rng(91)
    cases = [llrs.SamplingOptions(),
             llrs.SamplingOptions(temperature=1.3, top_p=0.95, top_k=0, repetition_penalty=1.0),
             llrs.SamplingOptions(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.1)]
    for vocab, seed in ((152064, 3), (1000, 4)):  # the second call is the smaller input
        model, kv = model_kv(llrs, backend, vocab, seed)
        for opts in cases:
            recent = rng.integers(0, vocab, 64).astype(np.uint32)
            for _ in range(4):
                u = float(rng.random())
                a, b = noalloc(llrs, kv, opts, recent, u), kv.sample(opts, u, recent)
                print(f"[noalloc] vocab {vocab} T={opts.temperature} u={u:.3f}: {a} vs {b}", flush=True)
                assert a == b
        # The window alone changes: the penalty must see the new one.
        assert noalloc(llrs, kv, cases[2], [], 0.5) == kv.sample(cases[2], 0.5, [])


def free_device_bytes(llrs) -> int:
    """hipMemGetInfo's free bytes of the current device, looked up through the
    library's own handle: the HIP runtime it links and has initialised (a
    separate dlopen of libamdhip64.so may load another copy that sees no
    device)."""
    f = llrs.lib().hipMemGetInfo
    f.restype, f.argtypes = C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    free, total = C.c_size_t(), C.c_size_t()
    assert f(C.byref(free), C.byref(total)) == 0
    return free.value


def test_sample_noalloc_allocates_nothing(llrs, backend):
    opts = llrs.SamplingOptions(temperature=0.8, top_p=0.9, top_k=40, repetition_penalty=1.1)
    recent = np.arange(64, dtype=np.uint32)
    _, warm = model_kv(llrs, backend, 1000, 7)
    noalloc(llrs, warm, opts, recent, 0.5)  # the sampler's code is resident before the probe
    _, kv = model_kv(llrs, backend, 152064, 6)  # a fresh cache: no sampler scratch yet
    backend.synchronize()
    before = free_device_bytes(llrs)
    for u in (0.1, 0.5, 0.9):
        noalloc(llrs, kv, opts, recent, u)
    after = free_device_bytes(llrs)
    print(f"[noalloc] free bytes {before} -> {after}", flush=True)
    assert after == before
    # The probe sees an allocation: llrs_sample's first call allocates its scratch.
    kv.sample(opts, 0.5, recent)
    allocated = free_device_bytes(llrs)
    print(f"[noalloc] llrs_sample's first call: free bytes {after} -> {allocated}", flush=True)
    assert allocated < after


def test_sample_noalloc_rejects_oversized_window(llrs, backend):
    _, kv = model_kv(llrs, backend, 1000, 5)
    with pytest.raises(llrs.LlrsError, match="repeat window"):
        noalloc(llrs, kv, llrs.SamplingOptions(), np.zeros(65537, np.uint32), 0.5)
