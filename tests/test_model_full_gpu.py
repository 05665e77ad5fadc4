"""GPU parity at the full shapes of the headline configs (MI355X).

Bar (north star): logits within 2e-2 max-abs of the scalar oracle's,
identical greedy token ids over 32 decode steps, K/V rows within 1e-3
(relative to the row scale).

cfg5: the Qwen2.5-7B-shape q4km model of the bench (28 layers, hidden 3584,
28/4 heads, FFN 18944, untied 152,064-row Q8_0 LM head), generated in HBM
from seed 5 and exported as GGUF for the oracle; the bench's own workload
shape: a 512-token random prompt through the batched MFMA prefill (128-token
tiles, the segmented Q+K product, the dual gate/up product, Q6_K down), then
32 greedy steps of the persistent decode kernel.  The oracle runs the same
544 forwards on the box's host threads with its scalar path (the reference's
scalar backend; src/engine.rs:189-223; src/model.rs:135-271); the K/V rows
of every layer are compared after the prefill and after the decode.

cfg4: the Qwen2.5-1.5B-shape uniform q4k model (12/2 heads, head_dim 128,
tied Q4_K LM head) prefilled to 4,000 positions on the GPU, in eight
512-token chunks.  The scalar oracle cannot repeat 4,000 forwards of 0.87 GB
in a test's time, so it checks the prefill where the chunks meet: for every
chunk boundary b, its state is seeded with the GPU's K/V rows of positions
0..b-1 and it computes positions b..b+7 itself, whose rows must match the
GPU's on every layer; and seeded with positions 0..3989, it computes
3990..3999 and the logits at 3999.  Then both decode 32 greedy steps from
position 4,000, where the persistent kernel's attention runs ~1,500 items
merged in two levels (src/model.rs:206-231).
"""
from __future__ import annotations

import os
import pathlib
import shutil
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
ORACLE_THREADS = 16  # the GPU box's CPU share


def scratch_path(tmp_path, name, nbytes):
    """/dev/shm when it has room (the 7B file is 4.8 GB), else tmp_path."""
    shm = pathlib.Path("/dev/shm")
    if shm.is_dir() and shutil.disk_usage(shm).free > 2 * nbytes:
        return shm / f"llrs_{os.getpid()}_{name}"
    return tmp_path / name


def kv_close(a, b, what):
    err = float(np.abs(a - b).max())
    scale = max(1.0, float(np.abs(b).max()))
    print(f"[full] {what}: max-abs err {err:.3e} (scale {scale:.2f})", flush=True)
    assert err <= 1e-3 * scale, what


def logits_close(lg, lo, what):
    err = float(np.abs(lg - lo).max())
    top = np.sort(lo)[-2:]
    print(f"[full] {what}: logits max-abs err {err:.3e}, oracle top-2 gap {top[1] - top[0]:.3e}",
          flush=True)
    assert err <= LOGIT_TOL, what


def oracle_steps(om, first_tok, start, n):
    """oq_decode_greedy's loop, one forward at a time with progress lines."""
    toks = []
    tok = first_tok
    for i in range(n):
        toks.append(tok)
        t0 = time.perf_counter()
        om.forward_token(tok, start + i)
        tok = om.argmax()
        print(f"[full] oracle step {i} at {start + i}: {time.perf_counter() - t0:.2f}s", flush=True)
    return np.array(toks, np.uint32)


def synth_pair(llrs, backend, oracle, cfg, path):
    t0 = time.perf_counter()
    model = llrs.HipQwen2Model.synthetic(backend, cfg)
    model.export_gguf(path)
    om = oracle.load(path, threads=ORACLE_THREADS)
    print(f"[full] model generated, exported to {path} and loaded by the oracle in "
          f"{time.perf_counter() - t0:.1f}s", flush=True)
    return model, om


@pytest.mark.timeout(600)
def test_config5_7b_q4km_prefill_and_greedy_parity(llrs, backend, oracle, tmp_path):
    cfg = llrs.SynthConfig(hidden_size=3584, intermediate_size=18944, num_attention_heads=28,
                           num_key_value_heads=4, num_hidden_layers=28, vocab_size=152064,
                           max_position_embeddings=32768, rope_theta=1e6, rms_norm_eps=1e-6,
                           tie_word_embeddings=False, recipe=llrs.LoadQuantization.Q4KM, seed=5)
    path = scratch_path(tmp_path, "cfg5.gguf", 4_800_000_000)
    try:
        model, om = synth_pair(llrs, backend, oracle, cfg, path)
        n_prompt, n_decode, ctx = 512, 32, 640
        prompt = np.random.default_rng(5).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
        kv = llrs.KVCache(model, ctx)
        assert kv.persistent
        model.prefill(prompt, 0, kv)
        # The batched prefill is deterministic: a second cache, the same bits.
        kv2 = llrs.KVCache(model, ctx)
        model.prefill(prompt, 0, kv2)
        np.testing.assert_array_equal(kv.logits().view(np.uint32), kv2.logits().view(np.uint32))
        for layer in (0, 27):
            np.testing.assert_array_equal(kv.layer(layer, "v", n_prompt), kv2.layer(layer, "v", n_prompt))
        del kv2
        om.new_state(ctx)
        t0 = time.perf_counter()
        for i, t in enumerate(prompt):
            om.forward_token(int(t), i, i + 1 == n_prompt)
            if i % 32 == 31:
                print(f"[full] oracle prefill {i + 1}/{n_prompt} ({time.perf_counter() - t0:.0f}s)", flush=True)
        logits_close(kv.logits(), om.logits(), "cfg5 prefill (512 tokens)")
        assert kv.argmax() == om.argmax()
        for layer in range(cfg.num_hidden_layers):
            for which in ("k", "v"):
                kv_close(kv.layer(layer, which, n_prompt), om.kv(layer, which, n_prompt),
                         f"cfg5 prefill layer {layer} {which}")
        got = model.decode_greedy(n_prompt, n_decode, kv)
        want = oracle_steps(om, om.argmax(), n_prompt, n_decode)
        print(f"[full] cfg5 tokens gpu={got.tolist()} oracle={want.tolist()}", flush=True)
        np.testing.assert_array_equal(got, want)
        logits_close(kv.logits(), om.logits(), "cfg5 after 32 greedy steps")
        n = n_prompt + n_decode
        for layer in range(cfg.num_hidden_layers):
            for which in ("k", "v"):
                kv_close(kv.layer(layer, which, n)[n_prompt:], om.kv(layer, which, n)[n_prompt:],
                         f"cfg5 decode rows layer {layer} {which}")
    finally:
        if path.exists():
            path.unlink()


@pytest.mark.timeout(600)
def test_config4_15b_q4k_depth_4000_greedy_parity(llrs, backend, oracle, tmp_path):
    cfg = llrs.SynthConfig(hidden_size=1536, intermediate_size=8960, num_attention_heads=12,
                           num_key_value_heads=2, num_hidden_layers=28, vocab_size=151936,
                           max_position_embeddings=32768, rope_theta=1e6, rms_norm_eps=1e-6,
                           tie_word_embeddings=True, recipe=llrs.LoadQuantization.Q4K, seed=4)
    path = scratch_path(tmp_path, "cfg4.gguf", 900_000_000)
    try:
        model, om = synth_pair(llrs, backend, oracle, cfg, path)
        n_prompt, n_decode, ctx, own = 4000, 32, 4096, 10
        prompt = np.random.default_rng(4).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
        kv = llrs.KVCache(model, ctx)
        assert kv.persistent
        model.prefill(prompt, 0, kv)
        L = cfg.num_hidden_layers
        gpu_rows = {(layer, which): kv.layer(layer, which, n_prompt) for layer in range(L) for which in ("k", "v")}
        # Where the 512-token prefill chunks meet: the oracle, seeded with
        # the GPU's rows before the boundary, computes the next 8 positions.
        for b in range(512, n_prompt, 512):
            om.new_state(ctx)
            for (layer, which), rows in gpu_rows.items():
                om.load_kv(layer, which, rows[:b])
            for i in range(b, b + 8):
                om.forward_token(int(prompt[i]), i, False)
            for (layer, which), rows in gpu_rows.items():
                kv_close(rows[b:b + 8], om.kv(layer, which, b + 8)[b:],
                         f"cfg4 prefill rows {b}..{b + 7} layer {layer} {which}")
        om.new_state(ctx)
        seed_to = n_prompt - own
        for layer in range(L):
            for which in ("k", "v"):
                om.load_kv(layer, which, kv.layer(layer, which, seed_to))
        print(f"[full] oracle seeded with the GPU's rows of positions 0..{seed_to - 1}", flush=True)
        for i in range(seed_to, n_prompt):
            om.forward_token(int(prompt[i]), i, i + 1 == n_prompt)
        logits_close(kv.logits(), om.logits(), "cfg4 prefill at position 3999")
        assert kv.argmax() == om.argmax()
        for layer in range(L):
            for which in ("k", "v"):
                a = kv.layer(layer, which, n_prompt)[seed_to:]
                b = om.kv(layer, which, n_prompt)[seed_to:]
                kv_close(a, b, f"cfg4 prefill rows {seed_to}..{n_prompt - 1} layer {layer} {which}")
        got = model.decode_greedy(n_prompt, n_decode, kv)
        want = oracle_steps(om, om.argmax(), n_prompt, n_decode)
        print(f"[full] cfg4 tokens gpu={got.tolist()} oracle={want.tolist()}", flush=True)
        np.testing.assert_array_equal(got, want)
        logits_close(kv.logits(), om.logits(), "cfg4 after 32 greedy steps")
        n = n_prompt + n_decode
        for layer in (0, L - 1):
            for which in ("k", "v"):
                kv_close(kv.layer(layer, which, n)[n_prompt:], om.kv(layer, which, n)[n_prompt:],
                         f"cfg4 decode rows layer {layer} {which}")
    finally:
        if path.exists():
            path.unlink()
