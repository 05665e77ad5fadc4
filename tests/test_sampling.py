"""Sampling: InferenceEngine::sample_current_logits (src/engine.rs:253-325).

The oracle's restatement (oq_sample) is pinned by hand-computed cases and by
an independent float64 restatement; the device sampler (llrs_sample) is then
compared with it on real logits for the same uniform draws.  The reference
draws its uniform number from rand::thread_rng(), so parity is "the same
token for the same draw"; draws that fall within 1e-5 of a boundary between
two candidates are not compared (the sums are f32 in different orders).
"""
from __future__ import annotations

import numpy as np
import pytest


def f64_sample(logits, temperature, top_k, top_p, penalty, recent, u):
    """Independent float64 restatement: (token, distance of u*kept from the
    nearest candidate boundary, relative to the kept mass)."""
    v = np.asarray(logits, dtype=np.float64).copy()
    seen = np.zeros(v.size, bool)
    seen[[t for t in recent if t < v.size]] = True
    if penalty != 1.0:
        v = np.where(seen, np.where(v > 0, v / penalty, v * penalty), v)
    if temperature > 0:
        v = v / temperature
    v = np.where(np.isfinite(v), v, -np.inf)
    order = np.lexsort((np.arange(v.size), -v))  # descending, lower index first
    if temperature <= 0:
        return int(order[0]), np.inf
    m = top_k if 0 < top_k < v.size else v.size
    vals = v[order[:m]]
    p = np.exp(vals - vals[0])
    if not np.isfinite(p.sum()) or p.sum() <= 0:
        return int(order[0]), np.inf
    p /= p.sum()
    cum = np.cumsum(p)
    hit = np.nonzero(cum >= top_p)[0]
    cutoff = int(hit[0]) + 1 if hit.size else m
    kept = cum[cutoff - 1]
    r = u * kept
    idx = int(np.searchsorted(cum[:cutoff], r))
    idx = min(idx, cutoff - 1)
    margin = float(np.min(np.abs(cum[:cutoff] - r)) / kept)
    return int(order[idx]), margin


# ---------------------------------------------------------------- the oracle

def test_greedy_and_top_k_1(oracle):
    lg = np.array([0.1, 2.5, -1.0, 2.4, 0.0], np.float32)
    assert oracle.sample(lg, 0.0, 40, 0.9, 1.0, [], 0.3) == 1
    for u in (0.0, 0.5, 0.999):
        assert oracle.sample(lg, 0.7, 1, 0.9, 1.0, [], u) == 1
    tie = np.array([1.0, 3.0, 3.0, 0.0], np.float32)
    assert oracle.sample(tie, 0.0, 0, 1.0, 1.0, [], 0.0) == 1  # equal values: lower index first


def test_uniform_logits_split_the_unit_interval(oracle):
    n = 8
    lg = np.zeros(n, np.float32)
    for k in range(n):
        assert oracle.sample(lg, 1.0, 0, 1.0, 1.0, [], (k + 0.5) / n) == k


def test_top_p_cutoff_and_draw(oracle):
    """p = (0.5, 0.3, 0.2), top_p 0.6: the cutoff keeps two candidates (0.5 <
    0.6 <= 0.8), random = u * 0.8 is decremented by 0.5 then 0.3."""
    lg = np.log(np.array([0.5, 0.3, 0.2], np.float32))
    assert oracle.sample(lg, 1.0, 0, 0.6, 1.0, [], 0.5) == 0   # 0.40 - 0.5 <= 0
    assert oracle.sample(lg, 1.0, 0, 0.6, 1.0, [], 0.7) == 1   # 0.56 - 0.5 > 0, then <= 0
    assert oracle.sample(lg, 1.0, 0, 0.6, 1.0, [], 0.99) == 1  # never the third
    assert oracle.sample(lg, 1.0, 0, 1.0, 1.0, [], 0.99) == 2  # top_p 1 keeps all three


def test_temperature_divides(oracle):
    """[2, 0] / 2 = [1, 0]: p0 = e / (e + 1) = 0.7311."""
    lg = np.array([2.0, 0.0], np.float32)
    assert oracle.sample(lg, 2.0, 0, 1.0, 1.0, [], 0.72) == 0
    assert oracle.sample(lg, 2.0, 0, 1.0, 1.0, [], 0.74) == 1
    assert oracle.sample(lg, 1.0, 0, 1.0, 1.0, [], 0.74) == 0  # at T = 1, p0 = 0.8808


def test_repetition_penalty_divides_positive_multiplies_negative(oracle):
    """recent {0, 2}, penalty 2: [1.0, 0.9, -0.5, -0.6] -> [0.5, 0.9, -1.0, -0.6],
    sorted 1, 0, 3, 2; the draw walks them in that order."""
    lg = np.array([1.0, 0.9, -0.5, -0.6], np.float32)
    assert oracle.sample(lg, 0.0, 0, 1.0, 2.0, [0, 2], 0.0) == 1
    assert oracle.sample(lg, 0.0, 0, 1.0, 1.0, [0, 2], 0.0) == 0  # penalty 1: off
    p = np.exp(np.array([0.9, 0.5, -0.6, -1.0]))
    p /= p.sum()
    edges = np.concatenate([[0.0], np.cumsum(p)])
    for k, tok in enumerate([1, 0, 3, 2]):
        u = (edges[k] + edges[k + 1]) / 2
        assert oracle.sample(lg, 1.0, 0, 1.0, 2.0, [0, 2, 9999], u) == tok  # 9999: outside the vocabulary


def test_non_finite_values_are_never_drawn(oracle):
    lg = np.array([np.nan, 1.0, np.inf, -np.inf], np.float32)
    for u in (0.0, 0.5, 0.999):
        assert oracle.sample(lg, 1.0, 0, 1.0, 1.0, [], u) == 1
    allinf = np.full(4, -np.inf, np.float32)
    assert oracle.sample(allinf, 1.0, 0, 1.0, 1.0, [], 0.5) == 0  # no finite total: the first


def test_oracle_matches_float64_restatement(oracle):
    rng = np.random.default_rng(17)
    checked = 0
    for trial in range(300):
        n = int(rng.integers(2, 300))
        lg = (rng.standard_normal(n) * rng.choice([0.5, 2.0, 8.0])).astype(np.float32)
        t = float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.7]))
        k = int(rng.choice([0, 1, 5, 40, n]))
        tp = float(rng.choice([0.1, 0.5, 0.9, 1.0]))
        pen = float(rng.choice([1.0, 1.1, 2.0]))
        recent = rng.integers(0, n, int(rng.integers(0, 8))).tolist()
        u = float(rng.random())
        want, margin = f64_sample(lg, t, k, tp, pen, recent, u)
        if margin < 1e-5:
            continue
        assert oracle.sample(lg, t, k, tp, pen, recent, u) == want, (trial, n, t, k, tp, pen, u)
        checked += 1
    assert checked > 250


def test_sampler_window(llrs):
    """The repeat window keeps the last repeat_last_n tokens (src/engine.rs:243-251)."""
    s = llrs.Sampler(llrs.SamplingOptions(), repeat_last_n=3)
    for t in (5, 6, 7, 8):
        s.remember(t)
    assert s.recent_tokens == [6, 7, 8]
    s0 = llrs.Sampler(repeat_last_n=0)
    s0.remember(1)
    assert s0.recent_tokens == []


# ------------------------------------------------------------ device sampler

@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [1000, 152064])
def test_device_sampler_matches_oracle(llrs, backend, oracle, tmp_path, vocab):
    cfg = llrs.SynthConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=1, vocab_size=vocab,
                           max_position_embeddings=64, recipe=llrs.LoadQuantization.Q4KM, seed=19,
                           tie_word_embeddings=False)
    cfg.write_gguf(tmp_path / "s.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "s.gguf", backend)
    kv = llrs.KVCache(model, 16)
    model.prefill(np.array([3, 14, 15, 92], np.uint32), 0, kv)
    lg = kv.logits()
    rng = np.random.default_rng(vocab)
    recent = rng.integers(0, vocab, 64).tolist()
    checked = 0
    for t in (0.0, 0.05, 0.7, 1.3):
        for k in (0, 1, 40, 1000):
            for tp in (0.5, 0.9, 1.0):
                for pen in (1.0, 1.1):
                    opts = llrs.SamplingOptions(temperature=t, top_p=tp, top_k=k, repetition_penalty=pen)
                    for u in (0.0, 0.137, 0.5, 0.861, 0.9999):
                        want, margin = f64_sample(lg, t, k, tp, pen, recent, u)
                        if margin < 1e-5:
                            continue
                        ref = oracle.sample(lg, t, k, tp, pen, recent, u)
                        assert ref == want
                        got = kv.sample(opts, u, recent)
                        assert got == ref, (t, k, tp, pen, u)
                        checked += 1
    print(f"[sample] vocab {vocab}: {checked} draws compared", flush=True)
    assert checked > 200


@pytest.mark.gpu
def test_device_sampler_validates_options(llrs, backend, tmp_path):
    cfg = llrs.SynthConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=1, vocab_size=500,
                           max_position_embeddings=64, recipe=llrs.LoadQuantization.Q4KM, seed=19,
                           tie_word_embeddings=False)
    cfg.write_gguf(tmp_path / "v.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "v.gguf", backend)
    kv = llrs.KVCache(model, 16)
    model.prefill(np.array([1, 2], np.uint32), 0, kv)
    bad = [dict(temperature=-0.1), dict(temperature=float("nan")), dict(top_p=0.0),
           dict(top_p=1.5), dict(repetition_penalty=0.0), dict(repetition_penalty=float("inf"))]
    for b in bad:
        with pytest.raises(llrs.LlrsError):
            kv.sample(llrs.SamplingOptions(**b), 0.5)
    for u in (-0.1, 1.0):
        with pytest.raises(llrs.LlrsError):
            kv.sample(llrs.SamplingOptions(), u)
    with pytest.raises(llrs.LlrsError):
        kv.sample(llrs.SamplingOptions(), 0.5, np.zeros(65537, np.uint32))
    tok = kv.sample(llrs.SamplingOptions(temperature=0.0), 0.5)
    assert tok == int(np.argmax(kv.logits()))  # distinct logits: the greedy pick


@pytest.mark.gpu
def test_sampling_loop_matches_oracle(llrs, backend, oracle, tmp_path):
    """The interactive loop (src/engine.rs:115-186, 243-325): sample with the
    repeat window, remember the token, feed it back.  Each step the device
    logits stay within 2e-2 of the oracle model's, and the device draw equals
    the oracle sampler's on the same logits and uniform number; that token is
    fed to both models, so a draw within rounding of a boundary (skipped)
    cannot derail the rest."""
    cfg = llrs.SynthConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=2, vocab_size=800,
                           max_position_embeddings=128, recipe=llrs.LoadQuantization.Q4KM, seed=53,
                           tie_word_embeddings=False)
    cfg.write_gguf(tmp_path / "loop.gguf")
    model = llrs.ModelLoader.load(tmp_path / "loop.gguf", backend)
    kv = llrs.KVCache(model, 64)
    om = oracle.load(tmp_path / "loop.gguf")
    om.new_state(64)
    prompt = np.array([11, 403, 77, 5, 260], np.uint32)
    model.prefill(prompt, 0, kv)
    om.prefill(prompt, 0)
    opts = llrs.SamplingOptions(temperature=0.9, top_p=0.95, top_k=50, repetition_penalty=1.15)
    sampler = llrs.Sampler(opts, repeat_last_n=16)
    for t in prompt:
        sampler.remember(int(t))
    rng = np.random.default_rng(53)
    compared = 0
    for step in range(24):
        u = float(rng.random())
        recent = list(sampler.recent_tokens)
        lg = kv.logits()
        assert float(np.abs(lg - om.logits()).max()) <= 2e-2
        want = oracle.sample(lg, opts.temperature, opts.top_k, opts.top_p,
                             opts.repetition_penalty, recent, u)
        _, margin = f64_sample(lg, opts.temperature, opts.top_k, opts.top_p,
                               opts.repetition_penalty, recent, u)
        got = sampler.sample(kv, u)
        if margin >= 1e-4:
            assert got == want, (step, got, want)
            compared += 1
        sampler.remember(want)
        pos = len(prompt) + step
        model.forward_token(want, pos, kv, llrs.LogitsMode.COMPUTE)
        om.forward_token(want, pos)
    print(f"[sample] loop: {compared} of 24 draws compared", flush=True)
    assert compared >= 20
