"""The generation loop on the GPU (llrs_generate: generate_with_metrics' token
loop, src/engine.rs:115-186) against the same loop over the CPU oracle.

The oracle loop below restates the reference: reset, the repeat window seeded
with the prompt's last repeat_last_n tokens (136-143), prefill, then per step
sample_current_logits (the oracle's oq_sample), push, remember (243-251),
stop after an EOS id, else forward at the next position.  The draws are the
caller's; each is placed in the middle of a candidate's probability interval
of the oracle's distribution (a candidate of probability >= 2%), so the
device sampler, whose logits differ from the oracle's by ~1e-4, draws the same
token.  Tokens must be equal, the EOS stop at the same step.
"""
from __future__ import annotations

import numpy as np
import pytest

from test_sampling import f64_sample

pytestmark = pytest.mark.gpu


def central_uniform(lg, opts, recent, rng):
    """A draw in the middle of a random candidate (p >= 2%) of the kept set."""
    v = np.asarray(lg, np.float64).copy()
    seen = np.zeros(v.size, bool)
    seen[[t for t in recent if t < v.size]] = True
    pen, t = opts.repetition_penalty, opts.temperature
    if pen != 1.0:
        v = np.where(seen, np.where(v > 0, v / pen, v * pen), v)
    v = v / t
    order = np.lexsort((np.arange(v.size), -v))
    m = opts.top_k if 0 < opts.top_k < v.size else v.size
    p = np.exp(v[order[:m]] - v[order[0]])
    p /= p.sum()
    cum = np.cumsum(p)
    hit = np.nonzero(cum >= opts.top_p)[0]
    cutoff = int(hit[0]) + 1 if hit.size else m
    kept = cum[cutoff - 1]
    ok = [i for i in range(cutoff) if p[i] >= 0.02]
    i = ok[int(rng.integers(len(ok)))]
    lo = cum[i - 1] if i else 0.0
    return float((lo + p[i] / 2) / kept)


def oracle_generate(oracle, om, prompt, opts, window, eos, max_new, ctx, rng=None, uniforms=None):
    recent = []

    def remember(t):
        if window == 0:
            return
        recent.append(int(t))
        if len(recent) > window:
            recent.pop(0)

    for t in prompt[-window:] if window else []:
        remember(t)
    om.new_state(ctx)
    om.prefill(prompt, 0)
    out, draws = [], []
    for i in range(min(max_new, ctx - len(prompt))):
        lg = om.logits()
        if uniforms is not None:
            u = float(uniforms[i])
        else:
            u = central_uniform(lg, opts, recent, rng) if opts.temperature > 0 else 0.0
        draws.append(u)
        if opts.temperature > 0:
            _, margin = f64_sample(lg, opts.temperature, opts.top_k, opts.top_p,
                                   opts.repetition_penalty, recent, u)
            assert margin > 5e-3, (i, margin)
        tok = oracle.sample(lg, opts.temperature, opts.top_k, opts.top_p, opts.repetition_penalty,
                            recent, u)
        out.append(tok)
        remember(tok)
        if tok in eos:
            break
        om.forward_token(tok, len(prompt) + len(out) - 1)
    return out, np.array(draws, np.float32)


def setup(llrs, backend, oracle, tmp_path, seed):
    cfg = llrs.SynthConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                           num_key_value_heads=2, num_hidden_layers=2, vocab_size=700,
                           max_position_embeddings=256, recipe=llrs.LoadQuantization.Q4KM,
                           seed=seed, tie_word_embeddings=False)
    path = tmp_path / "gen.gguf"
    cfg.write_gguf(path)
    return cfg, llrs.ModelLoader.load(path, backend), oracle.load(path)


def test_generate_sampled_with_eos_stop(llrs, backend, oracle, tmp_path):
    cfg, model, om = setup(llrs, backend, oracle, tmp_path, seed=61)
    opts = llrs.SamplingOptions(temperature=0.8, top_p=0.95, top_k=40, repetition_penalty=1.1)
    prompt = np.random.default_rng(61).integers(0, cfg.vocab_size, 20).astype(np.uint32)
    ctx, window, max_new = 64, 16, 24
    full, draws = oracle_generate(oracle, om, prompt, opts, window, [], max_new, ctx,
                                  rng=np.random.default_rng(7))
    engine = llrs.InferenceEngine(model, ctx, sampling=opts, repeat_last_n=window)
    got = engine.generate_with_metrics(prompt, max_new, uniforms=draws)
    print(f"[generate] gpu {got.token_ids}\n[generate] oracle {full}", flush=True)
    assert got.token_ids == full and not got.stopped_on_eos
    assert got.metrics.prompt_tokens == len(prompt) and got.metrics.generated_tokens == max_new
    # An EOS id first produced at step >= 6 stops both loops there, EOS kept.
    k = next(i for i in range(6, len(full)) if full[i] not in full[:i])
    eos = [full[k], cfg.vocab_size - 1]
    want, _ = oracle_generate(oracle, om, prompt, opts, window, eos, max_new, ctx, uniforms=draws)
    assert want == full[:k + 1]
    engine.eos_token_ids = eos
    got = engine.generate_with_metrics(prompt, max_new, uniforms=draws)
    assert got.token_ids == want and got.stopped_on_eos
    assert got.metrics.generated_tokens == k + 1


def test_generate_greedy_window_and_context_limit(llrs, backend, oracle, tmp_path):
    """Temperature 0 (no draws), a window longer than the prompt, and
    max_new_tokens beyond the context: the loop stops at the context's end."""
    cfg, model, om = setup(llrs, backend, oracle, tmp_path, seed=62)
    opts = llrs.SamplingOptions(temperature=0.0, top_p=0.9, top_k=40, repetition_penalty=1.3)
    prompt = np.random.default_rng(62).integers(0, cfg.vocab_size, 9).astype(np.uint32)
    ctx = 24
    want, _ = oracle_generate(oracle, om, prompt, opts, 64, [], 100, ctx)
    assert len(want) == ctx - len(prompt)
    engine = llrs.InferenceEngine(model, ctx, sampling=opts, repeat_last_n=64)
    got = engine.generate_with_metrics(prompt, 100, uniforms=np.zeros(100))
    assert got.token_ids == want


def test_generate_errors(llrs, backend, oracle, tmp_path):
    cfg, model, _ = setup(llrs, backend, oracle, tmp_path, seed=63)
    engine = llrs.InferenceEngine(model, 16)
    with pytest.raises(llrs.LlrsError, match="empty"):
        engine.generate_with_metrics(np.zeros(0, np.uint32), 4)
    with pytest.raises(llrs.LlrsError, match="but context is 16"):
        engine.generate_with_metrics(np.arange(16, dtype=np.uint32), 4)
    engine.sampling = llrs.SamplingOptions(top_p=0.0)
    with pytest.raises(llrs.LlrsError, match="top_p"):
        engine.generate_with_metrics(np.arange(4, dtype=np.uint32), 4)
