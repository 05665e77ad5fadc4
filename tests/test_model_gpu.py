"""GPU decode path vs the CPU oracle on synthetic Qwen2 models (MI355X).

Bar (north star): final logits within 2e-2 max-abs of the oracle's, and the
same greedy token ids over 32 decode steps (src/engine.rs:205-216, 233-241).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


def tiny_cfg(llrs, **kw):
    base = dict(hidden_size=256, intermediate_size=768, num_attention_heads=4,
                num_key_value_heads=2, num_hidden_layers=2, vocab_size=1000,
                max_position_embeddings=512, recipe=llrs.LoadQuantization.Q4KM, seed=7,
                tie_word_embeddings=False)
    base.update(kw)
    return llrs.SynthConfig(**base)


def make_pair(llrs, backend, oracle, cfg, path, ctx):
    cfg.write_gguf(path)
    model = llrs.ModelLoader.load_dynamic(path, backend)
    om = oracle.load(path)
    om.new_state(ctx)
    return model, llrs.KVCache(model, ctx), om


def compare_run(llrs, backend, oracle, cfg, path, prompt, n_decode, ctx):
    model, kv, om = make_pair(llrs, backend, oracle, cfg, path, ctx)
    print(f"[model] H={cfg.hidden_size} L={cfg.num_hidden_layers} V={cfg.vocab_size} "
          f"prompt={len(prompt)} decode={n_decode}", flush=True)
    model.prefill(prompt, 0, kv)
    om.prefill(prompt, 0)
    lg, lo = kv.logits(), om.logits()
    err = float(np.abs(lg - lo).max())
    print(f"[model] prefill logits max-abs err {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    assert kv.argmax() == om.argmax()
    got = model.decode_greedy(len(prompt), n_decode, kv)
    want = om.decode_greedy(len(prompt), n_decode)
    print(f"[model] tokens gpu={got[:8].tolist()}... oracle={want[:8].tolist()}...", flush=True)
    np.testing.assert_array_equal(got, want)
    err = float(np.abs(kv.logits() - om.logits()).max())
    print(f"[model] final logits max-abs err {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    n = len(prompt) + n_decode
    for layer in (0, cfg.num_hidden_layers - 1):
        for which in ("k", "v"):
            a, b = kv.layer(layer, which, n), om.kv(layer, which, n)
            assert float(np.abs(a - b).max()) <= 1e-3 * max(1.0, float(np.abs(b).max()))
    return model, kv, om


def test_tiny_q4km_greedy_parity(llrs, backend, oracle, tmp_path):
    cfg = tiny_cfg(llrs)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, 24).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "t.gguf", prompt, 32, 128)


@pytest.mark.parametrize("recipe", ["Q4K", "NONE"])
def test_tiny_other_recipes(llrs, backend, oracle, tmp_path, recipe):
    cfg = tiny_cfg(llrs, recipe=getattr(llrs.LoadQuantization, recipe), tie_word_embeddings=True,
                   num_key_value_heads=1, seed=11)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab_size, 9).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "r.gguf", prompt, 32, 64)


def test_head_dim_64_and_gqa_7(llrs, backend, oracle, tmp_path):
    """0.5B-like head geometry: 14 query heads over 2 KV heads, head_dim 64."""
    cfg = tiny_cfg(llrs, hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                   intermediate_size=1024, num_hidden_layers=1, vocab_size=800, seed=3)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab_size, 40).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "h.gguf", prompt, 32, 96)


def test_head_dim_128_long_context(llrs, backend, oracle, tmp_path):
    """7B-like head_dim 128 over a 330-token context: six attention chunks,
    the current position appended mid-chunk, partials merged across chunks.
    (Seed 24: the oracle's top-2 logit gap stays above 6e-3 on every step, far
    above the logit error, so greedy ties cannot flip a token.)"""
    cfg = tiny_cfg(llrs, hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                   intermediate_size=1024, num_hidden_layers=1, vocab_size=600, seed=24)
    prompt = np.random.default_rng(24).integers(0, cfg.vocab_size, 300).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "l.gguf", prompt, 32, 512)


@pytest.mark.parametrize("recipe", ["Q4KM", "Q4K"])
def test_prefill_continued_after_decode(llrs, backend, oracle, tmp_path, recipe):
    """A conversation's second turn: a 100-token prompt is prefilled, 6 tokens
    are decoded, then a 150-token follow-up is prefilled at position 106 (the
    batched prefill attending back over rows written by both the first
    prefill and the decode steps: its f16 K/V copy converts them), and 8
    more tokens are decoded; logits after each prefill, every greedy token
    and the K/V rows match the oracle run through the same calls
    (CausalModel::prefill with start_pos > 0, src/architecture.rs:60-77)."""
    cfg = tiny_cfg(llrs, hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                   intermediate_size=2048, num_hidden_layers=2, vocab_size=700, seed=67,
                   recipe=getattr(llrs.LoadQuantization, recipe))
    model, kv, om = make_pair(llrs, backend, oracle, cfg, tmp_path / "c.gguf", 320)
    rng = np.random.default_rng(67)
    p1 = rng.integers(0, cfg.vocab_size, 100).astype(np.uint32)
    p2 = rng.integers(0, cfg.vocab_size, 150).astype(np.uint32)
    model.prefill(p1, 0, kv)
    om.prefill(p1, 0)
    assert float(np.abs(kv.logits() - om.logits()).max()) <= LOGIT_TOL
    got = model.decode_greedy(100, 6, kv)
    np.testing.assert_array_equal(got, om.decode_greedy(100, 6))
    model.prefill(p2, 106, kv)
    om.prefill(p2, 106)
    err = float(np.abs(kv.logits() - om.logits()).max())
    print(f"[turn2] {recipe}: logits max-abs err after the second prefill {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    got = model.decode_greedy(256, 8, kv)
    np.testing.assert_array_equal(got, om.decode_greedy(256, 8))
    for layer in range(cfg.num_hidden_layers):
        for which in ("k", "v"):
            a, b = kv.layer(layer, which, 264), om.kv(layer, which, 264)
            assert float(np.abs(a - b).max()) <= 1e-3 * max(1.0, float(np.abs(b).max()))


@pytest.mark.parametrize("recipe,ffn,n", [("Q4KM", 18944, 512), ("Q4K", 18944, 512), ("Q4K", 2048, 40)],
                         ids=["q4km_7b_width", "q4k_7b_width", "q4k_split_k"])
def test_prefill_dual_gate_up(llrs, backend, oracle, tmp_path, monkeypatch, recipe, ffn, n):
    """Gate and up as one dual product (each 128-row tile holds 64 gate rows and
    the same 64 up rows) with SwiGLU in its epilogue, against the separate
    products and SwiGLU kernel (LLRS_PREFILL_DUAL=0) and the oracle.  Hidden
    1,536 (24 K chunks): at the 7B FFN width and 512 tokens the 296 dual
    tiles x 4 token tiles run as two rounds of tiles plus a last launch of
    40 with K split 3 ways (its reduction applies SwiGLU); at 40 tokens the
    whole product splits K 4 ways.  The q4k recipe also writes ffn_down's
    activation sums (Q4_K down) in the epilogue and in the reduction."""
    cfg = tiny_cfg(llrs, hidden_size=1536, num_attention_heads=12, num_key_value_heads=2,
                   intermediate_size=ffn, num_hidden_layers=2, max_position_embeddings=1024, seed=71,
                   recipe=getattr(llrs.LoadQuantization, recipe))
    cfg.write_gguf(tmp_path / "d.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "d.gguf", backend)
    om = oracle.load(tmp_path / "d.gguf")
    om.new_state(n + 16)
    prompt = np.random.default_rng(71).integers(0, cfg.vocab_size, n).astype(np.uint32)
    om.prefill(prompt, 0)
    kvs = []
    for dual in ("1", "0"):
        monkeypatch.setenv("LLRS_PREFILL_DUAL", dual)
        kv = llrs.KVCache(model, n + 16)
        model.prefill(prompt, 0, kv)
        kvs.append(kv)
    monkeypatch.delenv("LLRS_PREFILL_DUAL")
    lo = om.logits()
    errs = [float(np.abs(kv.logits() - lo).max()) for kv in kvs]
    diff = float(np.abs(kvs[0].logits() - kvs[1].logits()).max())
    print(f"[dual] {recipe} F={ffn} n={n}: logits err dual {errs[0]:.3e} separate {errs[1]:.3e}, "
          f"dual vs separate {diff:.3e}", flush=True)
    assert max(errs) <= LOGIT_TOL
    assert diff <= 1e-3
    for kv in kvs:
        assert kv.argmax() == om.argmax()
        for which in ("k", "v"):  # layer 1's rows depend on layer 0's FFN
            a, b = kv.layer(1, which, n), om.kv(1, which, n)
            assert float(np.abs(a - b).max()) <= 1e-3 * max(1.0, float(np.abs(b).max()))


@pytest.mark.parametrize("recipe,hidden,n", [("Q4KM", 1024, 40), ("Q4K", 1024, 300), ("Q4K", 256, 40)],
                         ids=["q_k_split_k", "q_k_v_split_k", "q_k_v_direct"])
def test_prefill_qkv_segmented(llrs, backend, oracle, tmp_path, monkeypatch, recipe, hidden, n):
    """Q and K (q4km: V is Q8_0) or Q, K and V (q4k) as one segmented Q4_K
    product, each 128-row tile in one segment, against the separate products
    (LLRS_PREFILL_QKV=0) and the oracle: hidden 1,024 splits K (the reduction
    writes each segment's columns to its own output with its bias), hidden 256
    does not (each tile writes its segment directly).  Layer 0's K and V rows
    come straight from the product."""
    cfg = tiny_cfg(llrs, hidden_size=hidden, num_attention_heads=hidden // 64 if hidden < 1024 else 8,
                   num_key_value_heads=2, intermediate_size=1024, num_hidden_layers=2, seed=73,
                   recipe=getattr(llrs.LoadQuantization, recipe))
    cfg.write_gguf(tmp_path / "q.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "q.gguf", backend)
    om = oracle.load(tmp_path / "q.gguf")
    om.new_state(n + 16)
    prompt = np.random.default_rng(73).integers(0, cfg.vocab_size, n).astype(np.uint32)
    om.prefill(prompt, 0)
    kvs = []
    for seg in ("1", "0"):
        monkeypatch.setenv("LLRS_PREFILL_QKV", seg)
        kv = llrs.KVCache(model, n + 16)
        model.prefill(prompt, 0, kv)
        kvs.append(kv)
    monkeypatch.delenv("LLRS_PREFILL_QKV")
    lo = om.logits()
    errs = [float(np.abs(kv.logits() - lo).max()) for kv in kvs]
    diff = float(np.abs(kvs[0].logits() - kvs[1].logits()).max())
    print(f"[qkv] {recipe} H={hidden} n={n}: logits err segmented {errs[0]:.3e} separate {errs[1]:.3e}, "
          f"segmented vs separate {diff:.3e}", flush=True)
    assert max(errs) <= LOGIT_TOL
    assert diff <= 1e-3
    for kv in kvs:
        assert kv.argmax() == om.argmax()
        for layer in range(cfg.num_hidden_layers):
            for which in ("k", "v"):
                a, b = kv.layer(layer, which, n), om.kv(layer, which, n)
                assert float(np.abs(a - b).max()) <= 1e-3 * max(1.0, float(np.abs(b).max()))


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_prefill_attention_f16_and_f32(llrs, backend, oracle, tmp_path, monkeypatch, hd):
    """The batched prefill's two attention kernels -- f16 hi/lo MFMAs over the
    blocked f16 copy of the layer's K/V rows (the default) and f32 MFMAs over
    the cache (LLRS_PREFILL_ATTN=f32) -- on a 600-token prompt (two chunks, the
    second attending back into the first chunk's rows; a ragged last 16-key
    block): both within the logits bar of the oracle, K/V within 1e-3, and
    within 1e-3 of each other."""
    cfg = tiny_cfg(llrs, hidden_size=hd * 8, num_attention_heads=8, num_key_value_heads=2,
                   intermediate_size=1024, num_hidden_layers=2, vocab_size=600, seed=61,
                   max_position_embeddings=1024)
    cfg.write_gguf(tmp_path / "a.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "a.gguf", backend)
    om = oracle.load(tmp_path / "a.gguf")
    om.new_state(640)
    prompt = np.random.default_rng(61).integers(0, cfg.vocab_size, 600).astype(np.uint32)
    om.prefill(prompt, 0)
    kvs = []
    for mode in ("f16", "f32"):
        if mode == "f32":
            monkeypatch.setenv("LLRS_PREFILL_ATTN", "f32")
        kv = llrs.KVCache(model, 640)
        model.prefill(prompt, 0, kv)
        kvs.append(kv)
    monkeypatch.delenv("LLRS_PREFILL_ATTN")
    lo = om.logits()
    errs = [float(np.abs(kv.logits() - lo).max()) for kv in kvs]
    diff = float(np.abs(kvs[0].logits() - kvs[1].logits()).max())
    print(f"[attn] hd={hd} logits err f16 {errs[0]:.3e} f32 {errs[1]:.3e}, f16 vs f32 {diff:.3e}", flush=True)
    assert max(errs) <= LOGIT_TOL
    assert diff <= 1e-3
    for kv in kvs:
        assert kv.argmax() == om.argmax()
        for layer in range(cfg.num_hidden_layers):
            for which in ("k", "v"):
                a, b = kv.layer(layer, which, 600), om.kv(layer, which, 600)
                assert float(np.abs(a - b).max()) <= 1e-3 * max(1.0, float(np.abs(b).max()))


def test_attention_task_sizes_across_2048(llrs, backend, oracle, tmp_path):
    """Attention items merge in tasks of T items (in LDS), then across a
    head's tasks (through the scratch partials).  At head_dim 128 a head of
    64 chunks (up to position 2,047) runs tasks of 4 items, from 65 chunks
    tasks of 8.  The decode runs from position 2,030 across 2,048.  (Seed 43:
    the oracle's top-2 logit gap stays above 4.5e-3 on every step.)"""
    cfg = tiny_cfg(llrs, hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                   intermediate_size=1024, num_hidden_layers=1, vocab_size=600,
                   max_position_embeddings=4096, seed=43)
    prompt = np.random.default_rng(43).integers(0, cfg.vocab_size, 2030).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "s.gguf", prompt, 32, 2200)


def test_gqa_16_head_dim_32(llrs, backend, oracle, tmp_path):
    """The widest supported group: 16 query heads on one KV head, head_dim 32."""
    cfg = tiny_cfg(llrs, hidden_size=512, num_attention_heads=16, num_key_value_heads=1,
                   intermediate_size=512, num_hidden_layers=2, vocab_size=500, seed=23)
    prompt = np.random.default_rng(23).integers(0, cfg.vocab_size, 70).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "g.gguf", prompt, 32, 128)


def test_prefill_128_token_tiles(llrs, backend, oracle, tmp_path):
    """A 300-token prompt through FFN matrices of 8192 rows: the batched prefill
    takes its 128-token GEMM tiles there (64-token tiles elsewhere) and still
    matches the oracle."""
    cfg = tiny_cfg(llrs, intermediate_size=8192, num_hidden_layers=1, seed=31)
    prompt = np.random.default_rng(31).integers(0, cfg.vocab_size, 300).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "w.gguf", prompt, 8, 320)


def test_prefill_split_last_round(llrs, backend, oracle, tmp_path):
    """A 512-token prompt through FFN matrices of 18944 rows (the 7B width): gate
    and up have 148 x 4 = 592 tiles of 128 rows x 128 tokens, more than the 512
    workgroup slots of a 256-CU part, so the last 80 run as their own launch
    with K split over the slots (the bias-free products start from zeros
    there); prefill, decode and KV still match the oracle (the oracle's
    smallest top-2 logit gap over the 9 greedy steps is 6.9e-3)."""
    cfg = tiny_cfg(llrs, intermediate_size=18944, num_hidden_layers=1, max_position_embeddings=1024,
                   seed=37)
    prompt = np.random.default_rng(37).integers(0, cfg.vocab_size, 512).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "s.gguf", prompt, 8, 528)


def test_prefill_two_chunks_head_dim_16(llrs, backend, oracle, tmp_path):
    """A 600-token prompt goes through the batched prefill as a 512-row chunk
    and an 88-row chunk starting at position 512, whose attention tiles reach
    back into the first chunk's cache rows; head_dim 16 (16 heads over 4 KV
    heads) takes the smallest attention tile kernel and the per-phase decode.
    (Seed 47: the oracle's smallest top-2 logit gap over the 9 greedy steps
    is 2.7e-2.)"""
    cfg = tiny_cfg(llrs, num_attention_heads=16, num_key_value_heads=4, max_position_embeddings=1024,
                   seed=47)
    prompt = np.random.default_rng(47).integers(0, cfg.vocab_size, 600).astype(np.uint32)
    compare_run(llrs, backend, oracle, cfg, tmp_path / "c.gguf", prompt, 8, 640)


def test_forward_token_matches_prefill(llrs, backend, oracle, tmp_path, monkeypatch):
    """The batched (MFMA) prefill agrees with the token-by-token loop of
    CausalModel::prefill (src/architecture.rs:60-77) within the logits bar;
    the token-by-token prefill is bit-identical to forward_token calls."""
    cfg = tiny_cfg(llrs, seed=13)
    cfg.write_gguf(tmp_path / "f.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "f.gguf", backend)
    prompt = np.array([5, 17, 999, 0, 42, 7, 7, 300], np.uint32)
    kv1, kv2, kv3 = (llrs.KVCache(model, 32) for _ in range(3))
    model.prefill(prompt, 0, kv1)
    for i, t in enumerate(prompt):
        model.forward_token(int(t), i, kv2,
                            llrs.LogitsMode.COMPUTE if i + 1 == len(prompt) else llrs.LogitsMode.SKIP)
    monkeypatch.setenv("LLRS_PREFILL_TOKENWISE", "1")
    model.prefill(prompt, 0, kv3)
    np.testing.assert_array_equal(kv3.logits(), kv2.logits())
    err = float(np.abs(kv1.logits() - kv2.logits()).max())
    print(f"[model] batched vs token-by-token prefill logits max-abs {err:.3e}", flush=True)
    assert err <= LOGIT_TOL
    assert kv1.argmax() == kv2.argmax()
    n = len(prompt)
    for which in ("k", "v"):
        a, b = kv1.layer(1, which, n), kv2.layer(1, which, n)
        assert float(np.abs(a - b).max()) <= 1e-2 * max(1.0, float(np.abs(b).max()))
    # Both leave the same device state for decoding on.
    np.testing.assert_array_equal(model.decode_greedy(n, 8, kv1), model.decode_greedy(n, 8, kv2))


@pytest.mark.parametrize("geom", [
    dict(),                                                   # Q4_K / Q8_0 V / Q6_K down, head_dim 64
    dict(hidden_size=512, intermediate_size=1024, seed=3),    # head_dim 128
    dict(hidden_size=384, num_attention_heads=6, intermediate_size=1024, seed=5),  # Q5_0 fallback
    dict(recipe=None, seed=9),                                # uniform Q4_K
], ids=["q4km_hd64", "q4km_hd128", "q4km_q5_0", "q4k"])
def test_persistent_decode_matches_per_phase(llrs, backend, oracle, tmp_path, monkeypatch, geom):
    """The persistent decode kernel (every layer in one launch, device-wide
    barriers between phases) computes bit-identical logits, tokens and KV
    rows to the launch-per-phase path: the same per-row arithmetic, only
    scheduled differently.  Both decode the oracle's greedy tokens."""
    if geom.get("recipe", 0) is None:
        geom = dict(geom, recipe=llrs.LoadQuantization.Q4K)
    cfg = tiny_cfg(llrs, **geom)
    cfg.write_gguf(tmp_path / "p.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "p.gguf", backend)
    om = oracle.load(tmp_path / "p.gguf")
    om.new_state(96)
    ctx = 96
    kv_p = llrs.KVCache(model, ctx)
    monkeypatch.setenv("LLRS_NO_PERSISTENT", "1")
    kv_s = llrs.KVCache(model, ctx)
    monkeypatch.delenv("LLRS_NO_PERSISTENT")
    assert kv_p.persistent and not kv_s.persistent
    prompt = np.array([3, 77, 512, 9, 1, 640], np.uint32)
    for i, t in enumerate(prompt):  # token-wise: every step through the decode kernels
        for kv in (kv_p, kv_s):
            model.forward_token(int(t), i, kv, llrs.LogitsMode.COMPUTE)
        om.forward_token(int(t), i)
        np.testing.assert_array_equal(kv_p.logits(), kv_s.logits())
        assert float(np.abs(kv_p.logits() - om.logits()).max()) <= LOGIT_TOL
    # 40 greedy steps cross the 32-position attention chunk boundary.
    got = model.decode_greedy(len(prompt), 40, kv_p)
    want = model.decode_greedy(len(prompt), 40, kv_s)
    print(f"[persistent] tokens {got[:8].tolist()}...", flush=True)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got, om.decode_greedy(len(prompt), 40))
    assert float(np.abs(kv_p.logits() - om.logits()).max()) <= LOGIT_TOL
    np.testing.assert_array_equal(kv_p.logits(), kv_s.logits())
    n = len(prompt) + 40
    for layer in (0, cfg.num_hidden_layers - 1):
        for which in ("k", "v"):
            np.testing.assert_array_equal(kv_p.layer(layer, which, n), kv_s.layer(layer, which, n))


@pytest.mark.parametrize("case", [
    dict(geom=dict(seed=21), prompt=1000, steps=48),
    dict(geom=dict(hidden_size=1024, num_attention_heads=16, num_key_value_heads=2, intermediate_size=1024,
                   num_hidden_layers=1, vocab_size=600, seed=22), prompt=4080, steps=32),
], ids=["split_at_1024", "multi_chunk_at_4096"])
def test_persistent_split_loads_match_per_phase(llrs, backend, tmp_path, monkeypatch, case):
    """From 1,024 positions the persistent kernel issues an attention item's
    key rows before the phase barrier and its value rows after it (below
    1,024 both before); past 2,048 items (16 heads at 4,096 positions) the
    multi-chunk instantiation does the same for its first sub-chunk.  The
    per-phase path loads both inside its attention launch.  Decoding across
    either position on both paths gives bit-identical tokens, logits and K/V
    rows."""
    cfg = tiny_cfg(llrs, max_position_embeddings=8192, **case["geom"])
    cfg.write_gguf(tmp_path / "s.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "s.gguf", backend)
    ctx = case["prompt"] + case["steps"] + 8
    kv_p = llrs.KVCache(model, ctx)
    monkeypatch.setenv("LLRS_NO_PERSISTENT", "1")
    kv_s = llrs.KVCache(model, ctx)
    monkeypatch.delenv("LLRS_NO_PERSISTENT")
    assert kv_p.persistent and not kv_s.persistent
    prompt = np.random.default_rng(case["geom"]["seed"]).integers(0, cfg.vocab_size, case["prompt"]).astype(np.uint32)
    print(f"[split loads] prompt {len(prompt)} steps {case['steps']}", flush=True)
    for kv in (kv_p, kv_s):
        model.prefill(prompt, 0, kv)
    got = model.decode_greedy(len(prompt), case["steps"], kv_p)
    want = model.decode_greedy(len(prompt), case["steps"], kv_s)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(kv_p.logits(), kv_s.logits())
    n = len(prompt) + case["steps"]
    for layer in (0, cfg.num_hidden_layers - 1):
        for which in ("k", "v"):
            np.testing.assert_array_equal(kv_p.layer(layer, which, n), kv_s.layer(layer, which, n))


def test_model_error_paths(llrs, backend, tmp_path):
    cfg = tiny_cfg(llrs, seed=17)
    cfg.write_gguf(tmp_path / "e.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "e.gguf", backend)
    kv = llrs.KVCache(model, 16)
    with pytest.raises(llrs.LlrsError, match="outside vocabulary"):
        model.forward_token(cfg.vocab_size, 0, kv)
    with pytest.raises(llrs.LlrsError, match="exceeds configured context"):
        model.forward_token(1, 16, kv)
    with pytest.raises(llrs.LlrsError, match="exceeds model limit"):
        llrs.KVCache(model, cfg.max_position_embeddings + 1)
    with pytest.raises(llrs.LlrsError, match="at least one token"):
        model.prefill(np.zeros(0, np.uint32), 0, kv)
    with pytest.raises(llrs.LlrsError, match="exceed context"):
        model.decode_greedy(10, 7, kv)


def test_config3_qwen05b_shape_greedy_parity(llrs, backend, oracle, tmp_path):
    """Benchmark config 3: Qwen2.5-0.5B shape, q4km, 128-token random prompt, 32 greedy steps."""
    cfg = llrs.SynthConfig(hidden_size=896, intermediate_size=4864, num_attention_heads=14,
                           num_key_value_heads=2, num_hidden_layers=24, vocab_size=151936,
                           max_position_embeddings=32768, rope_theta=1e6, rms_norm_eps=1e-6,
                           tie_word_embeddings=True, recipe=llrs.LoadQuantization.Q4KM, seed=3)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab_size, 128).astype(np.uint32)
    model, kv, om = compare_run(llrs, backend, oracle, cfg, tmp_path / "c3.gguf", prompt, 32, 4096)
    QT = llrs.QuantType
    # The q4km recipe at this shape: Q5_0 fallback (896 % 256 != 0), Q8_0 V/embeddings, Q6_K down.
    for name, qt in (("blk.0.attn_q.weight", QT.Q5_0), ("blk.0.ffn_gate.weight", QT.Q5_0),
                     ("blk.0.attn_v.weight", QT.Q8_0), ("token_embd.weight", QT.Q8_0),
                     ("blk.0.ffn_down.weight", QT.Q6K)):
        assert llrs.gguf_read_tensor(tmp_path / "c3.gguf", name)[1].quant_type == qt, name


@pytest.mark.parametrize("n_prompt", [70, 2100], ids=["one_task", "many_tasks"])
@pytest.mark.parametrize("decode_path", ["persistent", "per_phase"])
def test_softmax_uniform_fallback_on_gpu(llrs, backend, oracle, tmp_path, monkeypatch, decode_path, n_prompt):
    """A NaN query bias in layer 0 makes every score NaN: the GPU attention must
    fall back to the plain V mean as softmax_inplace does (src/model.rs:305-312).
    Covered: one position (single chunk); a 70-token prompt fed token by token
    through the decode step (from position 64 on, three 32-position chunks are
    merged, each chunk's partial non-finite); the batched prefill's attention
    tiles; then 8 decode steps from position 70, every step's logits against
    the oracle's.  A 2,100-token prompt then decodes past 2,100 positions
    (66 chunks per head at head_dim 64: 33 tasks of 2 items, whose LDS
    merges and the head's fold see non-finite partials, and the last task
    sums every task's V sums; the 70-token run has one task per head).  Once on the persistent decode kernel, once on the launch-per-phase
    path."""
    cfg = tiny_cfg(llrs, seed=29, num_hidden_layers=2, max_position_embeddings=4096)
    path = tmp_path / "n.gguf"
    cfg.write_gguf(path)
    _, bias = oracle.gguf_read_f32(path, "blk.0.attn_q.bias")
    raw = bytearray(path.read_bytes())
    old = bias.astype(np.float32).tobytes()
    at = raw.find(old)
    assert at > 0 and raw.find(old, at + 1) < 0
    raw[at:at + len(old)] = np.full(bias.size, np.nan, np.float32).tobytes()
    path.write_bytes(bytes(raw))
    prompt = np.random.default_rng(29).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
    ctx = n_prompt + 58
    if decode_path == "per_phase":
        monkeypatch.setenv("LLRS_NO_PERSISTENT", "1")
    model = llrs.ModelLoader.load_dynamic(path, backend)  # the patched file, not a rewrite
    kv, om = llrs.KVCache(model, ctx), oracle.load(path)
    assert kv.persistent == (decode_path == "persistent")

    def check(what):
        lg, lo = kv.logits(), om.logits()
        assert np.isfinite(lo).all()
        err = float(np.abs(lg - lo).max())
        print(f"[model] nan-q {decode_path} {what}: logits max-abs err {err:.3e}", flush=True)
        assert err <= LOGIT_TOL
        assert kv.argmax() == om.argmax()

    runs = ((1, False), (len(prompt), True), (len(prompt), False)) if n_prompt < 128 else ((len(prompt), False),)
    for n, tokenwise in runs:
        if tokenwise:
            monkeypatch.setenv("LLRS_PREFILL_TOKENWISE", "1")
        model.prefill(prompt[:n], 0, kv)
        monkeypatch.delenv("LLRS_PREFILL_TOKENWISE", raising=False)
        om.new_state(ctx)
        om.prefill(prompt[:n], 0)
        check(f"prompt {n} ({'token by token' if tokenwise else 'batched'})")
    for step in range(8):
        tok = om.argmax()
        pos = len(prompt) + step
        model.forward_token(tok, pos, kv)
        om.forward_token(tok, pos)
        check(f"decode at {pos}")


@pytest.mark.parametrize("flag", [0, 1], ids=["barrier", "attention_merge"])
def test_wait_flag_reported_once_then_recovers(llrs, backend, tmp_path, flag):
    """A device-side wait that gave up (set here from the host) fails the next
    call with LLRS_E_HIP; the flag is then cleared, so a fresh prefill and
    decode compute the same tokens as an untouched cache."""
    cfg = tiny_cfg(llrs, seed=19)
    cfg.write_gguf(tmp_path / "w.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "w.gguf", backend)
    prompt = np.array([11, 22, 33, 44, 55], np.uint32)
    ref = llrs.KVCache(model, 64)
    model.prefill(prompt, 0, ref)
    want = model.decode_greedy(len(prompt), 12, ref)
    kv = llrs.KVCache(model, 64)
    assert kv.persistent
    model.prefill(prompt, 0, kv)
    assert llrs.lib().llrs_kv_debug_set_wait_flag(kv.handle, flag) == 0
    with pytest.raises(llrs.LlrsError, match="timed out"):
        model.decode_greedy(len(prompt), 4, kv)
    model.prefill(prompt, 0, kv)
    np.testing.assert_array_equal(model.decode_greedy(len(prompt), 12, kv), want)
    # llrs_kv_reset clears a pending flag too.
    assert llrs.lib().llrs_kv_debug_set_wait_flag(kv.handle, flag) == 0
    kv.reset()
    model.prefill(prompt, 0, kv)
    np.testing.assert_array_equal(model.decode_greedy(len(prompt), 12, kv), want)


@pytest.mark.parametrize("n,ffn", [(40, 8192), (512, 18944)], ids=["split_k", "last_round_split"])
def test_batched_prefill_is_deterministic(llrs, backend, tmp_path, n, ffn):
    """Two batched prefills of one prompt leave bit-identical K/V rows and
    logits: the split-K GEMM partials are reduced in a fixed order (the
    reference is bit-reproducible for any thread count, src/backend.rs:143-162).
    40 tokens split K over several workgroups for every matrix; 512 tokens
    through FFN matrices of 18,944 rows run gate and up as a full round of
    tiles plus a last round split over the slots."""
    cfg = tiny_cfg(llrs, hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                   intermediate_size=ffn, num_hidden_layers=2, seed=37)
    cfg.write_gguf(tmp_path / "d.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "d.gguf", backend)
    prompt = np.random.default_rng(37).integers(0, cfg.vocab_size, n).astype(np.uint32)
    kvs = [llrs.KVCache(model, 512) for _ in range(2)]
    for kv in kvs:
        model.prefill(prompt, 0, kv)
    np.testing.assert_array_equal(kvs[0].logits().view(np.uint32), kvs[1].logits().view(np.uint32))
    for layer in range(cfg.num_hidden_layers):
        for which in ("k", "v"):
            np.testing.assert_array_equal(kvs[0].layer(layer, which, n).view(np.uint32),
                                          kvs[1].layer(layer, which, n).view(np.uint32))


@pytest.mark.parametrize("n,recipe", [(40, "Q4KM"), (300, "Q4KM"), (256, "Q4K")],
                         ids=["40_q4km", "300_q4km", "256_q4k"])
def test_prefill_gemm_kernels_agree(llrs, backend, tmp_path, monkeypatch, n, recipe):
    """The eight-wave prefill GEMM and the four-wave one (LLRS_PREFILL_GEMM=4)
    run the same MFMA sequence per output on f32 weights (hi + lo planes;
    LLRS_PREFILL_CODES=f32 keeps Q4_K and Q6_K on that product too), so a batched
    prefill leaves bit-identical K/V rows and logits with either: 64- and
    128-token tiles, split K, a ragged last token tile, and the Q4_K, Q6_K,
    Q8_0 and Q5_0 stagings (hidden 384 puts the q4km recipe on its Q5_0
    fallback)."""
    hidden = 384 if n == 300 else 1024
    cfg = tiny_cfg(llrs, hidden_size=hidden, num_attention_heads=hidden // 128 * 2,
                   num_key_value_heads=2, intermediate_size=2048, num_hidden_layers=2, seed=41,
                   recipe=getattr(llrs.LoadQuantization, recipe))
    cfg.write_gguf(tmp_path / "g.gguf")
    model = llrs.ModelLoader.load_dynamic(tmp_path / "g.gguf", backend)
    prompt = np.random.default_rng(41).integers(0, cfg.vocab_size, n).astype(np.uint32)
    kvs = []
    monkeypatch.setenv("LLRS_PREFILL_CODES", "f32")
    for kernel in ("8", "4"):
        monkeypatch.setenv("LLRS_PREFILL_GEMM", kernel)
        kv = llrs.KVCache(model, 512)
        model.prefill(prompt, 0, kv)
        kvs.append(kv)
    monkeypatch.delenv("LLRS_PREFILL_GEMM")
    monkeypatch.delenv("LLRS_PREFILL_CODES")
    print(f"[prefill-kernels] n={n} {recipe}: logits[:3] {kvs[0].logits()[:3]}", flush=True)
    np.testing.assert_array_equal(kvs[0].logits().view(np.uint32), kvs[1].logits().view(np.uint32))
    for layer in range(cfg.num_hidden_layers):
        for which in ("k", "v"):
            np.testing.assert_array_equal(kvs[0].layer(layer, which, n).view(np.uint32),
                                          kvs[1].layer(layer, which, n).view(np.uint32))


def write_q4k_zero_d(llrs, tmp_path, cfg, down_q6k=False):
    """The synthetic model with every matrix quantized to Q4_K on the host (with
    down_q6k, ffn_down to Q6_K), then d set to 0 in chosen 256-column blocks of
    q, o, gate and ffn_down (Q4_K: the block's first f16, dmin kept; Q6_K: its
    last f16): in row r the blocks b with (r + b) % 5 == 0, and every block of
    rows 3 and 4.  value_at (src/quant.rs:349-456) then gives -dmin * m (Q4_K)
    or 0 (Q6_K) for all 256 columns of such a block."""
    from gguf_write import qwen2_metadata, write_gguf
    from hf_checkpoint import gguf_names
    f32 = tmp_path / "f32.gguf"
    llrs.SynthConfig(**{**cfg.__dict__, "recipe": llrs.LoadQuantization.NONE}).write_gguf(f32)
    tensors, zeroed = [], 0
    for name in gguf_names(cfg.num_hidden_layers, tied=False):
        _, t = llrs.gguf_read_tensor(f32, name)
        rows, cols = t.shape if len(t.shape) == 2 else (1, t.shape[0])
        if rows == 1 or not name.endswith(".weight"):
            tensors.append((name, 0, rows, cols, bytes(t.data)))
            continue
        q6 = down_q6k and name.endswith("ffn_down.weight")
        ty = llrs.QuantType.Q6K if q6 else llrs.QuantType.Q4K
        q = llrs.QuantTensor.quantize(ty, np.frombuffer(t.data, np.float32), rows, cols)
        data = bytearray(q.data)
        if any(name.endswith(s) for s in ("attn_q.weight", "attn_output.weight", "ffn_gate.weight",
                                          "ffn_down.weight")):
            bb, doff = (210, 208) if q6 else (144, 0)  # block bytes, offset of d
            nb = cols // 256
            rb = nb * bb
            for r in range(rows):
                for b in range(nb):
                    if (r + b) % 5 == 0 or r in (3, 4):
                        o = r * rb + b * bb + doff
                        data[o:o + 2] = b"\x00\x00"
                        zeroed += 1
        tensors.append((name, int(q.quant_type), rows, cols, bytes(data)))
    assert zeroed > 0
    path = tmp_path / "zero_d.gguf"
    write_gguf(path, qwen2_metadata(cfg), tensors)
    return path


@pytest.mark.parametrize("n,down_q6k", [(40, False), (300, False), (300, True)],
                         ids=["64_token_tiles", "128_token_tiles", "q6k_down"])
def test_prefill_q4k_integer_codes(llrs, backend, oracle, tmp_path, monkeypatch, n, down_q6k):
    """The prefill products on the integer codes -- Q4_K: sc * q as exact f16,
    d applied per 256-column block, the dmin * m term from 32-column
    activation sums; Q6_K (ffn_down in the q6k_down case): sc * (q - 32) as
    f16 hi + lo, d per block -- on a model whose q, o, gate and ffn_down have
    blocks with d = 0, among them the first and the last block of a row and
    whole rows: within the logits bar of the oracle (and K/V within 1e-3),
    within 1e-3 of the f32-weight products (LLRS_PREFILL_CODES=f32), and
    bit-identical from run to run.  Hidden 1,024 (4 blocks a row) and FFN
    2,048 (ffn_down: 8 a row)."""
    cfg = tiny_cfg(llrs, hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                   intermediate_size=2048, num_hidden_layers=2, seed=53,
                   recipe=llrs.LoadQuantization.Q4K)
    path = write_q4k_zero_d(llrs, tmp_path, cfg, down_q6k)
    model = llrs.ModelLoader.load_dynamic(path, backend)
    om = oracle.load(path)
    om.new_state(512)
    prompt = np.random.default_rng(53).integers(0, cfg.vocab_size, n).astype(np.uint32)
    kvs = []
    for mode in ("int", "int", "f32"):
        if mode == "f32":
            monkeypatch.setenv("LLRS_PREFILL_CODES", "f32")
        kv = llrs.KVCache(model, 512)
        model.prefill(prompt, 0, kv)
        kvs.append(kv)
    monkeypatch.delenv("LLRS_PREFILL_CODES")
    om.prefill(prompt, 0)
    lo = om.logits()
    err = float(np.abs(kvs[0].logits() - lo).max())
    diff = float(np.abs(kvs[0].logits() - kvs[2].logits()).max())
    print(f"[q4k-int] n={n} logits err vs oracle {err:.3e}, vs f32 product {diff:.3e}", flush=True)
    assert err <= LOGIT_TOL
    assert diff <= 1e-3
    assert kvs[0].argmax() == om.argmax()
    np.testing.assert_array_equal(kvs[0].logits().view(np.uint32), kvs[1].logits().view(np.uint32))
    for layer in range(cfg.num_hidden_layers):
        for which in ("k", "v"):
            a, b = kvs[0].layer(layer, which, n), om.kv(layer, which, n)
            assert float(np.abs(a - b).max()) <= 1e-3 * max(1.0, float(np.abs(b).max()))
            np.testing.assert_array_equal(a.view(np.uint32), kvs[1].layer(layer, which, n).view(np.uint32))


def write_mixed_q4km(llrs, tmp_path, cfg, v_types, down_types):
    """A GGUF laid out like llama.cpp's Q4_K_M files (src/loader.rs:437-441
    keeps such files' tensors verbatim): Q4_K embeddings and q/k/o/gate/up,
    a Q6_K LM head, and per layer the given attn_v / ffn_down types.  The
    weights are the synthetic F32 model's, quantized on the host."""
    from gguf_write import qwen2_metadata, write_gguf
    from hf_checkpoint import gguf_names
    f32 = tmp_path / "f32.gguf"
    llrs.SynthConfig(**{**cfg.__dict__, "recipe": llrs.LoadQuantization.NONE}).write_gguf(f32)
    QT = llrs.QuantType
    tensors = []
    for name in gguf_names(cfg.num_hidden_layers, tied=False):
        _, t = llrs.gguf_read_tensor(f32, name)
        rows, cols = t.shape if len(t.shape) == 2 else (1, t.shape[0])
        vals = np.frombuffer(t.data, np.float32)
        ty = None
        if name.endswith("attn_v.weight"):
            ty = v_types[int(name.split(".")[1])]
        elif name.endswith("ffn_down.weight"):
            ty = down_types[int(name.split(".")[1])]
        elif name == "output.weight":
            ty = QT.Q6K
        elif name.endswith(".weight") and rows > 1:
            ty = QT.Q4K
        if ty is None:
            tensors.append((name, 0, rows, cols, bytes(t.data)))
        else:
            q = llrs.QuantTensor.quantize(ty, vals, rows, cols)
            tensors.append((name, int(q.quant_type), rows, cols, bytes(q.data)))
    path = tmp_path / "mixed.gguf"
    write_gguf(path, qwen2_metadata(cfg), tensors)
    return path


@pytest.mark.parametrize("hidden", [256, 512], ids=["hd64", "hd128"])
def test_persistent_decode_per_layer_type_mix(llrs, backend, oracle, tmp_path, monkeypatch, hidden):
    """Layers whose attn_v and ffn_down types differ (Q4_K / Q6_K / Q8_0 V,
    Q4_K / Q6_K down) select the persistent kernel's per-layer instantiation;
    it matches the oracle over 32 greedy steps and the launch-per-phase path
    bit for bit."""
    QT = llrs.QuantType
    cfg = tiny_cfg(llrs, hidden_size=hidden, intermediate_size=768, num_hidden_layers=4, seed=47)
    v = [QT.Q6K, QT.Q4K, QT.Q8_0, QT.Q6K]
    down = [QT.Q6K, QT.Q4K, QT.Q4K, QT.Q6K]
    path = write_mixed_q4km(llrs, tmp_path, cfg, v, down)
    for l in range(4):
        assert llrs.gguf_read_tensor(path, f"blk.{l}.attn_v.weight")[1].quant_type == v[l]
        assert llrs.gguf_read_tensor(path, f"blk.{l}.ffn_down.weight")[1].quant_type == down[l]
    model = llrs.ModelLoader.load_dynamic(path, backend)
    kv = llrs.KVCache(model, 96)
    assert kv.persistent
    om = oracle.load(path)
    om.new_state(96)
    prompt = np.random.default_rng(47).integers(0, cfg.vocab_size, 24).astype(np.uint32)
    model.prefill(prompt, 0, kv)
    om.prefill(prompt, 0)
    assert float(np.abs(kv.logits() - om.logits()).max()) <= LOGIT_TOL
    got = model.decode_greedy(len(prompt), 32, kv)
    want = om.decode_greedy(len(prompt), 32)
    print(f"[mixed] tokens {got[:8].tolist()}...", flush=True)
    np.testing.assert_array_equal(got, want)
    assert float(np.abs(kv.logits() - om.logits()).max()) <= LOGIT_TOL
    monkeypatch.setenv("LLRS_NO_PERSISTENT", "1")
    kv_s = llrs.KVCache(model, 96)
    monkeypatch.delenv("LLRS_NO_PERSISTENT")
    assert not kv_s.persistent
    model.prefill(prompt, 0, kv_s)
    np.testing.assert_array_equal(model.decode_greedy(len(prompt), 32, kv_s), got)
    np.testing.assert_array_equal(kv_s.logits(), kv.logits())


@pytest.mark.timeout(300)
def test_attention_past_32k_positions(llrs, backend, oracle, tmp_path):
    """At 32K positions with 8 heads an attention item covers
    ceil(chunks x heads / 2,048) consecutive chunks: four up to position
    32,767 (256 items per head), five from 32,768 (205), the persistent
    kernel's multi-chunk instantiation, each head merged in two levels.  A
    32,760-token prompt goes through the
    batched prefill; the oracle is seeded with the GPU's K/V rows of positions
    0..32,749 and computes the last 10 prompt positions itself; then 16 steps
    cross position 32,768 token by token, both sides fed the oracle's greedy
    token (teacher forcing), logits compared at every step and tokens
    wherever the oracle's top-2 gap exceeds 2e-3."""
    cfg = tiny_cfg(llrs, hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                   intermediate_size=1024, num_hidden_layers=1, vocab_size=600,
                   max_position_embeddings=40000, seed=45)
    ctx, n_prompt, own = 32800, 32760, 10
    path = tmp_path / "k32.gguf"
    model, kv, om = make_pair(llrs, backend, oracle, cfg, path, ctx)
    assert kv.persistent
    prompt = np.random.default_rng(45).integers(0, cfg.vocab_size, n_prompt).astype(np.uint32)
    model.prefill(prompt, 0, kv)
    seed_to = n_prompt - own
    for which in ("k", "v"):
        om.load_kv(0, which, kv.layer(0, which, seed_to))
    for i in range(seed_to, n_prompt):
        om.forward_token(int(prompt[i]), i, i + 1 == n_prompt)
    err = float(np.abs(kv.logits() - om.logits()).max())
    print(f"[k32] prefill logits err {err:.2e}", flush=True)
    assert err <= LOGIT_TOL
    tok, checked = om.argmax(), 0
    for i in range(16):
        p = n_prompt + i
        model.forward_token(tok, p, kv)
        om.forward_token(tok, p, True)
        lg, lo = kv.logits(), om.logits()
        err = float(np.abs(lg - lo).max())
        top2 = np.sort(lo.astype(np.float64))[-2:]
        print(f"[k32] position {p} logits err {err:.2e} oracle gap {top2[1] - top2[0]:.2e}", flush=True)
        assert err <= LOGIT_TOL
        if top2[1] - top2[0] > 2e-3:
            assert kv.argmax() == om.argmax()
            checked += 1
        tok = om.argmax()
    assert checked >= 8
    n = n_prompt + 16
    for which in ("k", "v"):
        a, b = kv.layer(0, which, n)[n_prompt:], om.kv(0, which, n)[n_prompt:]
        assert float(np.abs(a - b).max()) <= 1e-3 * max(1.0, float(np.abs(b).max()))
