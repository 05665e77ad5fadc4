"""Pins the oracle's model-level arithmetic (oracle/oracle_model.c) with an
independent float64 restatement of Qwen2Model::forward_impl (src/model.rs:135-271).

The reference holds no test of RMSNorm, RoPE, attention, softmax, SwiGLU or
the LM head, so these tests check the oracle against
  - a float64 numpy forward pass written from the model definition (not from
    the oracle's C code) on tiny F32 models: a wrong RoPE pairing or sign, a
    dropped bias, a wrong KV-head mapping or attention scale moves the logits
    by orders of magnitude more than the f32-vs-f64 tolerance;
  - softmax_inplace's uniform fallback (src/model.rs:305-312): a NaN query
    bias makes every score NaN, so the layer's attention output must be the
    plain mean of the V rows;
  - closed forms at position 0: RoPE is the identity and attention returns
    the V row.
"""
from __future__ import annotations

import numpy as np
import pytest

F64 = np.float64


def tiny(llrs, **kw):
    base = dict(hidden_size=64, intermediate_size=96, num_attention_heads=4, num_key_value_heads=2,
                num_hidden_layers=2, vocab_size=128, max_position_embeddings=64,
                recipe=llrs.LoadQuantization.NONE, tie_word_embeddings=False, seed=41,
                weight_std=0.2, rope_theta=10000.0)
    base.update(kw)
    return llrs.SynthConfig(**base)


class F64Qwen2:
    """Qwen2 decode in float64 from the GGUF tensors (llama.cpp tensor names)."""

    def __init__(self, oracle, path, cfg):
        self.c = cfg
        self.hd = cfg.hidden_size // cfg.num_attention_heads
        self.w = {}
        names = ["token_embd.weight", "output_norm.weight"]
        names += [] if cfg.tie_word_embeddings else ["output.weight"]
        for l in range(cfg.num_hidden_layers):
            for n in ("attn_norm.weight", "attn_q.weight", "attn_q.bias", "attn_k.weight",
                      "attn_k.bias", "attn_v.weight", "attn_v.bias", "attn_output.weight",
                      "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"):
                names.append(f"blk.{l}.{n}")
        for n in names:
            _, a = oracle.gguf_read_f32(path, n)
            self.w[n] = a.astype(F64).reshape(a.shape[0], -1) if a.shape[0] > 1 else a.reshape(-1).astype(F64)
        self.k = [[] for _ in range(cfg.num_hidden_layers)]
        self.v = [[] for _ in range(cfg.num_hidden_layers)]
        self.nan_attention_layers = set()

    def vec(self, name):
        return self.w[name].reshape(-1)

    def rmsnorm(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.c.rms_norm_eps) * w

    def rope(self, x, pos):
        hd, half = self.hd, self.hd // 2
        inv = self.c.rope_theta ** (-2.0 * np.arange(half) / hd)
        cs, sn = np.cos(pos * inv), np.sin(pos * inv)
        x = x.reshape(-1, hd)
        a, b = x[:, :half], x[:, half:]
        return np.concatenate([a * cs - b * sn, a * sn + b * cs], axis=1).reshape(-1)

    def forward(self, tok, pos):
        c, hd = self.c, self.hd
        G = c.num_attention_heads // c.num_key_value_heads
        h = self.w["token_embd.weight"][tok].copy()
        for l in range(c.num_hidden_layers):
            p = f"blk.{l}."
            x = self.rmsnorm(h, self.vec(p + "attn_norm.weight"))
            q = self.w[p + "attn_q.weight"] @ x + self.vec(p + "attn_q.bias")
            k = self.w[p + "attn_k.weight"] @ x + self.vec(p + "attn_k.bias")
            v = self.w[p + "attn_v.weight"] @ x + self.vec(p + "attn_v.bias")
            q, k = self.rope(q, pos), self.rope(k, pos)
            self.k[l].append(k)
            self.v[l].append(v)
            K, V = np.stack(self.k[l]), np.stack(self.v[l])  # [pos+1, kv_width]
            out = np.empty(c.hidden_size)
            for head in range(c.num_attention_heads):
                kvh = head // G
                kh, vh = K[:, kvh * hd:(kvh + 1) * hd], V[:, kvh * hd:(kvh + 1) * hd]
                if l in self.nan_attention_layers:
                    wts = np.full(pos + 1, 1.0 / (pos + 1))  # softmax_inplace fallback
                else:
                    s = kh @ q[head * hd:(head + 1) * hd] / np.sqrt(hd)
                    e = np.exp(s - s.max())
                    wts = e / e.sum()
                out[head * hd:(head + 1) * hd] = wts @ vh
            h = h + self.w[p + "attn_output.weight"] @ out
            x = self.rmsnorm(h, self.vec(p + "ffn_norm.weight"))
            g = self.w[p + "ffn_gate.weight"] @ x
            u = self.w[p + "ffn_up.weight"] @ x
            h = h + self.w[p + "ffn_down.weight"] @ (g / (1.0 + np.exp(-g)) * u)
        x = self.rmsnorm(h, self.vec("output_norm.weight"))
        head_w = self.w["token_embd.weight" if c.tie_word_embeddings else "output.weight"]
        return head_w @ x


def run_both(oracle, model64, path, tokens):
    om = oracle.load(path)
    om.new_state(len(tokens) + 1)
    for pos, t in enumerate(tokens):
        om.forward_token(int(t), pos, True)
        want = model64.forward(int(t), pos)
        got = om.logits().astype(F64)
        err = np.abs(got - want).max() / max(1.0, np.abs(want).max())
        print(f"[oracle-f64] pos {pos} max rel err {err:.2e}", flush=True)
        assert err < 2e-5, (pos, err)
    return om


@pytest.mark.parametrize("kw", [dict(), dict(num_key_value_heads=1, tie_word_embeddings=True, seed=43),
                                dict(num_attention_heads=8, num_key_value_heads=8, seed=47)])
def test_oracle_forward_matches_float64_restatement(llrs, oracle, tmp_path, kw):
    cfg = tiny(llrs, **kw)
    path = tmp_path / "m.gguf"
    cfg.write_gguf(path)
    tokens = np.random.default_rng(cfg.seed).integers(0, cfg.vocab_size, 12)
    run_both(oracle, F64Qwen2(oracle, path, cfg), path, tokens)


def test_float64_check_is_sensitive(llrs, oracle, tmp_path):
    """The comparison above fails for a plausible slip: interleaved (GPT-J)
    instead of split-half RoPE pairing."""
    cfg = tiny(llrs)
    path = tmp_path / "m.gguf"
    cfg.write_gguf(path)
    m = F64Qwen2(oracle, path, cfg)

    def interleaved(x, pos, hd=m.hd):
        inv = cfg.rope_theta ** (-2.0 * np.arange(hd // 2) / hd)
        cs, sn = np.cos(pos * inv), np.sin(pos * inv)
        x = x.reshape(-1, hd // 2, 2)
        a, b = x[..., 0], x[..., 1]
        return np.stack([a * cs - b * sn, a * sn + b * cs], axis=-1).reshape(-1)

    m.rope = interleaved
    om = oracle.load(path)
    om.new_state(8)
    errs = []
    for pos, t in enumerate([3, 9, 27, 81]):
        om.forward_token(t, pos, True)
        want = m.forward(t, pos)
        errs.append(np.abs(om.logits() - want).max() / max(1.0, np.abs(want).max()))
    assert errs[0] < 2e-5  # position 0: every rotation is the identity
    assert max(errs[1:]) > 1e-3


def nan_q_bias(llrs, oracle, tmp_path, layer=0):
    """A GGUF whose layer-`layer` query bias is NaN: every score of that layer is NaN."""
    cfg = tiny(llrs, seed=53)
    path = tmp_path / "n.gguf"
    cfg.write_gguf(path)
    _, bias = oracle.gguf_read_f32(path, f"blk.{layer}.attn_q.bias")
    raw = bytearray(path.read_bytes())
    old = bias.astype(np.float32).tobytes()
    at = raw.find(old)
    assert at > 0 and raw.find(old, at + 1) < 0
    raw[at:at + len(old)] = np.full(bias.size, np.nan, np.float32).tobytes()
    path.write_bytes(bytes(raw))
    return cfg, path


def test_softmax_uniform_fallback(llrs, oracle, tmp_path):
    cfg, path = nan_q_bias(llrs, oracle, tmp_path)
    m = F64Qwen2(oracle, path, cfg)
    m.nan_attention_layers = {0}
    tokens = np.random.default_rng(5).integers(0, cfg.vocab_size, 6)
    om = run_both(oracle, m, path, tokens)
    assert np.isfinite(om.logits()).all()


def test_position_zero_closed_forms(llrs, oracle, tmp_path):
    """At position 0 the cached key is the unrotated k projection and the
    attention output is the V row, so the oracle's cache equals the plain
    projections of the normed embedding."""
    cfg = tiny(llrs, num_hidden_layers=1, seed=59)
    path = tmp_path / "z.gguf"
    cfg.write_gguf(path)
    m = F64Qwen2(oracle, path, cfg)
    om = oracle.load(path)
    om.new_state(4)
    om.forward_token(17, 0, True)
    x = m.rmsnorm(m.w["token_embd.weight"][17], m.vec("blk.0.attn_norm.weight"))
    k = m.w["blk.0.attn_k.weight"] @ x + m.vec("blk.0.attn_k.bias")
    v = m.w["blk.0.attn_v.weight"] @ x + m.vec("blk.0.attn_v.bias")
    np.testing.assert_allclose(om.kv(0, "k", 1).reshape(-1), k, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(om.kv(0, "v", 1).reshape(-1), v, rtol=1e-5, atol=1e-6)
