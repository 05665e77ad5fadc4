"""The engine's end-of-sequence discovery (find_eos_tokens, src/engine.rs:340-387),
host only.

Pinned by the `tokenizers` Python package: it wraps the Rust `tokenizers`
crate the reference depends on (Cargo.toml:15 asks for 0.19; the package
here is 0.22, whose token_to_id keeps the same order: added tokens, then the
model's vocabulary), so Tokenizer.token_to_id there is the reference's own
lookup, run on the same tokenizer.json files.  generation_config.json cases follow serde_json's
as_u64 + u32::try_from (non-negative integers below 2^32 count; floats,
negatives, larger values and non-numbers are skipped).
"""
from __future__ import annotations

import json

import pytest

tokenizers = pytest.importorskip("tokenizers")


def bpe_tokenizer(vocab: dict, added: list) -> "tokenizers.Tokenizer":
    from tokenizers import AddedToken, Tokenizer
    from tokenizers.models import BPE
    tok = Tokenizer(BPE(vocab=vocab, merges=[]))
    tok.add_special_tokens([AddedToken(t, special=True) for t in added])
    return tok


def unigram_tokenizer(pieces: list) -> "tokenizers.Tokenizer":
    from tokenizers import Tokenizer
    from tokenizers.models import Unigram
    return Tokenizer(Unigram([(p, -1.0) for p in pieces]))


def reference_eos(tok, gen_config) -> list[int]:
    """find_eos_tokens restated over the package's token_to_id."""
    ids = []
    if gen_config is not None:
        eos = gen_config.get("eos_token_id")
        vals = eos if isinstance(eos, list) else [eos]
        for v in vals:
            if isinstance(v, int) and not isinstance(v, bool) and 0 <= v < 2 ** 32:
                ids.append(v)
    for t in ("<|im_end|>", "<|endoftext|>"):
        i = tok.token_to_id(t)
        if i is not None:
            ids.append(i)
    return sorted(set(ids))


def write_dir(tmp_path, tok, gen_config, raw_gen=None):
    tok.save(str(tmp_path / "tokenizer.json"))
    if raw_gen is not None:
        (tmp_path / "generation_config.json").write_text(raw_gen)
    elif gen_config is not None:
        (tmp_path / "generation_config.json").write_text(json.dumps(gen_config))
    return tmp_path


VOCAB = {"a": 0, "b": 1, "<|endoftext|>": 7, "c": 2, "<|im_end|>": 9, "d": 3}


@pytest.mark.parametrize("gen", [None, {"eos_token_id": 5}, {"eos_token_id": [5, 9, 2 ** 32, -1, 1.5, "x", 7]},
                                 {"eos_token_id": "7"}, {"bos_token_id": 1}, {"eos_token_id": [151645, 151643]}],
                         ids=["no_config", "number", "array_mixed", "string", "no_eos_key", "qwen"])
def test_eos_from_vocab_and_generation_config(llrs, tmp_path, gen):
    # the special tokens live in the model vocabulary here (not added tokens)
    tok = bpe_tokenizer(VOCAB, [])
    d = write_dir(tmp_path, tok, gen)
    assert llrs.find_eos_tokens(d) == reference_eos(tok, gen)
    # A file path resolves to its directory (model_dir, src/engine.rs:340-346).
    (d / "model.gguf").write_bytes(b"")
    assert llrs.find_eos_tokens(d / "model.gguf") == reference_eos(tok, gen)


def test_eos_from_added_tokens_take_precedence(llrs, tmp_path):
    """Qwen2 files hold <|endoftext|> / <|im_end|> as added tokens (ids after
    the BPE vocabulary); token_to_id looks at the added tokens first."""
    tok = bpe_tokenizer({"a": 0, "b": 1, "c": 2}, ["<|endoftext|>", "<|im_start|>", "<|im_end|>"])
    d = write_dir(tmp_path, tok, {"eos_token_id": 4})
    want = reference_eos(tok, {"eos_token_id": 4})
    assert want == sorted({4, tok.token_to_id("<|endoftext|>"), tok.token_to_id("<|im_end|>")})
    assert llrs.find_eos_tokens(d) == want


def test_eos_unigram_vocabulary_and_absent_tokens(llrs, tmp_path):
    tok = unigram_tokenizer(["<unk>", "x", "<|im_end|>", "y"])
    d = write_dir(tmp_path, tok, None)
    assert llrs.find_eos_tokens(d) == reference_eos(tok, None) == [2]
    tok2 = unigram_tokenizer(["<unk>", "x", "y"])
    d2 = tmp_path / "none"
    d2.mkdir()
    write_dir(d2, tok2, None)
    assert llrs.find_eos_tokens(d2) == reference_eos(tok2, None) == []


def test_eos_errors(llrs, tmp_path):
    with pytest.raises(llrs.LlrsError, match="tokenizer.json"):
        llrs.find_eos_tokens(tmp_path)  # InferenceEngine::from_path needs tokenizer.json
    tok = bpe_tokenizer(VOCAB, [])
    d = write_dir(tmp_path, tok, None, raw_gen="{not json")
    with pytest.raises(llrs.LlrsError, match="generation_config.json"):
        llrs.find_eos_tokens(d)
    (d / "generation_config.json").unlink()
    (d / "tokenizer.json").write_text("[1, 2")
    with pytest.raises(llrs.LlrsError, match="tokenizer.json"):
        llrs.find_eos_tokens(d)
