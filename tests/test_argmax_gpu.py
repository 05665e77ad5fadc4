"""The device argmax's edge cases: argmax_current_logits (src/engine.rs:233-241)
takes max_by(f32::total_cmp), so the LAST index wins a tie and a positive NaN
ranks above +inf (a negative NaN below -inf).

The LM head of a tiny synthetic model is replaced by planted rows whose
logits are known exactly: every row is zero except a few that hold one
nonzero weight in column j, so their logit is one product (no sum can round
differently between rows).  Two pairs of identical rows tie exactly, one pair
positive, one negative; one more row may hold a NaN.  The fused LM-head
argmax (Q8_0 rows, tuned GEMV) and the generic path (F32 rows, argmax
kernel) must both return the index the oracle's argmax returns on the same
logits: the larger index of the positive pair.
"""
from __future__ import annotations

import numpy as np
import pytest

from gguf_write import rewrite
from hf_checkpoint import gguf_names

pytestmark = pytest.mark.gpu

F16_ONE, F16_NAN = 0x3C00, 0x7E00


def tiny(llrs, recipe, seed):
    return llrs.SynthConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                            num_key_value_heads=2, num_hidden_layers=2, vocab_size=1000,
                            max_position_embeddings=256, recipe=recipe, seed=seed,
                            tie_word_embeddings=False)


def planted_q8_0(vocab, cols, j, rows_pos, rows_neg, nan_row=None):
    """Q8_0 rows: block j//32 of rows_pos holds code +1 at column j with d = 1,
    rows_neg code -1; every other block has d = 0.  nan_row has d = NaN."""
    nb = cols // 32
    blk = np.zeros((vocab, nb, 34), np.uint8)
    b, e = j // 32, j % 32
    for rows, code in ((rows_pos, 1), (rows_neg, -1)):
        for r in rows:
            blk[r, b, 0:2] = np.frombuffer(np.uint16(F16_ONE).tobytes(), np.uint8)
            blk[r, b, 2 + e] = np.uint8(code & 0xFF)
    if nan_row is not None:
        blk[nan_row, b, 0:2] = np.frombuffer(np.uint16(F16_NAN).tobytes(), np.uint8)
        blk[nan_row, b, 2 + e] = 1
    return blk.tobytes()


def planted_f32(vocab, cols, j, rows_pos, rows_neg, nan_row=None):
    w = np.zeros((vocab, cols), np.float32)
    w[list(rows_pos), j] = 1.0
    w[list(rows_neg), j] = -1.0
    if nan_row is not None:
        w[nan_row, j] = np.nan
    return w.tobytes()


def run(llrs, backend, oracle, tmp_path, recipe, lm_type, nan):
    cfg = tiny(llrs, recipe, seed=71)
    src, dst = tmp_path / "src.gguf", tmp_path / "planted.gguf"
    cfg.write_gguf(src)
    names = gguf_names(cfg.num_hidden_layers, tied=False)
    prompt = np.array([3, 141, 59, 265, 358, 979], np.uint32)
    V, H = cfg.vocab_size, cfg.hidden_size
    # The pairs' rows lie in different workgroups' row ranges and row quads.
    pos_rows, neg_rows = (5, V - 3), (6, V - 5)
    nan_row = 500 if nan else None
    # The planted logits are +-x_j of the final normalised hidden state (and
    # its digitised value on the GPU), nonzero for this model and prompt.
    j = 77
    data = (planted_q8_0 if lm_type == 8 else planted_f32)(V, H, j, pos_rows, neg_rows, nan_row)
    rewrite(llrs, src, dst, cfg, names, {"output.weight": (lm_type, V, H, data)})
    model = llrs.ModelLoader.load_dynamic(dst, backend)
    kv = llrs.KVCache(model, 64)
    model.prefill(prompt, 0, kv)
    lg = kv.logits()
    a, b = lg[list(pos_rows)], lg[list(neg_rows)]
    print(f"[argmax] type={lm_type} nan={nan} pair+ {a} pair- {b} "
          f"nan-row bits {lg.view(np.uint32)[nan_row] if nan else 0:#x}", flush=True)
    # The pairs tie exactly, bit for bit.
    assert lg.view(np.uint32)[pos_rows[0]] == lg.view(np.uint32)[pos_rows[1]]
    assert lg.view(np.uint32)[neg_rows[0]] == lg.view(np.uint32)[neg_rows[1]]
    assert a[0] != 0 and a[0] == -b[0]
    want = int(oracle.lib.oq_argmax(lg.ctypes.data_as(oracle_f32p()), lg.size))
    # The token the prefill's LM-head launch recorded for the next position
    # (the fused epilogue for Q8_0, the argmax kernel for F32), then
    # llrs_argmax (the argmax kernel) over the same logits.
    got_step = int(kv.tokens(len(prompt), 1)[0])
    assert got_step == want, (got_step, want)
    assert kv.argmax() == want
    winner = pos_rows[1] if a[0] > 0 else neg_rows[1]
    if not nan:
        assert want == winner
    else:
        bits = int(lg.view(np.uint32)[nan_row])
        assert np.isnan(lg[nan_row])
        # A NaN with the sign bit clear ranks above everything; set, below.
        assert want == (nan_row if bits >> 31 == 0 else winner)
    # The oracle model computes the same planted logits on the same file.
    om2 = oracle.load(dst)
    om2.new_state(64)
    om2.prefill(prompt, 0)
    ol = om2.logits()
    np.testing.assert_array_equal(ol[list(pos_rows)], ol[pos_rows[0]])
    if not nan:
        assert om2.argmax() == winner


def oracle_f32p():
    import ctypes as C
    return C.POINTER(C.c_float)


@pytest.mark.parametrize("nan", [False, True], ids=["ties", "ties+nan"])
def test_fused_lm_head_argmax_ties_last_index(llrs, backend, oracle, tmp_path, nan):
    """Q8_0 LM head: the tuned GEMV's fused argmax (key = total-order value,
    index), reduced across workgroups with atomicMax."""
    run(llrs, backend, oracle, tmp_path, llrs.LoadQuantization.Q4KM, 8, nan)


@pytest.mark.parametrize("nan", [False, True], ids=["ties", "ties+nan"])
def test_generic_lm_head_argmax_ties_last_index(llrs, backend, oracle, tmp_path, nan):
    """F32 LM head (recipe NONE): the generic GEMV, then the argmax kernel."""
    run(llrs, backend, oracle, tmp_path, llrs.LoadQuantization.NONE, 0, nan)
