"""The product's block encoders (QuantTensor::quantize_*, src/quant.rs:650-967;
llama.rs_amd/csrc/quant_encode.h) pinned by an independent float64
restatement (tests/quant_f64.py), host only.

Each encoded block must be the restatement's bytes, or differ only by a
decision float32 arithmetic cannot resolve: for Q8_0, Q5_0 and Q4_K, one
near-tie taken the other way (quant_f64.explain); for Q6_K, whose x^2-weighted
trial criteria often agree to 1e-6 across trials, any admissible trial per
group (quant_f64.q6_k_accepts).  Exact agreement must hold on at least 80%
of the blocks (all of them for Q8_0 and Q5_0 here), so the check is not
carried by its tolerances.  Mistakes
planted in the restatement (half-to-even rounding, Q8_0 codes from the
binary16 d, Q6_K weights |x|, Q4_K weights x^2, Q4_K trials coded against the
initial min) must each be caught.  Closed forms pin the special blocks:
all-zero, constant, exact half-way values, NaN and infinity.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest

import quant_f64 as Q

BLOCKS = {"Q8_0": 1500, "Q5_0": 1500, "Q6K": 120, "Q4K": 120}


def draw(dist: str, n: int, rng) -> np.ndarray:
    if dist == "normal":
        x = rng.standard_normal(n) * 0.02
    elif dist == "heavy":  # Student t, 2 degrees of freedom: outliers in most blocks
        x = rng.standard_t(2, n) * 0.02
    elif dist == "scaled":  # blocks of very different magnitude, 1e-6 .. 1e3
        x = rng.standard_normal(n) * np.repeat(10.0 ** rng.uniform(-6, 3, n // 32 + 1), 32)[:n]
    else:  # "sparse": mostly zeros, some exact duplicates
        x = np.where(rng.random(n) < 0.7, 0.0, rng.choice([0.25, -0.5, 1.0, 3.0], n))
        x = x + np.where(rng.random(n) < 0.1, rng.standard_normal(n), 0.0)
    return x.astype(np.float32)


def encode(llrs, name, x, nblocks):
    bs = Q.ENCODERS[name][1]
    t = llrs.QuantTensor.quantize(getattr(llrs.QuantType, name), x, nblocks, bs)
    assert t.quant_type.name == name
    return t.data


def agreement(llrs, name, x):
    """(exact, accepted, total) over the blocks of x."""
    _, bs, tsz = Q.ENCODERS[name]
    n = x.size // bs
    data = encode(llrs, name, x, n)
    exact = accepted = 0
    for b in range(n):
        xb, pb = x[b * bs:(b + 1) * bs], data[b * tsz:(b + 1) * tsz]
        if name == "Q6K":
            if Q.q6_k(xb) == pb:
                exact += 1
                accepted += 1
            elif Q.q6_k_accepts(xb, pb):
                accepted += 1
        else:
            k = Q.explain(name, xb, pb)
            exact += k is None
            accepted += k != -1
    return exact, accepted, n


@pytest.mark.parametrize("dist", ["normal", "heavy", "scaled", "sparse"])
@pytest.mark.parametrize("name", ["Q8_0", "Q5_0", "Q6K", "Q4K"])
def test_encoder_matches_f64_restatement(llrs, name, dist):
    rng = np.random.default_rng(zlib.crc32(f"{name}/{dist}".encode()))
    n = BLOCKS[name] // (2 if dist in ("scaled", "sparse") else 1)
    x = draw(dist, n * Q.ENCODERS[name][1], rng)
    exact, accepted, total = agreement(llrs, name, x)
    print(f"[quant-pin] {name} {dist}: {exact}/{total} exact, {accepted}/{total} accepted")
    assert accepted == total
    # Q6_K sub-blocks of 8-bit scale 0 keep their trial's codes, so trial
    # near-ties show in the bytes more often where magnitudes vary.
    assert exact >= 0.8 * total


@pytest.mark.parametrize("mistake,name,dist", [
    ("q8_f16_d", "Q8_0", "normal"),
    ("q6_weights_abs", "Q6K", "normal"),
    ("q4_weights_sq", "Q4K", "normal"),
    ("fixed_min", "Q4K", "normal"),
])
def test_planted_mistakes_are_caught(llrs, mistake, name, dist):
    """The same comparison with a mistake planted in the restatement refuses
    at least 10% of the blocks (the comparison itself demands all): the
    tolerances do not absorb a wrong algorithm, even one as close as coding
    Q8_0 from the binary16-rounded d."""
    rng = np.random.default_rng(7)
    n = 60 if name in ("Q6K", "Q4K") else 400
    x = draw(dist, n * Q.ENCODERS[name][1], rng)
    Q.PLANT.add(mistake)
    try:
        exact, accepted, total = agreement(llrs, name, x)
    finally:
        Q.PLANT.clear()
    print(f"[quant-pin] planted {mistake}: {accepted}/{total} accepted")
    assert accepted <= 0.9 * total


def halfway_block(name):
    """A block whose scaled values fall exactly half-way between codes."""
    if name == "Q8_0":  # d = 1 exactly: codes round(x)
        return np.array([127.0, -0.5, 0.5, 1.5, 2.5, -2.5, -126.5, 126.5] + [0.0] * 24, np.float32)
    if name == "Q5_0":  # x* = -16 -> d = 1: codes floor(x + 16.5)
        return np.array([-16.0, -0.5, 0.5, 1.5, -1.5, 14.5, -15.5] + [0.0] * 25, np.float32)
    raise KeyError(name)


def test_rounding_is_half_away_from_zero(llrs):
    """f32::round and floor(x + 16.5) at exact half-way values (closed form),
    and the planted half-to-even rounding is caught on them."""
    x8 = halfway_block("Q8_0")
    b8 = encode(llrs, "Q8_0", x8, 1)
    assert np.frombuffer(b8[:2], np.float16)[0] == 1.0
    assert list(np.frombuffer(b8[2:10], np.int8)) == [127, -1, 1, 2, 3, -3, -127, 127]
    x5 = halfway_block("Q5_0")
    b5 = encode(llrs, "Q5_0", x5, 1)
    assert np.frombuffer(b5[:2], np.float16)[0] == 1.0
    q = [(b5[6 + j] & 15) | (((int.from_bytes(b5[2:6], "little") >> j) & 1) << 4) for j in range(7)]
    assert q == [0, 16, 17, 18, 15, 31, 1]
    assert b8 == Q.q8_0(x8) and b5 == Q.q5_0(x5)
    Q.PLANT.add("half_even")
    try:
        assert Q.q8_0(x8) != b8  # (Q5_0 floors: no rounding mode to plant)
    finally:
        Q.PLANT.clear()


def test_all_zero_blocks(llrs):
    z = np.zeros(256, np.float32)
    assert encode(llrs, "Q8_0", z, 8) == bytes(34 * 8)
    # d = 0, every code floor(0 + 16.5) = 16: all high bits set, low nibbles 0
    assert encode(llrs, "Q5_0", z, 8) == (bytes(2) + b"\xff" * 4 + bytes(16)) * 8
    assert encode(llrs, "Q6K", z, 1) == bytes(210)
    assert encode(llrs, "Q4K", z, 1) == bytes(144)
    # -0.0 behaves as 0.0
    assert encode(llrs, "Q6K", -z, 1) == bytes(210)
    assert encode(llrs, "Q4K", -z, 1) == bytes(144)


@pytest.mark.parametrize("c", [0.75, -0.75, 3e-3, -40.0])
def test_constant_blocks(llrs, c):
    x = np.full(256, c, np.float32)
    b8 = encode(llrs, "Q8_0", x, 8)
    assert np.frombuffer(b8[2:34], np.int8).tolist() == [127 if c > 0 else -127] * 32
    b5 = encode(llrs, "Q5_0", x, 8)
    # d = c / -16: every code floor(-16 + 16.5) = 0
    assert np.frombuffer(b5[:2], np.float16)[0] == np.float16(c / -16)
    assert b5[2:22] == bytes(20)
    b6, b4 = encode(llrs, "Q6K", x, 1), encode(llrs, "Q4K", x, 1)
    assert Q.q6_k_accepts(x, b6) and Q.explain("Q4K", x, b4) != -1
    # Q6_K closed form: every group fits c exactly (level L times scale c / L),
    # so every group's 8-bit scale is -128 and every code the same level.
    codes, sc, _ = Q.q6_k_unpack(b6)
    assert sc.tolist() == [-128] * 16 and len(set(codes.tolist())) == 1
    # Q4_K closed form: c > 0 is coded 15 over min 0; c < 0 is coded 0 over
    # min -c (the range is [min(c, 0), max(c, 0)]).
    qs = np.frombuffer(b4[16:], np.uint8)
    assert set((qs & 15).tolist()) | set((qs >> 4).tolist()) == ({15} if c > 0 else {0})


def test_nan_and_infinity(llrs):
    """NaN is ignored by the block maximum and codes as 0 (Rust's saturating
    cast); an infinite element makes d infinite and every code 0."""
    x = np.array([0.5, np.nan, -1.0, 0.25] + [0.0] * 28, np.float32)
    b8 = encode(llrs, "Q8_0", x, 1)
    assert b8 == Q.q8_0(x)
    assert np.frombuffer(b8[2:6], np.int8).tolist() == [64, 0, -127, 32]
    b5 = encode(llrs, "Q5_0", x, 1)
    assert b5 == Q.q5_0(x)
    xi = np.array([1.0, np.inf] + [0.5] * 30, np.float32)
    b8 = encode(llrs, "Q8_0", xi, 1)
    assert b8 == Q.q8_0(xi) and np.frombuffer(b8[:2], np.uint16)[0] == 0x7C00
    assert b8[2:] == bytes(32)
    assert encode(llrs, "Q5_0", xi, 1) == Q.q5_0(xi)


def test_emitted_codes_follow_the_emitted_scales(llrs):
    """Read back from the product's bytes alone: Q4_K codes are
    round((x + dmin * m) / (d * s)) in [0, 15], Q6_K codes
    round(x / (d * s)) in [-32, 31], for every sub-block of nonzero scale;
    the largest scale and min codes are 63 (Q4_K), the largest |scale| code
    -128 (Q6_K)."""
    rng = np.random.default_rng(3)
    x = draw("normal", 256 * 40, rng)
    b = encode(llrs, "Q4K", x, 40)
    for k in range(40):
        blk, xb = b[k * 144:(k + 1) * 144], x[k * 256:(k + 1) * 256].astype(np.float64)
        d, dm = np.frombuffer(blk[:4], np.float16).astype(np.float64)
        s12 = np.frombuffer(blk[4:16], np.uint8).astype(np.int64)
        sc = [s12[g] & 63 if g < 4 else (s12[g + 4] & 15) | ((s12[g - 4] >> 6) << 4) for g in range(8)]
        mn = [s12[g + 4] & 63 if g < 4 else (s12[g + 4] >> 4) | ((s12[g] >> 6) << 4) for g in range(8)]
        qs = np.frombuffer(blk[16:], np.uint8).astype(np.int64)
        codes = np.concatenate([np.concatenate([qs[p * 32:(p + 1) * 32] & 15, qs[p * 32:(p + 1) * 32] >> 4])
                                for p in range(4)])
        assert max(sc) == 63 and max(mn) == 63
        for g in range(8):
            if d * sc[g] != 0:
                y = (xb[32 * g:32 * g + 32] + dm * mn[g]) / (d * sc[g])
                assert Q._round_ok(y, codes[32 * g:32 * g + 32], lo=0, hi=15), (k, g)
    b = encode(llrs, "Q6K", x, 40)
    for k in range(40):
        codes, sc, d16 = Q.q6_k_unpack(b[k * 210:(k + 1) * 210])
        d, xb = Q.f16v(d16), x[k * 256:(k + 1) * 256].astype(np.float64)
        assert sc.min() == -128
        for g in range(16):
            if d * sc[g] != 0:
                y = xb[16 * g:16 * g + 16] / (d * sc[g])
                assert Q._round_ok(y, codes[16 * g:16 * g + 16] - 32, lo=-32, hi=31), (k, g)
