"""Pins the CPU oracle's primitives and unit stages against the reference's
committed golden vectors (sim/vectors, copied under tests/fixtures) and the
known-answer tests of verification/tests/test_{fixed,gemm,nonlinear,
selector}.py, plus mathematical checks (brute force, closed forms)."""

import math
import random
from fractions import Fraction

import numpy as np
import pytest

import fixture_io as fx


# ------------------------------------------------------------ fixture health

def test_fixture_hashes_match_reference_manifests():
    for suite in ("fixed", "requant", "divsqrt", "nonlinear", "softmax", "layernorm"):
        man = fx.manifest(suite)
        for f in man["files"]:
            assert fx.sha256(fx.FIXTURES / suite / f["name"]) == f["sha256"], f["name"]
    gem = fx.manifest("gemm")
    for f in gem["files"]:
        assert fx.sha256(fx.FIXTURES / "gemm" / f["name"]) == f["sha256"], f["name"]
    sel = fx.manifest("selector")
    for f in sel["files"]:
        path = fx.FIXTURES / "selector" / f["path"].replace("\\", "/")
        assert fx.sha256(path) == f["sha256"], f["path"]


# ------------------------------------------------------------ fixed.py

@pytest.mark.parametrize("suite,count", [("fixed", 137), ("requant", 1037)])
def test_requant_vectors(oracle, suite, count):
    recs = fx.requant_records(suite)
    assert len(recs) == count
    bad = [(v, s, d, e, oracle.requant(v, s, d, 8)) for v, s, d, e in recs
           if oracle.requant(v, s, d, 8) != e]
    assert not bad, bad[:5]


def test_udiv_isqrt_vectors(oracle):
    recs = fx.udiv_records()
    assert len(recs) == 1031
    for n, d, q, r in recs:
        assert oracle.udiv(n, d) == (q, r)
    recs = fx.isqrt_records()
    assert len(recs) == 1036
    for x, root, rem in recs:
        assert oracle.isqrt(x) == (root, rem)


def test_fixed_known_answers(oracle):
    # verification/tests/test_fixed.py:13-38
    assert [oracle.round_shift_away(v, 1) for v in (1, -1, 3, -3)] == [1, -1, 2, -2]
    assert oracle.sat_signed(128, 8) == 127 and oracle.sat_signed(-129, 8) == -128
    assert oracle.requant(255, -8, -7, 8) == 127
    assert oracle.requant(-255, -8, -7, 8) == -128
    assert oracle.udiv(10, 3) == (3, 1) and oracle.udiv(0, 5) == (0, 0)
    with pytest.raises(ValueError):
        oracle.udiv(10, 0)
    assert oracle.isqrt(0) == (0, 0) and oracle.isqrt(15) == (3, 6)
    assert oracle.isqrt(16) == (4, 0)


def test_round_div_brute_force(oracle):
    # round to nearest, ties away from zero, sign from the numerator
    # (fixed.py:57-70), checked with exact rationals.
    for num in range(-60, 61):
        for den in range(1, 13):
            q = Fraction(abs(num), den)
            mag = math.floor(q + Fraction(1, 2))
            assert oracle.round_div(num, den) == (-mag if num < 0 else mag), (num, den)
    for num, den in ((6, -3), (-7, -2), (7, -2)):
        mag = math.floor(Fraction(abs(num), abs(den)) + Fraction(1, 2))
        assert oracle.round_div(num, den) == (-mag if num < 0 else mag)
    with pytest.raises(ValueError):
        oracle.round_div(1, 0)


def test_rsa_and_requant_against_rationals(oracle):
    rng = random.Random(5)
    for _ in range(3000):
        v = rng.randint(-(1 << 40), 1 << 40)
        s = rng.randint(1, 45)
        q = Fraction(abs(v), 1 << s)
        mag = math.floor(q + Fraction(1, 2))
        assert oracle.round_shift_away(v, s) == (-mag if v < 0 else mag)
    for _ in range(3000):
        v = rng.randint(-(1 << 40), 1 << 40)
        src, dst = rng.randint(-32, 31), rng.randint(-32, 31)
        exact = Fraction(v) * Fraction(2) ** (src - dst)
        mag = math.floor(abs(exact) + Fraction(1, 2))
        r = -mag if exact < 0 else mag
        assert oracle.requant(v, src, dst, 8) == max(-128, min(127, r))
        assert oracle.requant(v, src, dst, 32) == max(-(1 << 31), min((1 << 31) - 1, r))


def test_isqrt_against_math(oracle):
    rng = random.Random(7)
    vals = [rng.randrange(1 << 64) for _ in range(2000)] + [(1 << 64) - 1, (1 << 32) ** 2 - 1]
    for v in vals:
        r = math.isqrt(v)
        assert oracle.isqrt(v) == (r, v - r * r)


# ------------------------------------------------------------ nonlinear.py

def test_gelu_plan_vectors(oracle):
    recs = fx.nonlinear_records()
    assert len(recs) == 1109
    bad = [(x, g, oracle.gelu(x)) for x, g, _ in recs if oracle.gelu(x) != g]
    assert not bad, bad[:5]
    bad = [(x, p, oracle.plan_sigmoid(x)) for x, _, p in recs if oracle.plan_sigmoid(x) != p]
    assert not bad, bad[:5]


def test_gelu_plan_known_answers(oracle):
    # verification/tests/test_nonlinear.py:29-37, 62-85
    kat = {0: 0, 1: 1, -1: 0, 32768: 22817, -32768: -9802, 163965: 161556,
           -163965: -2404, 8388607: 8323583, -8388608: 0}
    for x, y in kat.items():
        assert oracle.gelu(x) == y, x
    plan = {0: 32768, 65536: 49152, 155648: 60160, 327680: 65536, -65536: 16384,
            -155648: 5376, -327680: 0, 65535: 49151, 65537: 49152, 155647: 60415,
            155649: 60160, 327679: 65535, 327681: 65536}
    for x, y in plan.items():
        assert oracle.plan_sigmoid(x) == y, x
    for x in (0, 1, 65536, 155648, 327680, -(1 << 23), (1 << 23) - 1):
        assert oracle.plan_sigmoid(-x) == 65536 - oracle.plan_sigmoid(x)


def test_gelu_properties_full_domain_sample(oracle):
    # x * sigmoid-like gain: sign preserved (or zero) and |gelu(x)| <= |x| + 1.
    for x in list(range(-70000, 70000, 97)) + [(1 << 23) - 1, -(1 << 23)]:
        y = oracle.gelu(x)
        assert (y == 0) or (y > 0) == (x > 0)
        assert abs(y) <= abs(x) + 1


def test_softmax_vectors(oracle):
    rows = fx.softmax_rows()
    assert len(rows) == 273
    assert sum(len(r[0]) for r in rows) == 25552
    for x, att, sel in rows:
        assert np.array_equal(oracle.softmax_attention(x), att), x[:4]
        assert np.array_equal(oracle.softmax_selector(x), sel), x[:4]


def test_softmax_known_answers(oracle):
    # verification/tests/test_nonlinear.py:93-131
    for row in ([0], [12345], [-(1 << 23)], [(1 << 23) - 1]):
        assert list(oracle.softmax_attention(row)) == [255]
        assert list(oracle.softmax_selector(row)) == [65536]
    assert list(oracle.softmax_selector([0, 0])) == [32768, 32768]
    for row in ([0] * 3, [0] * 197, [1, 2, 3, 4], [-(1 << 23), (1 << 23) - 1, 0]):
        assert abs(int(oracle.softmax_selector(row).sum()) - 65536) <= 197
        assert int(oracle.softmax_attention(row).astype(int).sum()) <= 256
    row = list(range(-20, 21))
    s = oracle.softmax_selector(row)
    assert list(s) == sorted(s)
    with pytest.raises(ValueError):
        oracle.softmax_selector([])


def test_layernorm_vectors(oracle):
    rows = fx.layernorm_rows()
    assert len(rows) == 71
    for x, g, b, exps, warn, expected in rows:
        out, neg = oracle.layernorm(x, g, b, *exps)
        assert np.array_equal(out, expected), exps
        assert neg == warn


def test_layernorm_known_answers(oracle):
    g64, b0 = np.full(192, 64), np.zeros(192)
    out, warn = oracle.layernorm(np.zeros(192), g64, b0, -7, -6, -7, -7)
    assert not out.any() and not warn
    out, _ = oracle.layernorm(np.full(192, 42), g64, np.full(192, 5), -7, -6, -7, -7)
    assert (out == 5).all()
    out, warn = oracle.layernorm(np.array([127] * 95 + [90] * 97), g64, b0, -23, -6, -7, -7)
    assert warn and not out.any()
    out, _ = oracle.layernorm(np.arange(-128, 64), g64, b0, -7, -6, -7, -7)
    assert list(out) == sorted(out)
    for bad_exp in (1, -33):
        with pytest.raises(ValueError):
            oracle.layernorm(np.zeros(192), g64, b0, bad_exp, -6, -7, -7)


# ------------------------------------------------------------ gemm.py

def test_gemm_scenarios(oracle):
    names = []
    for sc in fx.gemm_scenarios():
        s0, s1, dst = sc["scales"]
        for h in range(sc["heads"]):
            bias = None if sc["bias"] is None else sc["bias"][h * sc["n"]:(h + 1) * sc["n"]]
            acc = oracle.gemm(sc["a"][h], sc["b"][h], bias, sc["transpose"], sc["unsigned"])
            got = oracle.gemm_writeback(acc, s0 + s1, dst, sc["bits"])
            assert np.array_equal(got, sc["expected"][h]), (sc["name"], h)
        assert set(sc["pad"]) <= {0xA5}
        names.append(sc["name"])
    assert names == ["mini", "ordinary", "full", "tail", "large", "head", "transpose",
                     "unsigned"]


def test_mac_bank(oracle):
    cases = fx.mac_bank_cases()
    assert len(cases) == 40
    for a, b, unsigned, rm, cm, k, expected in cases:
        A = np.repeat(np.array(a)[:, None], k, axis=1)
        B = np.repeat(np.array(b)[None, :], k, axis=0)
        acc = oracle.gemm(A, B, None, False, unsigned)
        mask = np.outer([(rm >> r) & 1 for r in range(8)], [(cm >> c) & 1 for c in range(8)])
        assert np.array_equal(acc * mask, expected)


def test_gemm_known_answers(oracle):
    # verification/tests/test_gemm.py:10-20, 36-48, 64-79
    a = [[1, 2, 3], [-1, 0, 1]]
    b = [[1, 2], [3, 4], [5, 6]]
    assert oracle.gemm(a, b, [7, -7]).tolist() == [[29, 21], [11, -3]]
    assert oracle.gemm(a, np.array(b).T, [7, -7], True).tolist() == [[29, 21], [11, -3]]
    assert oracle.gemm([[128]], [[-128]], None, False, True).tolist() == [[-16384]]
    assert oracle.gemm([[255]], [[-1]], None, False, True).tolist() == [[-255]]
    assert oracle.gemm_writeback([[1 << 40, -(1 << 40), 5]], -14, -14, 32).tolist() == \
        [[(1 << 31) - 1, -(1 << 31), 5]]
    with pytest.raises(ValueError):
        oracle.gemm_writeback([[1]], -14, -7, 16)


def test_gemm_matches_float_free_numpy(oracle):
    rng = np.random.default_rng(3)
    for m, n, k in ((1, 1, 1), (7, 9, 5), (197, 192, 192), (33, 1000, 192), (5, 64, 768)):
        a = rng.integers(-128, 128, (m, k))
        b = rng.integers(-128, 128, (k, n))
        bias = rng.integers(-(1 << 31), 1 << 31, n)
        want = a.astype(np.int64) @ b.astype(np.int64) + bias
        assert np.array_equal(oracle.gemm(a, b, bias), want)
        au = rng.integers(0, 256, (m, k))
        assert np.array_equal(oracle.gemm(au, b, None, False, True),
                              au.astype(np.int64) @ b.astype(np.int64))


# ------------------------------------------------------------ selector.py

def test_selector_finalize_vectors(oracle):
    seen = []
    for name, meta, tokens, scores, expected in fx.selector_cases():
        pkg = bool(meta["input_package_present"])
        normals = tokens[1:-1] if pkg else tokens[1:]
        incoming = tokens[-1] if pkg else None
        out, kept, st = oracle.finalize_tokens(tokens[0], normals, incoming, scores)
        assert np.array_equal(out, expected), name
        assert st.token_count == meta["next_token_count"]
        assert st.package_present == meta["next_package_present"]
        assert st.warnings == meta["warning_flags"]
        seen.append(name)
    assert sorted(seen) == sorted(["keep_all", "prune_all", "mixed", "threshold_eq",
                                   "incoming_package", "zero_den"])


def test_fuse_vectors(oracle):
    scores, weights, expected, warns, warn_bits = fx.fuse_triples()
    for i in range(len(expected)):
        fused, warn = oracle.fuse_head_scores(scores[i].reshape(3, 1), weights[i].reshape(1, 3))
        assert fused[0] == expected[i]
        assert warn == warns[i] == warn_bits[i]


def _sentinel(n):
    return np.array([[((t * 53 + 7) % 251) - 125] * 192 for t in range(n)], np.int8)


def test_finalize_known_answers(oracle):
    # verification/tests/test_selector.py:36-178
    out, _, st = oracle.finalize_tokens([1, 2], [[3, 4], [5, 6]], None, [32768, 32767])
    assert out.tolist() == [[1, 2], [3, 4], [5, 6]] and st.package_present
    out, _, st = oracle.finalize_tokens([1], [[2]], [9], [65536, 65536])
    assert out.tolist() == [[1], [2], [9]]
    token_a = [0, 100] + [100] * 190
    token_b = [-19, 0] + [-19] * 190
    out, _, _ = oracle.finalize_tokens([0] * 192, [token_a, token_b], None, [3, 1])
    assert out[-1][0] == -5 and out[-1][1] == 75
    with pytest.raises(ValueError):
        oracle.finalize_tokens([1], np.zeros((0, 1)), [9], [1])
    # package = score-weighted mean of the pruned candidates (closed form)
    toks = _sentinel(12)
    scores = [50000 if t % 2 == 0 else 1000 for t in range(11)]
    out, kept, st = oracle.finalize_tokens(toks[0], toks[1:], None, scores)
    assert kept.tolist() == [0, 2, 4, 6, 8, 10]
    pruned = [(toks[1 + t].astype(int), scores[t]) for t in range(11) if t % 2]
    den = sum(s for _, s in pruned)
    for d in range(192):
        num = sum(s * int(tok[d]) for tok, s in pruned)
        mag = math.floor(Fraction(abs(num), den) + Fraction(1, 2))
        assert out[-1][d] == max(-128, min(127, -mag if num < 0 else mag))
    fused, warn = oracle.fuse_head_scores([[0], [32768], [65536]], [[65536, 65536, 0]])
    assert fused[0] == 16384 and warn == 0
    fused, warn = oracle.fuse_head_scores([[1000], [2000], [3000]], [[0, 0, 0]])
    assert fused[0] == 2000 and warn == 1
