"""GPU parity of the HIP primitives and single kernels against the
reference's committed vectors and the CPU oracle (bit-exact)."""

import numpy as np
import pytest

import fixture_io as fx

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from heatvit_amd import ops as o
    return o


@pytest.mark.parametrize("suite", ["fixed", "requant"])
def test_requant_vectors(ops, suite):
    recs = fx.requant_records(suite)
    for src in range(-32, 32):
        for dst in range(-32, 32):
            sel = [(v, e) for v, s, d, e in recs if s == src and d == dst]
            if sel:
                got = ops.requant([v for v, _ in sel], src, dst, 8)
                assert got.tolist() == [e for _, e in sel], (src, dst)


def test_gelu_plan_vectors(ops):
    recs = fx.nonlinear_records()
    xs = np.array([r[0] for r in recs])
    assert ops.gelu(xs).tolist() == [r[1] for r in recs]
    assert ops.plan_sigmoid(xs).tolist() == [r[2] for r in recs]


def test_gelu_exhaustive_24bit(ops, oracle):
    # Every Q8.16 input the call sites can produce (requant to 24 bits
    # precedes every gelu), against the oracle's exact integer division.
    xs = np.arange(-(1 << 23), 1 << 23, dtype=np.int64)
    got = ops.gelu(xs)
    want = oracle.gelu_array(xs)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(int(xs[i]), int(got[i]), int(want[i])) for i in bad[:5]]


def test_softmax_vectors(ops):
    rows = fx.softmax_rows()
    att, sel = ops.softmax_rows([r[0] for r in rows])
    for (x, want_att, want_sel), a, s in zip(rows, att, sel):
        assert np.array_equal(a, want_att), x[:4]
        assert np.array_equal(s, want_sel), x[:4]


def test_layernorm_vectors(ops):
    for x, g, b, exps, warn, expected in fx.layernorm_rows():
        out, neg = ops.layernorm_rows(x[None], g, b, *exps)
        assert np.array_equal(out[0], expected), exps
        assert bool(neg[0]) == warn


def test_layernorm_random_rows_vs_oracle(ops, oracle):
    rng = np.random.default_rng(11)
    for _ in range(24):
        exps = (int(rng.integers(-32, 1)), int(rng.integers(-32, 32)),
                int(rng.integers(-32, 32)), int(rng.integers(-32, 32)))
        x = rng.integers(-128, 128, (300, 192))
        g = rng.integers(-128, 128, 192)
        b = rng.integers(-128, 128, 192)
        out, _ = ops.layernorm_rows(x, g, b, *exps)
        assert np.array_equal(out, oracle.layernorm_rows(x, g, b, *exps)), exps


@pytest.mark.parametrize("rows", [40001, 9003, 257])
def test_layernorm_row_groups_vs_oracle(ops, oracle, rows):
    """The int32 LayerNorm shares each row's constants among R rows of an
    8-lane group, R = 4 or 1 by the live row count (>= 32768 or
    fewer); ragged tails, degenerate rows (constant, one outlier, extremes)
    and negative-variance flags included."""
    rng = np.random.default_rng(rows)
    x = rng.integers(-128, 128, (rows, 192))
    x[::7] = rng.integers(-128, 128, (len(x[::7]), 1))          # constant rows
    x[3::11, 5] = 127                                          # one outlier
    x[5::13] = rng.choice([-128, 127], (len(x[5::13]), 192))    # extremes
    g = rng.integers(-128, 128, 192)
    b = rng.integers(-128, 128, 192)
    for exps in ((-7, -6, -7, -7), (-12, -5, -20, -9), (-16, -4, -20, -3), (-4, -8, -24, -2)):
        out, neg = ops.layernorm_rows(x, g, b, *exps)
        assert np.array_equal(out, oracle.layernorm_rows(x, g, b, *exps)), (rows, exps)
        want_neg = [oracle.layernorm(x[r], g, b, *exps)[1] for r in range(0, rows, 997)]
        assert [bool(v) for v in neg[::997]] == [bool(v) for v in want_neg], (rows, exps)


def test_gemm_scenarios(ops):
    """Every scenario of the reference's GEMM vectors, the unsigned-A one
    (gemm_numpy a_unsigned) included."""
    names = []
    for sc in fx.gemm_scenarios():
        s0, s1, dst = sc["scales"]
        for h in range(sc["heads"]):
            w = sc["b"][h].T if sc["transpose"] else sc["b"][h]
            bias = None if sc["bias"] is None else sc["bias"][h * sc["n"]:(h + 1) * sc["n"]]
            got = ops.gemm_writeback(sc["a"][h], w, bias, s0 + s1, dst, sc["bits"],
                                     a_unsigned=sc["unsigned"])
            assert np.array_equal(got, sc["expected"][h]), (sc["name"], h)
        names.append(sc["name"])
    assert "unsigned" in names and len(names) == 8


@pytest.mark.parametrize("m,n,k", [(197, 197, 64), (64, 100, 64), (1000, 192, 224),
                                   (33, 40, 2048)])
def test_gemm_unsigned_a_vs_oracle(ops, oracle, m, n, k):
    """Unsigned A (gemm.py:93-114) against the oracle: every epilogue, A
    bytes across 0..255 with all-255 rows and columns, weights at -128."""
    rng = np.random.default_rng(m + 3 * n + k)
    a = rng.integers(0, 256, (m, k))
    a[::5] = 255
    a[:, ::7] = 0
    w = rng.integers(-128, 128, (k, n))
    w[:, ::3] = -128
    bias = rng.integers(-(1 << 20), 1 << 20, n)
    acc = oracle.gemm(a, w, bias, a_unsigned=True)
    for src, dst in ((-14, -7), (-8, -15), (-30, 5)):
        assert np.array_equal(ops.gemm_writeback(a, w, bias, src, dst, 8, a_unsigned=True),
                              oracle.gemm_writeback(acc, src, dst, 8)), (src, dst)
    assert np.array_equal(ops.gemm_writeback(a, w, bias, -14, -14, 32, a_unsigned=True),
                          oracle.gemm_writeback(acc, -14, -14, 32))
    q = oracle.requant_array(acc, -14, -16, 24)
    want = oracle.requant_array(oracle.gelu_array(q).astype(np.int64), -16, -7, 8)
    assert np.array_equal(ops.gemm_writeback(a, w, bias, -14, -7, 8, epilogue="gelu",
                                             a_unsigned=True), want)
    # wide biases take the exact 64-bit epilogue
    wide = bias.copy()
    wide[::2] = rng.choice([(1 << 31) - 1, -(1 << 31)], len(wide[::2]))
    acc = oracle.gemm(a, w, wide, a_unsigned=True)
    assert np.array_equal(ops.gemm_writeback(a, w, wide, -20, -4, 8, a_unsigned=True),
                          oracle.gemm_writeback(acc, -20, -4, 8))


def test_gemm_unsigned_a_extremes(ops, oracle):
    """K = 65536 with A = 255 and W = -128 or 127 everywhere: the largest
    accumulators unsigned A allows (-2^31 + 2^23 and 2^31 - 2^24 - 2^23 ...),
    through the int32 output."""
    k = 65536
    a = np.full((3, k), 255)
    w = np.full((k, 64), -128)
    w[:, 1::2] = 127
    acc = oracle.gemm(a, w, None, a_unsigned=True)
    assert acc.min() == -255 * 128 * k and acc.max() == 255 * 127 * k
    assert np.array_equal(ops.gemm_writeback(a, w, None, 0, 0, 32, a_unsigned=True),
                          oracle.gemm_writeback(acc, 0, 0, 32))


@pytest.mark.parametrize("m,n,k", [(1, 1000, 192), (197, 576, 192), (1000, 768, 192),
                                   (333, 192, 768), (64, 100, 64), (4099, 192, 192)])
def test_gemm_epilogues_vs_oracle(ops, oracle, m, n, k):
    rng = np.random.default_rng(m * 7 + n)
    a = rng.integers(-128, 128, (m, k))
    w = rng.integers(-128, 128, (k, n))
    bias = rng.integers(-(1 << 20), 1 << 20, n)
    acc = oracle.gemm(a, w, bias)
    for src, dst in ((-14, -7), (-20, -4), (-8, -12), (-30, 5)):
        assert np.array_equal(ops.gemm_writeback(a, w, bias, src, dst, 8),
                              oracle.gemm_writeback(acc, src, dst, 8)), (src, dst)
    assert np.array_equal(ops.gemm_writeback(a, w, bias, -14, -14, 32),
                          oracle.gemm_writeback(acc, -14, -14, 32))
    # GELU post-op (transformer.py:349-358), every element
    for src, dst in ((-14, -7), (-22, -5)):
        q = oracle.requant_array(acc, src, -16, 24)
        want = oracle.requant_array(oracle.gelu_array(q).astype(np.int64), -16, dst, 8)
        got = ops.gemm_writeback(a, w, bias, src, dst, 8, epilogue="gelu")
        assert np.array_equal(got, want), (src, dst)
    # residual align-add (transformer.py:96-101), every element: the aligned
    # sum stays below 2^58 for these exponents, so int64 holds it exactly
    res = rng.integers(-128, 128, (m, n))
    for mid, rexp, out in ((-7, -6, -7), (-9, -4, -5), (-30, 20, -3)):
        t = oracle.gemm_writeback(acc, -14, mid, 8).astype(np.int64)
        c = min(rexp, mid)
        aligned = (res.astype(np.int64) << (rexp - c)) + (t << (mid - c))
        want = oracle.requant_array(aligned, c, out, 8)
        got = ops.gemm_writeback(a, w, bias, -14, out, 8, epilogue="residual", mid_exp=mid,
                                 residual=res, res_exp=rexp)
        assert np.array_equal(got, want.reshape(got.shape)), (mid, rexp, out)


@pytest.mark.parametrize("k", [192, 64])
def test_gemm_int32_writeback_shifts(ops, oracle, k):
    """The int32 epilogue (gemm_writeback with output_bits 32,
    gemm.py:123-131) with right, zero and left shifts, on gathered rows
    (the classifier head's shape at K = 192) and whole rows; the wide biases
    put some column tiles on the exact path and the others on the int32
    shift."""
    rng = np.random.default_rng(k)
    a = rng.integers(-128, 128, (300, k))
    w = rng.integers(-128, 128, (k, 1000))
    rows = np.sort(rng.choice(300, 64, replace=False)).astype(np.int32)
    narrow = rng.integers(-(1 << 20), 1 << 20, 1000)
    wide = narrow.copy()
    wide[::97] = rng.choice([-1, 1], wide[::97].size) * ((1 << 31) - 1 - rng.integers(0, 1 << 20, wide[::97].size))
    for bias in (narrow, wide):
        acc_g = oracle.gemm(a[rows], w, bias)
        acc = oracle.gemm(a, w, bias)
        for src, dst in ((-14, -14), (-14, -9), (-20, -4), (-9, -14), (-8, -13), (-30, -2),
                         (-4, -30)):
            got = ops.gemm_writeback(a, w, bias, src, dst, 32, a_rows=rows)
            assert np.array_equal(got, oracle.gemm_writeback(acc_g, src, dst, 32)), (src, dst)
            got = ops.gemm_writeback(a, w, bias, src, dst, 32)
            assert np.array_equal(got, oracle.gemm_writeback(acc, src, dst, 32)), (src, dst)


def test_gemm_gather_rows(ops, oracle):
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (500, 192))
    w = rng.integers(-128, 128, (192, 1000))
    rows = np.array([0, 197, 7, 499, 3], np.int32)
    got = ops.gemm_writeback(a, w, None, -14, -14, 32, a_rows=rows)
    want = oracle.gemm_writeback(oracle.gemm(a[rows], w, None), -14, -14, 32)
    assert np.array_equal(got, want)


def test_finalize_vectors():
    from heatvit_amd.selector import finalize_tokens
    for name, meta, tokens, scores, expected in fx.selector_cases():
        pkg = bool(meta["input_package_present"])
        r = finalize_tokens(tokens[0], tokens[1:-1] if pkg else tokens[1:],
                            tokens[-1] if pkg else None, scores)
        assert np.array_equal(r.tokens, expected), name
        assert len(r.tokens) == meta["next_token_count"]
        assert int(r.package_present) == meta["next_package_present"]
        assert r.warnings == meta["warning_flags"]


def test_finalize_random_vs_oracle(oracle):
    from heatvit_amd.selector import finalize_tokens
    rng = np.random.default_rng(9)
    for trial in range(30):
        n = int(rng.integers(2, 198))
        toks = rng.integers(-128, 128, (n, 192))
        pkg = bool(trial % 2) and n >= 3
        c = n - 1
        scores = rng.integers(0, 65537, c)
        if trial % 5 == 0:
            scores[:] = 0  # zero denominator fallback
        if trial % 7 == 0:
            scores[rng.integers(0, c, c // 2)] = 32768  # threshold ties
        normal = toks[1:-1] if pkg else toks[1:]
        inc = toks[-1] if pkg else None
        r = finalize_tokens(toks[0], normal, inc, scores)
        want, kept, st = oracle.finalize_tokens(toks[0], normal, inc, scores)
        assert np.array_equal(r.tokens, want), trial
        assert np.array_equal(r.kept_index, kept)
        assert (r.kept_normal_count, r.pruned_normal_count, r.warnings, int(r.package_present)) \
            == (st.kept_normal_count, st.pruned_normal_count, st.warnings, st.package_present)


def test_gemm_wide_bias_columns_take_exact_fallback(ops, oracle):
    # Columns whose bias is too large for the int32 epilogue path must still
    # match (they run the 64-bit requant), next to int32-path columns.
    rng = np.random.default_rng(21)
    m, k, n = 130, 192, 576
    a = rng.integers(-128, 128, (m, k))
    w = rng.integers(-128, 128, (k, n))
    bias = rng.integers(-(1 << 20), 1 << 20, n)
    bias[::3] = rng.integers(-(1 << 31), 1 << 31, len(bias[::3]))
    bias[1] = (1 << 31) - 1
    bias[2] = -(1 << 31)
    acc = oracle.gemm(a, w, bias)
    for src, dst in ((-14, -7), (-40, -8), (-3, 10)):
        assert np.array_equal(ops.gemm_writeback(a, w, bias, src, dst, 8),
                              oracle.gemm_writeback(acc, src, dst, 8)), (src, dst)
    q = oracle.requant_array(acc, -22, -16, 24)
    want = oracle.requant_array(oracle.gelu_array(q).astype(np.int64), -16, -9, 8)
    assert np.array_equal(ops.gemm_writeback(a, w, bias, -22, -9, 8, epilogue="gelu"), want)
