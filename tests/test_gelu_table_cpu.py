"""The GELU post-op step-table generator (heatvit_amd/csrc/gen_gelu_lut.py)
against the oracle: its restated gelu equals the oracle's nonlinear.gelu
on the whole 24-bit Q8.16 domain, its post-op equals fixed.requant, and a
table's lookup equals the post-op everywhere (a corrupted table word is
caught)."""

import importlib.util
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def gen():
    spec = importlib.util.spec_from_file_location(
        "gen_gelu_lut", ROOT / "heatvit_amd" / "csrc" / "gen_gelu_lut.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def domain(gen):
    q = np.arange(-(1 << 23), 1 << 23, dtype=np.int64)
    return q, gen.gelu_q16(q)


def test_restated_gelu_matches_oracle(oracle, domain):
    q, y = domain
    assert np.array_equal(y, oracle.gelu_array(q).astype(np.int64))


def test_post_op_matches_requant(oracle, gen, domain):
    q, y = domain
    idx = np.random.default_rng(5).integers(0, len(q), 200000)
    for so in (gen.SO_MIN, 7, gen.SO_MAX):
        want = oracle.requant_array(y[idx], -16, so - 16, 8)
        assert np.array_equal(gen.post(y[idx], so), want), so


@pytest.mark.parametrize("so", [3, 6, 7, 12])
def test_table_lookup_is_exact_and_checked(gen, domain, so):
    q, y = domain
    o = gen.post(y, so)
    qlo, qhi, l1, l2 = gen.build_table(so, q, o)
    assert np.array_equal(gen.lookup(qlo, qhi, l1, l2, q), o)
    # G is constant outside [qlo, qhi]
    assert (o[q <= qlo] == o[q == qlo][0]).all() and (o[q >= qhi] == o[q == qhi][0]).all()
    assert qlo % (1 << gen.S1) == 0
    n1e = len(l1) + (len(l1) & 1)
    assert 4 * (n1e + len(l2)) <= gen.MAX_BYTES
    bad = l2.copy()
    # the entry of q = qlo sits at the first coarse word's byte offset plus
    # 4 * (qlo >> s2), into the whole table (coarse words, padded to even,
    # then entries)
    w = int(l1[0])
    w = w - (1 << 32) if w >= 1 << 31 else w
    at = (w >> 5) + 4 * (qlo >> (w & 31))
    bad[at // 4 - n1e] ^= 1   # value at qlo, off by one
    assert not np.array_equal(gen.lookup(qlo, qhi, l1, bad, q), o)
