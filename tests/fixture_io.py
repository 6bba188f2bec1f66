"""Decoders for the reference's committed golden vectors (tests/fixtures).

The packings follow the writers in the reference's tools/:
  generate_unit_vectors.py:58-65 (requant), :139-205 (udiv/isqrt),
  :208-258 (GELU/PLAN), :261-312 (softmax), :315-373 (layernorm);
  generate_gemm_vectors.py:82-113 (MAC bank), :162-322 (GEMM scenarios);
  generate_selector_vectors.py:48-235 (finalize / fuse cases).
Every .mem line is one little-endian word written as unprefixed hex.
"""

import hashlib
import json
from pathlib import Path

import numpy as np

FIXTURES = Path(__file__).resolve().parent / "fixtures"


def sha256(path):
    return hashlib.sha256(Path(path).read_bytes()).hexdigest()


def read_words(path, header=False):
    words = [int(line, 16) for line in Path(path).read_text().split()]
    if header:
        count = words[0]
        words = words[1:]
        return count, words
    return words


def signed(value, bits):
    value &= (1 << bits) - 1
    return value - (1 << bits) if value >> (bits - 1) else value


def field(word, lo, bits, is_signed=False):
    v = (word >> lo) & ((1 << bits) - 1)
    return signed(v, bits) if is_signed else v


def manifest(suite):
    return json.loads((FIXTURES / suite / "manifest.json").read_text())


# --------------------------------------------------------------- unit suites

def requant_records(suite):
    """(value, src_exp, dst_exp, expected int8) tuples; suite 'fixed' has no
    header word, suite 'requant' has one."""
    path = FIXTURES / suite / "requant.mem"
    if suite == "requant":
        count, words = read_words(path, header=True)
        assert count == len(words)
    else:
        words = read_words(path)
    return [(field(w, 0, 48, True), field(w, 48, 6, True), field(w, 54, 6, True),
             field(w, 60, 8, True)) for w in words]


def udiv_records():
    count, words = read_words(FIXTURES / "divsqrt" / "udiv.mem", header=True)
    assert count == len(words)
    return [(field(w, 0, 64), field(w, 64, 64), field(w, 128, 64), field(w, 192, 64))
            for w in words]


def isqrt_records():
    count, words = read_words(FIXTURES / "divsqrt" / "isqrt.mem", header=True)
    assert count == len(words)
    return [(field(w, 0, 48), field(w, 48, 32), field(w, 80, 48)) for w in words]


def nonlinear_records():
    """(x, gelu(x), plan(x)) with x and gelu 24-bit signed, plan 17-bit."""
    count, words = read_words(FIXTURES / "nonlinear" / "nonlinear.mem", header=True)
    assert count == len(words)
    return [(field(w, 0, 24, True), field(w, 24, 24, True), field(w, 48, 17))
            for w in words]


def softmax_rows():
    """List of (x[], attention u8[], selector Q0.16[]) rows."""
    count, words = read_words(FIXTURES / "softmax" / "softmax.mem", header=True)
    assert count == len(words)
    rows, i = [], 0
    while i < len(words):
        n = field(words[i], 0, 8)
        chunk = words[i:i + n]
        assert all(field(w, 0, 8) == n for w in chunk)
        rows.append((np.array([field(w, 8, 24, True) for w in chunk], np.int32),
                     np.array([field(w, 32, 8) for w in chunk], np.uint8),
                     np.array([field(w, 40, 17) for w in chunk], np.int32)))
        i += n
    return rows


def layernorm_rows():
    """List of (x, gamma, beta, (x_exp, g_exp, b_exp, out_exp), warn, expected)."""
    count, words = read_words(FIXTURES / "layernorm" / "layernorm.mem", header=True)
    rows, i = [], 0
    for _ in range(count):
        cfg = words[i]
        exps = tuple(field(cfg, 6 * j, 6, True) for j in range(4))
        warn = bool(field(cfg, 24, 1))
        ch = words[i + 1:i + 193]
        x = np.array([field(w, 0, 8, True) for w in ch], np.int8)
        g = np.array([field(w, 8, 8, True) for w in ch], np.int8)
        b = np.array([field(w, 16, 8, True) for w in ch], np.int8)
        e = np.array([field(w, 24, 8, True) for w in ch], np.int8)
        rows.append((x, g, b, exps, warn, e))
        i += 193
    assert i == len(words)
    return rows


# --------------------------------------------------------------- GEMM suites

def _bytes_of(path):
    out = bytearray()
    for w in read_words(path):
        out += int(w).to_bytes(8, "little")
    return bytes(out)


def gemm_scenarios():
    """Yields dicts with A [H][M][K] (uint8 view when unsigned), B [H][K][N] or
    [H][N][K] (transpose), bias [H*N] or None, exps and expected [H][M][N]."""
    man = manifest("gemm")
    for sc in man["scenarios"]:
        name, m, n, k = sc["name"], sc["m"], sc["n"], sc["k"]
        heads = sc["heads"] or 1
        a_raw = _bytes_of(FIXTURES / "gemm" / f"{name}_a.mem")
        w_raw = _bytes_of(FIXTURES / "gemm" / f"{name}_w.mem")
        e_raw = _bytes_of(FIXTURES / "gemm" / f"{name}_expected.mem")
        a = np.frombuffer(a_raw[:heads * m * k],
                          np.uint8 if sc["unsigned"] else np.int8).reshape(heads, m, k)
        b_bytes = heads * n * k
        b = np.frombuffer(w_raw[:b_bytes], np.int8)
        b = b.reshape(heads, n, k) if sc["transpose"] else b.reshape(heads, k, n)
        bias = None
        if sc["bias"]:
            off = b_bytes + (-b_bytes) % 8
            bias = np.frombuffer(w_raw[off:off + 4 * heads * n], "<i4").astype(np.int32)
        esize = 4 if sc["output_bits"] == 32 else 1
        dt = "<i4" if esize == 4 else np.int8
        expected = np.frombuffer(e_raw[:heads * m * n * esize], dt).reshape(heads, m, n)
        pad = e_raw[heads * m * n * esize:]
        yield dict(name=name, m=m, n=n, k=k, heads=heads, a=a, b=b, bias=bias,
                   transpose=sc["transpose"], unsigned=sc["unsigned"],
                   bits=sc["output_bits"], expected=expected, pad=pad,
                   scales=_SCENARIO_SCALES[name])


# src0/src1/dst exponents per scenario (generate_gemm_vectors.py:397-416).
_SCENARIO_SCALES = {
    "mini": (-7, -7, -7), "ordinary": (-7, -7, -7), "full": (-7, -7, -7),
    "tail": (-7, -7, -14), "large": (-7, -7, -7), "head": (-7, -7, -7),
    "transpose": (-7, -7, -7), "unsigned": (-8, -7, -15),
}


def mac_bank_cases():
    """(a[8], b[8], unsigned, row_mask, col_mask, k, expected[8][8])."""
    count, words = read_words(FIXTURES / "gemm" / "mac_bank.mem", header=True)
    assert count == len(words) and count % 35 == 0
    cases = []
    for i in range(0, count, 35):
        w0, w1, w2 = words[i:i + 3]
        unsigned = bool(field(w2, 16, 1))
        a = [field(w0, 8 * j, 8, not unsigned) for j in range(8)]
        b = [field(w1, 8 * j, 8, True) for j in range(8)]
        accs = []
        for w in words[i + 3:i + 35]:
            accs += [field(w, 0, 32, True), field(w, 32, 32, True)]
        cases.append((a, b, unsigned, field(w2, 0, 8), field(w2, 8, 8), field(w2, 17, 14),
                       np.array(accs, np.int64).reshape(8, 8)))
    return cases


# --------------------------------------------------------------- selector

def _int8_stream(path, count):
    return np.frombuffer(_bytes_of(path)[:count], np.int8)


def _q016_stream(path, count):
    return np.frombuffer(_bytes_of(path)[:4 * count], "<u4").astype(np.int32)


def selector_cases():
    man = manifest("selector")
    for name, meta in man["cases"].items():
        d = FIXTURES / "selector" / name
        n, c = meta["tokens"], meta["candidates"]
        tokens = _int8_stream(d / "tokens.mem", n * 192).reshape(n, 192)
        scores = _q016_stream(d / "scores.mem", c)
        n_out = meta["next_token_count"]
        out = _int8_stream(d / "output.mem", n_out * 192).reshape(n_out, 192)
        yield name, meta, tokens, scores, out


def fuse_triples():
    d = FIXTURES / "selector" / "zero_den"
    meta = manifest("selector")["cases"]["zero_den"]
    cnt = meta["fuse_candidates"]
    scores = _q016_stream(d / "fuse_scores.mem", 3 * cnt).reshape(cnt, 3)
    weights = _q016_stream(d / "fuse_weights.mem", 3 * cnt).reshape(cnt, 3)
    expected = _q016_stream(d / "fuse_expected.mem", cnt)
    warns = _int8_stream(d / "fuse_warn.mem", cnt)
    return scores, weights, expected, warns, meta["fuse_warn_bits"]
