"""Generates gelu_lut.inc: step tables of the GEMM+GELU post-op

    G_so(q) = sat8(round_shift_away(gelu(q), so))       q: 24-bit signed Q8.16

(requant(gelu(q), -16, dst, 8) with so = dst + 16; nonlinear.py:60-80 and
fixed.py:15-45 / transformer.py:349-358), one table per so in [3, 12].

G_so is a step function of q with a few hundred changes.  qlo is a
multiple of 2^S1 = 256 (rounded down from the last value below the first
change).  Table layout (32-bit words):
  L1[b], b = (c >> S1) - (qlo >> S1) with c = clamp(q, qlo, qhi): bits 0..4
      s2, bits 5..31 a signed byte offset, from the table's start, chosen
      so that the entry of c is at offset + 4 * (c >> s2) (arithmetic
      shift; the bucket starts at a multiple of 2^S1, so its entries start
      at multiples of 2^s2).  A lookup reads c >> s2 and c mod 2^s2 with the
      word itself as the shift amount and the field width (the hardware
      takes its low five bits);
  (L1 holds n1e words, its length rounded up to even; L2 follows it)
  L2, one word per 2^s2 values of c, at most one change inside it: byte 0
      G at the entry's first c, byte 1 G from the change on (byte 0 again
      when there is none), bits 16..31 the low 16 bits of the c at which
      the change happens (the entry's first c when there is none).  An
      entry's 2^s2 <= 256 values of c lie inside one aligned block of 2^16,
      so comparing low 16 bits compares the values: the lookup is byte 1
      when (c mod 2^16) >= bits 16..31, else byte 0 (one 16-bit compare and
      one byte select).
  G is constant for q <= qlo and for q >= qhi.  Each table is padded to a
  multiple of four words, so tables start on 16-byte boundaries.  s2 is the
  largest value in [0, S1] that leaves at most one change inside every entry
  of the bucket.  Every table must fit in 31,744 bytes, the LDS the fused
  FFN kernel has beside its 50,176-byte hidden block at two workgroups per
  CU.

The generator restates gelu in numpy, builds each table, emulates the
lookup for every q of the 24-bit domain and refuses to write a table that
differs from G_so anywhere.

Run:  python gen_gelu_lut.py OUT.inc
"""

import sys

import numpy as np

SO_MIN, SO_MAX = 3, 12
S1 = 8
MAX_BYTES = 31744


def gelu_q16(x):
    """nonlinear.gelu (nonlinear.py:60-80) over an int64 array."""
    x = np.asarray(x, np.int64)
    ip = x + (x >> 1) + (x >> 3) + (x >> 4)
    ip2 = ip + (ip >> 1) - (ip >> 4)
    a = np.abs(ip2)
    q = a >> 16
    frac = ((a & 0xFFFF) * 11 + 15) >> 4
    e_neg = np.where(q <= 16, (65536 - frac) >> np.minimum(q, 16), 0)
    e_pos = np.where(q <= 7, np.minimum((65536 + frac) << np.minimum(q, 7), (1 << 23) - 1),
                     (1 << 23) - 1)
    e = np.where(ip2 < 0, e_neg, e_pos)
    den = 65536 + e
    sig = ((e << 16) + (den >> 1)) // den
    return np.clip(rsa(x * sig, 16), -(1 << 23), (1 << 23) - 1)


def rsa(v, s):
    """round_shift_away (fixed.py:15-26) for s >= 1."""
    h = 1 << (s - 1)
    return np.where(v >= 0, (v + h) >> s, -((-v + h) >> s))


def post(y, so):
    return np.clip(rsa(y, so), -128, 127)


def build_table(so, q, o):
    """(qlo, qhi, L1 words, L2 words) of G_so with at most one change per
    entry, given o = G_so(q) over the whole domain q (ascending)."""
    ch = np.nonzero(np.diff(o))[0] + 1          # o[i] != o[i - 1]
    qlo, qhi = (int(q[ch[0]] - 1) // (1 << S1)) << S1, int(q[ch[-1]])
    base = qlo - int(q[0])
    span = qhi - qlo
    uo = o[base:base + span + 1]                # G at u = c - qlo = 0 .. span
    cu = ch - base                              # change positions in u
    n1 = span // (1 << S1) + 1
    n1e = n1 + (n1 & 1)
    l1 = np.zeros(n1, np.uint32)
    l2 = []
    for b in range(n1):
        lo = b << S1
        sel = cu[(cu >= lo) & (cu < lo + (1 << S1))] - lo

        def worst(s2):
            inner = sel[(sel & ((1 << s2) - 1)) != 0]
            return int(np.bincount(inner >> s2).max()) if len(inner) else 0

        s2 = S1
        while s2 > 0 and worst(s2) > 1:
            s2 -= 1
        if worst(s2) > 1:
            raise RuntimeError(f"so={so}: more than one change at one offset")
        off = 4 * n1e + 4 * (len(l2) - ((qlo + lo) >> s2))
        if not -(1 << 26) <= off < (1 << 26):
            raise RuntimeError(f"so={so}: coarse offset {off} exceeds 27 bits")
        l1[b] = ((off << 5) & 0xFFFFFFFF) | s2
        for fb in range(1 << (S1 - s2)):
            u0 = lo + (fb << s2)
            t0 = int(uo[min(u0, span)])
            t1, at = t0, 0
            for c in sel[(sel >> s2) == fb]:
                d = int(c) - (fb << s2)
                if d:                           # d == 0: t0 already holds it
                    t1, at = int(uo[lo + c]), d
            cabs = qlo + u0 + at                # the c of the change
            l2.append((t0 & 255) | ((t1 & 255) << 8) | ((cabs & 0xFFFF) << 16))
    return qlo, qhi, l1, np.array(l2, np.uint32)


def lookup(qlo, qhi, l1, l2, q):
    """The device lookup, restated over an array of q."""
    def sx(v, bits):
        v = v.astype(np.int64)
        return np.where(v >= 1 << (bits - 1), v - (1 << bits), v)

    c = np.clip(q, qlo, qhi)
    w1 = sx(l1[(c >> S1) - (qlo >> S1)], 32)
    s2 = w1 & 31
    n1e = len(l1) + (len(l1) & 1)
    # byte address in the whole table (L1, padding, L2) -> L2 word index
    f2 = ((w1 >> 5) + 4 * (c >> s2)) // 4 - n1e
    a = l2[f2].astype(np.int64)
    return sx(np.where((c & 0xFFFF) >= ((a >> 16) & 0xFFFF), (a >> 8) & 255, a & 255), 8)


def main(out):
    q = np.arange(-(1 << 23), 1 << 23, dtype=np.int64)
    y = gelu_q16(q)
    words, info = [], []
    for so in range(SO_MIN, SO_MAX + 1):
        o = post(y, so)
        qlo, qhi, l1, l2 = build_table(so, q, o)
        if not np.array_equal(lookup(qlo, qhi, l1, l2, q), o):
            raise RuntimeError(f"so={so}: table lookup differs from the post-op")
        n1e = len(l1) + (len(l1) & 1)
        body = list(l1) + [0] * (n1e - len(l1)) + list(l2)
        body += [0] * (-len(body) % 4)          # 16-byte multiples
        if 4 * len(body) > MAX_BYTES:
            raise RuntimeError(f"so={so}: table of {4 * len(body)} bytes exceeds {MAX_BYTES}")
        info.append((qlo, qhi, n1e, len(l2), len(words), len(body)))
        words += body
    lines = [
        "// Generated by gen_gelu_lut.py: step tables of",
        "// sat8(round_shift_away(gelu(q), so)) for so in "
        f"[{SO_MIN}, {SO_MAX}] (layout in the generator).",
        "namespace hv {",
        f"constexpr int kGeluLutSoMin = {SO_MIN}, kGeluLutSoMax = {SO_MAX};",
        f"static_assert(kGeluCoarseShift == {S1}, \"coarse bucket width of the tables\");",
        "// n2 one-word entries; a table is `words` words from `off`, both",
        "// multiples of 4",
        "struct GeluLutInfo { int qlo, qhi, n1e, n2, off, words; };",
        "constexpr GeluLutInfo kGeluLutInfo[] = {",
    ]
    lines += [f"  {{{', '.join(str(v) for v in t)}}}," for t in info]
    max_words = max(t[-1] for t in info)
    lines += ["};", f"constexpr int kGeluLutWords = {len(words)};",
              f"constexpr int kGeluLutMaxWords = {max_words};",
              "__device__ const unsigned kGeluLut[kGeluLutWords] __attribute__((aligned(16))) = {"]
    for i in range(0, len(words), 8):
        lines.append("  " + " ".join(f"0x{int(w):08x}u," for w in words[i:i + 8]))
    lines += ["};", "}  // namespace hv", ""]
    with open(out, "w") as fh:
        fh.write("\n".join(lines))


if __name__ == "__main__":
    main(sys.argv[1])
