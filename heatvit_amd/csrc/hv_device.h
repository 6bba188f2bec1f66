// hv_device.h -- device-side integer primitives of HeatViT-T's golden model.
//
// Each helper restates one reference function bit for bit on the ranges
// its call sites reach (noted per helper); the kernels use them in their
// epilogues.  Exponent-dependent shifts are uniform per launch, so the
// branches below do not diverge within a wavefront.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hv {

typedef long long i64;
typedef unsigned long long u64;
typedef __int128 i128;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- fixed.py

// round_shift_away (fixed.py:15-25) for shift >= 0 and |v| < 2^62.
__device__ __forceinline__ i64 rsa_pos(i64 v, int s) {
  if (s == 0) return v;
  if (s >= 63) return 0;
  u64 mag = v < 0 ? (u64)(-v) : (u64)v;
  mag = (mag + (1ull << (s - 1))) >> s;
  return v < 0 ? -(i64)mag : (i64)mag;
}

// sat_signed (fixed.py:28-34), bits <= 63.
__device__ __forceinline__ i64 sat_bits(i64 v, int bits) {
  const i64 hi = (1ll << (bits - 1)) - 1, lo = -hi - 1;
  return v > hi ? hi : (v < lo ? lo : v);
}

// sat_signed(v << sl, bits) without forming an out-of-range value.
__device__ __forceinline__ i64 sat_shl(i64 v, int sl, int bits) {
  const i64 hi = (1ll << (bits - 1)) - 1, lo = -hi - 1;
  if (v == 0) return 0;
  if (sl >= bits) return v > 0 ? hi : lo;
  if (v > (hi >> sl)) return hi;
  if (v < (lo >> sl)) return lo;
  return (i64)((u64)v << sl);
}

// requant (fixed.py:37-45) with shift = dst_exp - src_exp; |v| < 2^62.
__device__ __forceinline__ i64 requant_shift(i64 v, int shift, int bits) {
  return shift >= 0 ? sat_bits(rsa_pos(v, shift), bits) : sat_shl(v, -shift, bits);
}

// 128-bit variants for LayerNorm and exponent-aligned adds; |v| < 2^125.
__device__ __forceinline__ i128 rsa128(i128 v, int s) {
  if (s <= 0) return v * ((i128)1 << (-s));
  if (s > 126) return 0;
  i128 mag = v < 0 ? -v : v;
  mag = (mag + ((i128)1 << (s - 1))) >> s;
  return v < 0 ? -mag : mag;
}

__device__ __forceinline__ i64 sat128(i128 v, int bits) {
  const i128 hi = ((i128)1 << (bits - 1)) - 1, lo = -hi - 1;
  return (i64)(v > hi ? hi : (v < lo ? lo : v));
}

__device__ __forceinline__ i64 requant128(i128 v, int shift, int bits) {
  if (shift >= 0) return sat128(rsa128(v, shift), bits);
  const i128 hi = ((i128)1 << (bits - 1)) - 1, lo = -hi - 1;
  const int sl = -shift;
  if (v == 0) return 0;
  if (sl >= bits) return v > 0 ? (i64)hi : (i64)lo;
  if (v > (hi >> sl)) return (i64)hi;
  if (v < (lo >> sl)) return (i64)lo;
  return (i64)(v * ((i128)1 << sl));
}

// round_div (fixed.py:57-70) for den > 0: nearest, ties away from zero.
__host__ __device__ __forceinline__ i64 round_div_pos(i64 num, i64 den) {
  u64 mag = num < 0 ? (u64)(-num) : (u64)num;
  u64 q = mag / (u64)den, r = mag - q * (u64)den;
  if (2 * r >= (u64)den) q += 1;
  return num < 0 ? -(i64)q : (i64)q;
}

// round_div_pos for |num| < 2^52 and 0 < den < 2^52 from one double
// quotient: num and den are exact in double, and when num / den is not an
// integer its distance to the next integer (at least 1 / den) exceeds the
// quotient's rounding error (at most num / den * 2^-53 < 1 / den), so the
// truncated double quotient is floor(num / den); the remainder test rounds.
__host__ __device__ __forceinline__ i64 round_div_pos_d(i64 num, i64 den) {
  const u64 mag = num < 0 ? (u64)(-num) : (u64)num;
  u64 q = (u64)((double)mag / (double)den);
  const u64 r = mag - q * (u64)den;
  if (2 * r >= (u64)den) q += 1;
  return num < 0 ? -(i64)q : (i64)q;
}

// _align_add_requant (transformer.py:96-101): both operands int8.  The
// aligned sum needs more than 64 bits only when the exponents differ by
// more than 54; that case takes the 128-bit route.
__device__ __forceinline__ int align_add_i8(int a, int a_exp, int b, int b_exp, int out_exp) {
  const int c = a_exp < b_exp ? a_exp : b_exp;
  const int da = a_exp - c, db = b_exp - c;
  if (da <= 54 && db <= 54) {
    i64 s = (i64)((u64)(i64)a << da) + (i64)((u64)(i64)b << db);
    return (int)requant_shift(s, out_exp - c, 8);
  }
  i128 s = (i128)a * ((i128)1 << da) + (i128)b * ((i128)1 << db);
  return (int)requant128(s, out_exp - c, 8);
}

// requant (fixed.py:37-45) in int32 arithmetic for |v| < 2^30; lo/hi are
// the saturation bounds of the target width.  rsa for negative v uses
// (v + 2^(s-1) - 1) >> s, the floor form of -((-v + 2^(s-1)) >> s).
__device__ __forceinline__ int requant_i32(int v, int shift, int lo, int hi) {
  int r;
  if (shift > 0) {
    r = shift >= 31 ? 0 : (v + (1 << (shift - 1)) - (v < 0 ? 1 : 0)) >> shift;
  } else if (shift == 0) {
    r = v;
  } else {
    const int sl = -shift;
    if (sl >= 31) return v > 0 ? hi : (v < 0 ? lo : 0);
    const i64 w = (i64)v * (1ll << sl);
    return w > hi ? hi : (w < lo ? lo : (int)w);
  }
  return r > hi ? hi : (r < lo ? lo : r);
}

// _align_add_requant with host-precomputed shifts da = a_exp - c,
// db = b_exp - c, os = out_exp - c (c = min(a_exp, b_exp)); int32 when
// da, db <= 21 (then |sum| <= 2^29).
__device__ __forceinline__ int align_add_pre(int a, int b, int da, int db, int os, bool narrow) {
  if (narrow) return requant_i32(a * (1 << da) + b * (1 << db), os, -128, 127);
  if (da <= 54 && db <= 54)
    return (int)requant_shift((i64)((u64)(i64)a << da) + (i64)((u64)(i64)b << db), os, 8);
  return (int)requant128((i128)a * ((i128)1 << da) + (i128)b * ((i128)1 << db), os, 8);
}

// ---------------------------------------------------------------- nonlinear.py

// gelu (nonlinear.py:60-80), ShiftGELU on Q8.16.  Domain: the 24-bit signed
// range, which every call site guarantees (requant(..., -16, 24) first).
// Everything stays in 32-bit lanes:
//  * |ip2| < 2^25, so q = |ip2| >> 16 < 2^9; ib < 2^17 makes ib >> min(q, 31)
//    zero for every q > 16, and ib << min(q, 8) >= 2^24 exceeds the cap for
//    every q > 7, so both branch conditions become clamps;
//  * e <= 2^23 - 1 gives den < 2^24 and sig < 2^16 - 500 (sig -> 2^16 only
//    as e -> inf); the quotient estimate from the float reciprocal is within
//    one of sig, and its remainder, below 2^25 in magnitude, is exact in
//    wrapping 32-bit arithmetic, so one correction step finishes the division;
//  * |x| * sig < 2^39: with |x| = ah * 2^16 + al (ah < 2^7) the rounded shift
//    is ah * sig + ((al * sig + 2^15) >> 16), two 24-bit products, and its
//    magnitude stays below |x| < 2^23, so the 24-bit saturation never acts.
__host__ __device__ __forceinline__ unsigned mul_u24(unsigned a, unsigned b) {
  return (a & 0xFFFFFFu) * (b & 0xFFFFFFu);
}

// Device operations behind gelu_q16_r: the single-precision reciprocal of
// the quotient estimate (any value within a few ulp of 1/d works, the
// correction step is exact), and an empty register constraint on ip that
// emits nothing but keeps the compiler from evaluating (3 * ip) >> 1 as a
// 64-bit average of ip's summands.
struct RcpHw {
  __device__ static float rcp(float d) { return __builtin_amdgcn_rcpf(d); }
  __device__ static int opaque(int v) {
    asm("" : "+v"(v));
    return v;
  }
};

template <typename R>
__host__ __device__ __forceinline__ int gelu_q16_r(int x) {
  const int ip = R::opaque(x + (x >> 1) + (x >> 3) + (x >> 4));
  // ip + (ip >> 1) == (3 * ip) >> 1 for every integer ip (floor of 1.5 ip);
  // |3 ip| < 2^26.
  const int ip2 = ((3 * ip) >> 1) - (ip >> 4);
  const unsigned a = (unsigned)(ip2 < 0 ? -ip2 : ip2);
  const unsigned q = a >> 16;
  const unsigned frac = (mul_u24(a & 0xFFFFu, 11u) + 15u) >> 4;
  // Both branches of nonlinear.gelu, selected without a divergent branch.
  const unsigned e_neg = (65536u - frac) >> (q < 31u ? q : 31u);
  const unsigned sh = (65536u + frac) << (q < 8u ? q : 8u);
  const unsigned e_pos = sh < (1u << 23) - 1 ? sh : (1u << 23) - 1;
  const unsigned e = ip2 < 0 ? e_neg : e_pos;
  const unsigned den = 65536u + e;
  // e / den < 1, so the estimate stays below 65536.5 plus a few ulp and
  // sig <= 65536; with den < 2^24 the product below is a 24-bit multiply
  // whose low 32 bits are all the wrapping remainder needs.
  const float est = (float)e * 65536.0f * R::rcp((float)den) + 0.5f;
  unsigned sig = (unsigned)est;
  const int rem = (int)((e << 16) + (den >> 1) - mul_u24(sig, den));
  sig = sig + (rem >= (int)den ? 1u : 0u) + (unsigned)(rem >> 31);
  const unsigned ax = (unsigned)(x < 0 ? -x : x);
  const unsigned y = mul_u24(ax >> 16, sig) + ((mul_u24(ax & 0xFFFFu, sig) + 32768u) >> 16);
  return x < 0 ? -(int)y : (int)y;
}

__device__ __forceinline__ int gelu_q16(int x) { return gelu_q16_r<RcpHw>(x); }

// The low bytes of four words as one word, a in the low byte (three byte
// permutes).
__device__ __forceinline__ unsigned pack_lo4(unsigned a, unsigned b, unsigned c, unsigned d) {
  return __builtin_amdgcn_perm(__builtin_amdgcn_perm(d, c, 0x0c0c0400u),
                               __builtin_amdgcn_perm(b, a, 0x0c0c0400u), 0x05040100u);
}

// requant of |v| < 2^30 to [lo, hi] by a launch-uniform shift s in
// [-30, 30].  s >= 1: round_shift_away is (v + 2^(s-1) - (v < 0)) >> s.
// s <= 0: the left shift saturates, so v is first clamped to
// [(lo >> -s) - 1, (hi >> -s) + 1], which keeps v << -s inside int32 and
// outside [lo, hi] exactly when the unclamped value is.
struct Rq {
  int s, rnd, vlo, vhi, lo, hi;
};

__device__ __forceinline__ Rq rq_setup(int s, int lo, int hi) {
  Rq r;
  r.s = s;
  r.lo = lo;
  r.hi = hi;
  r.rnd = s > 0 ? 1 << (s - 1) : 0;
  r.vlo = s > 0 ? 0 : (lo >> -s) - 1;
  r.vhi = s > 0 ? 0 : (hi >> -s) + 1;
  return r;
}

__device__ __forceinline__ int rq(int v, const Rq &r) {
  const int t = r.s > 0 ? (v + r.rnd + (v >> 31)) >> r.s : min(max(v, r.vlo), r.vhi) << -r.s;
  return min(max(t, r.lo), r.hi);
}

// The same with the direction fixed at compile time (LEFT: s <= 0).
template <bool LEFT>
__device__ __forceinline__ int rq_dir(int v, const Rq &r) {
  const int t = LEFT ? min(max(v, r.vlo), r.vhi) << -r.s : (v + r.rnd + (v >> 31)) >> r.s;
  return min(max(t, r.lo), r.hi);
}

// The shift of rq_dir_nowrap without the final clamp (for a consumer that
// clamps to a narrower range itself).
template <bool LEFT>
__device__ __forceinline__ int shift_nowrap(int v, const Rq &r) {
  return LEFT ? (int)((unsigned)v << -r.s) : (v + r.rnd + (v >> 31)) >> r.s;
}

// rq_dir for a v whose left shift cannot leave int32 (|v| <= (2^31 - 1) >>
// -s, which the caller guarantees): the shift needs no pre-clamp.
template <bool LEFT>
__device__ __forceinline__ int rq_dir_nowrap(int v, const Rq &r) {
  const int t = LEFT ? (int)((unsigned)v << -r.s) : (v + r.rnd + (v >> 31)) >> r.s;
  return min(max(t, r.lo), r.hi);
}

// requant(gelu(requant(v, src, -16, 24)), -16, dst, 8): the GEMM+GELU
// post-op of ffn (transformer.py:349-358) and selector._gemm_gelu
// (selector.py:89-99).  shift_in = -16 - src_exp, shift_out = dst_exp + 16.
__device__ __forceinline__ int gelu_post(i64 v, int shift_in, int shift_out) {
  const int q = (int)requant_shift(v, shift_in, 24);
  return (int)requant_shift(gelu_q16(q), shift_out, 8);
}

// requant(gelu(q), -16, so - 16, 8) from a GELU step table (layout in
// gen_gelu_lut.py) staged in LDS at `lut`: [qlo, qhi] the table's clamp
// (qlo a multiple of 2^kGeluCoarseShift), cb = -4 * (qlo >> kGeluCoarseShift)
// the byte offset that makes (c >> kGeluCoarseShift) << 2 address the coarse
// words.  The coarse word of c = clamp(q) holds s2 in its low five bits and,
// above them, a byte offset such that c's entry sits at offset + 4 * (c >>
// s2); the word itself is the shift amount (the hardware reads its low five
// bits).  The entry's bytes 0 and 1 are the value before and after its one
// change and bits 16..31 the low 16 bits of the c where it changes (an
// entry's values of c share one aligned block of 2^16, so the low halves
// compare as the values): the result is the value in the low byte of the
// returned word (the upper bits are not cleared).
constexpr int kGeluCoarseShift = 8;

__device__ __forceinline__ unsigned gelu_table_u8(int q, const unsigned *lut, int cb, int qlo,
                                                  int qhi) {
  int c;
  asm("v_med3_i32 %0, %1, %2, %3" : "=v"(c) : "v"(q), "v"(qlo), "v"(qhi));
  const char *t = reinterpret_cast<const char *>(lut);
  int b = c >> kGeluCoarseShift;
  asm("" : "+v"(b));  // keeps b * 4 + cb one shift-add (not a shift, mask and add)
  const int w1 = *reinterpret_cast<const int *>(t + cb + b * 4);
  const unsigned w = *reinterpret_cast<const unsigned *>(t + (w1 >> 5) + (c >> (w1 & 31)) * 4);
  return ((unsigned)c & 0xFFFFu) >= (w >> 16) ? w >> 8 : w;
}

// gelu_table_u8 of N values in stages (the N coarse reads, then the N
// fine reads, then the selects) with scheduling barriers between them, so
// each stage's LDS reads are in flight together (the compiler had issued
// them eight at a time).
template <int N>
__device__ __forceinline__ void gelu_table_u8_n(const int (&q)[N], unsigned (&o)[N],
                                                const unsigned *lut, int cb, int qlo, int qhi) {
  const char *t = reinterpret_cast<const char *>(lut);
  int c[N], w1[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(c[j]) : "v"(q[j]), "v"(qlo), "v"(qhi));
    int b = c[j] >> kGeluCoarseShift;
    asm("" : "+v"(b));
    w1[j] = *reinterpret_cast<const int *>(t + cb + b * 4);
  }
  __builtin_amdgcn_sched_barrier(0);
  unsigned w[N];
#pragma unroll
  for (int j = 0; j < N; ++j)
    w[j] = *reinterpret_cast<const unsigned *>(t + (w1[j] >> 5) + (c[j] >> (w1[j] & 31)) * 4);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < N; ++j) o[j] = ((unsigned)c[j] & 0xFFFFu) >= (w[j] >> 16) ? w[j] >> 8 : w[j];
}
// gelu_table_u8_n with the results packed four to a word (value j in byte
// j % 4 of word j / 4): instead of shifting each entry past its change and
// packing the low bytes, one byte permute per pair of entries picks byte 0
// or 1 of each (the selector from the two comparisons), and a third joins
// the pairs.
template <int N>
__device__ __forceinline__ void gelu_table_pack_n(const int (&q)[N], unsigned (&o)[N / 4],
                                                  const unsigned *lut, int cb, int qlo, int qhi) {
  static_assert(N % 4 == 0, "whole words");
  const char *t = reinterpret_cast<const char *>(lut);
  int c[N], w1[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(c[j]) : "v"(q[j]), "v"(qlo), "v"(qhi));
    int b = c[j] >> kGeluCoarseShift;
    asm("" : "+v"(b));
    w1[j] = *reinterpret_cast<const int *>(t + cb + b * 4);
  }
  __builtin_amdgcn_sched_barrier(0);
  unsigned w[N];
#pragma unroll
  for (int j = 0; j < N; ++j)
    w[j] = *reinterpret_cast<const unsigned *>(t + (w1[j] >> 5) + (c[j] >> (w1[j] & 31)) * 4);
  __builtin_amdgcn_sched_barrier(0);
  unsigned pair[N / 2];
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const int a = 2 * k, b = a + 1;
    const bool pb = ((unsigned)c[b] & 0xFFFFu) >= (w[b] >> 16);
    // entry a's comparison as a lane mask, added as the carry-in of one
    // add (the compiler otherwise spends a select and an or on it)
    const unsigned long long pa =
        __builtin_amdgcn_uicmp((unsigned)c[a] & 0xFFFFu, w[a] >> 16, 35 /* unsigned >= */);
    // bytes 0-3 of the pool are w[a], 4-7 w[b]; the upper two bytes zero
    const unsigned selb = pb ? 0x0c0c0500u : 0x0c0c0400u;
    unsigned sel;
    unsigned long long carry_out;
    asm("v_addc_co_u32_e64 %0, %1, %2, 0, %3" : "=v"(sel), "=s"(carry_out) : "v"(selb), "s"(pa));
    pair[k] = __builtin_amdgcn_perm(w[b], w[a], sel);
  }
#pragma unroll
  for (int k = 0; k < N / 4; ++k)
    o[k] = __builtin_amdgcn_perm(pair[2 * k + 1], pair[2 * k], 0x05040100u);
}

// The same as a sign-extended int.
__device__ __forceinline__ int gelu_table(int q, const unsigned *lut, int cb, int qlo, int qhi) {
  return (int)(int8_t)gelu_table_u8(q, lut, cb, qlo, qhi);
}

// plan_sigmoid (nonlinear.py:83-95).
__device__ __forceinline__ int plan_sigmoid(int x) {
  const int ax = x < 0 ? -x : x;
  int y;
  if (ax >= 327680) y = 65536;
  else if (ax >= 155648) y = (ax >> 5) + 55296;
  else if (ax >= 65536) y = (ax >> 3) + 40960;
  else y = (ax >> 2) + 32768;
  return x < 0 ? 65536 - y : y;
}

// _softmax_exp (nonlinear.py:98-106) for x_tilde in [-(2^31 - 1), 0].
// shifted < 2^17, so its square is one 32x32->64 multiply-add; the Q16
// polynomial term stays below 2^32; e < 2^17 makes e >> min(z, 31) equal
// to the reference's e >> z for every z.
__host__ __device__ __forceinline__ unsigned softmax_exp(int xt) {
  const unsigned nx = (unsigned)(-xt);
  const unsigned z = nx / 45426u;
  const int p = xt + (int)(z * 45426u);              // (-45426, 0]
  const unsigned s = (unsigned)(p + 88670) & 0x1FFFFu;  // (43244, 88670]
  const unsigned square = (unsigned)(((u64)s * s + 32768u) >> 16);   // <= 119971
  const unsigned e = ((23495u * square + 32768u) >> 16) + 22544u;    // < 2^17
  return e >> (z < 31u ? z : 31u);
}

// The same exponential from nx = -x_tilde >= 0 (the row maximum minus the
// element) in 24-bit multiply-adds: beyond 17 * 45426 the result is 0 (e <
// 2^17 shifted by z >= 17), so nx is clamped there, z = nx / 45426 <= 17
// needs no further clamp, s = 88670 - nx + 45426 z lies in (43244, 88670],
// its square is one 32x32->64 multiply-add and 23495 * square < 2^32.
__host__ __device__ __forceinline__ unsigned softmax_exp_nx(unsigned nx) {
  const unsigned n = nx < 17u * 45426u ? nx : 17u * 45426u;
  const unsigned z = n / 45426u;
  const unsigned s = mul_u24(z, 45426u) + (88670u - n);
  const unsigned square = (unsigned)(((u64)s * s + 32768u) >> 16);
  return (((mul_u24(23495u, square) + 32768u) >> 16) + 22544u) >> z;
}

// The same exponential from t = max(x_tilde, -17 * 45426) in seven 32/64-bit
// multiply-adds and shifts.  z16 = floor(-t / 45426) + 16 is the high word
// of -t * 94549 + 16 * 2^32 (94549 = ceil(2^32 / 45426)); the quotient this
// gives is one too large at 16 arguments just below a multiple of 45426,
// where s then is 88671 instead of 43245 and the result is the same, so the
// function equals the reference's exponential for every t (an exhaustive
// check over all 772,243 arguments pins it).  X = 23495 * square + 2^15 +
// 22544 * 2^16 < 2^33 holds the polynomial as X >> 16, and one 64-bit shift
// by z16 applies both the >> 16 and the >> z.
__host__ __device__ __forceinline__ unsigned softmax_exp_t(int t) {
  const unsigned z16 = (unsigned)((u64)((i64)t * -94549ll + (16ll << 32)) >> 32);
  const unsigned s = mul_u24(z16, 45426u) + (unsigned)(88670 - 16 * 45426) + (unsigned)t;
  const unsigned square = (unsigned)(((u64)s * s + 32768u) >> 16);
  const u64 x = (u64)square * 23495u + (32768u + (22544ull << 16));
  return (unsigned)(x >> z16);
}

// softmax_exp_t(q - mx) with the row maximum folded into the constants:
// k1 = 16 * 2^32 + 94549 * mx and c1s = (88670 - 16 * 45426 - mx) * 2^8
// (mod 2^32), so q * -94549 + k1 = (q - mx) * -94549 + 16 * 2^32 exactly
// and the remainder term takes q - mx in its constant; q is already clamped
// to at least mx - 17 * 45426.  The remainder is carried as s8 = 2^8 s
// (s <= 88671, so s8 < 2^25): square = floor((s^2 + 2^15) / 2^16) is then
// the high word of s8^2 + 2^31, one 64-bit multiply-add without a shift.
__host__ __device__ __forceinline__ unsigned softmax_exp_qm(int q, i64 k1, unsigned c1s) {
  const unsigned z16 = (unsigned)((u64)((i64)q * -94549ll + k1) >> 32);
  unsigned t8 = ((unsigned)q << 8) + c1s;
#ifdef __HIP_DEVICE_COMPILE__
  asm("" : "+v"(t8));  // one shift-add, then one 24-bit multiply-add
#endif
  const unsigned s8 = mul_u24(z16, 45426u << 8) + t8;
  const unsigned square = (unsigned)(((u64)s8 * s8 + (1ull << 31)) >> 32);
  const u64 x = (u64)square * 23495u + (32768u + (22544ull << 16));
  return (unsigned)(x >> z16);
}

// The attention's UQ0.8 probability minus 128 (the signed P - 128 operand
// of the P.V product): p = min(rsa(rsa(e * recip, 16), 8), 255), whose
// first rounding's discarded bits cannot carry past a multiple of 2^8, so p
// = min((e * recip + 2^15 + 2^23) >> 24, 255).  With r256 = recip * 2^8 the
// high word of e * r256 + (2^15 + 2^23) * 2^8 - 128 * 2^32 is p - 128
// before the clamp (e, recip < 2^17).
__host__ __device__ __forceinline__ int softmax_prob_m128_raw(unsigned e, unsigned r256) {
  const i64 v = (i64)e * (i64)r256 + (((32768ll + (1ll << 23)) << 8) - (128ll << 32));
  return (int)(v >> 32);
}
__host__ __device__ __forceinline__ int softmax_prob_m128(unsigned e, unsigned r256) {
  const int p = softmax_prob_m128_raw(e, r256);
  return p < 127 ? p : 127;
}

// softmax_exp_t(0), the largest exponential of a row: every argument is
// at most 0, and no softmax_exp_t over [-17 * 45426, 0] exceeds it.
constexpr unsigned kSoftmaxExp0 = 65554u;

// round_div(2^32, sum) for a row sum that includes exp(0) = 65554, so
// 65554 <= sum < 2^32 and the result is below 2^17 (nonlinear.py:119):
// float estimate, exact correction on the remainder.
__host__ __device__ __forceinline__ unsigned softmax_recip(u64 sum) {
  const u64 num = 1ull << 32;
  u64 q = (u64)(4294967296.0f / (float)sum);
  while (q * sum > num) --q;
  while ((q + 1) * sum <= num) ++q;
  const u64 r = num - q * sum;
  return (unsigned)(2 * r >= sum ? q + 1 : q);
}

// The same for 65554 <= sum < 2^24 (rows of at most 255 exponentials, each
// <= exp(0) = 65554) in 32-bit lanes without branches: the float quotient
// 2^32 * rcp(sum) is within 2^-7 of 2^32 / sum < 2^16, so its truncation q
// is within one of the floor; the remainder r = 2^32 - q * sum then lies in
// [-sum, 2 * sum), exact in wrapping 32-bit arithmetic (q, sum < 2^24 make
// q * sum a 24-bit multiply), and one correction each way plus the rounding
// test finish the division.
template <typename R>
__host__ __device__ __forceinline__ unsigned softmax_recip24_r(unsigned sum) {
  unsigned q = (unsigned)(4294967296.0f * R::rcp((float)sum));
  int r = (int)(0u - mul_u24(q, sum));
  const int lo = r >> 31;  // r < 0: q was one too large
  q += (unsigned)lo;
  r += (int)(sum & (unsigned)lo);
  const unsigned hi = r >= (int)sum ? 1u : 0u;  // q was one too small
  q += hi;
  r -= (int)(sum & (0u - hi));
  return q + (2u * (unsigned)r >= sum ? 1u : 0u);
}
__device__ __forceinline__ unsigned softmax_recip24(unsigned sum) {
  return softmax_recip24_r<RcpHw>(sum);
}

// ratio = rsa(e * recip, 16); with delta2 = 65536 the scaled value equals
// the ratio (nonlinear.py:120-121).  e, recip < 2^17.
__host__ __device__ __forceinline__ unsigned softmax_ratio(unsigned e, unsigned recip) {
  return (unsigned)(((u64)e * recip + 32768u) >> 16);
}

// softmax_attention narrowing (nonlinear.py:133): min(rsa(scaled, 8), 255).
__host__ __device__ __forceinline__ unsigned prob_u8(unsigned ratio) {
  const unsigned p = (ratio + 128u) >> 8;
  return p > 255u ? 255u : p;
}

// floor square root over u64 (fixed.isqrt, fixed.py:73-80): double estimate
// and exact integer correction.
__host__ __device__ __forceinline__ u64 isqrt_u64(u64 x) {
  u64 r = (u64)__builtin_sqrt((double)x);
  while (r > 0 && r * r > x) --r;
  while ((r + 1) * (r + 1) <= x) ++r;
  return r;
}

// ---------------------------------------------------------------- layernorm
// int32 element path of nonlinear.layernorm (nonlinear.py:136-186) for
// input scales in [-16, -4] (s = x_scale + 32 in [16, 28], the x^2 rounding
// shift -(2*x_scale + 32) <= 0 so sum_square = (sum x^2) << t exactly).
//
// norm = sat24(rsa(V, 48)) with V = (x*2^s - mean) * inv, inv =
// round_div(2^48, sd) >= 1.  V < 0 exactly when x <= xt = floor((mean - 1)
// / 2^s), and rsa(V, 48) = floor((V + 2^47 - n) / 2^48) with n = [V < 0].
// With Y_n = mean*inv - 2^47 + n and K_n = ceil(Y_n / 2^s), V + 2^47 - n =
// 2^s (x*inv - K_n) + R_n for some R_n in [0, 2^s), and a remainder below
// 2^s does not move the floor by 2^48, so
//   rsa(V, 48) = floor((x*inv - K_n) / 2^(48 - s)).
// K_1 = K_0 + 1 when 2^s divides Y_0 (a "tie" row), else K_1 = K_0.  With
// |x| <= 128, inv < 2^42 and |mean| <= 2^(s+7), x*inv - K_0 is an integer
// of magnitude below 2^51, so one double fma of x with inv*2^(s-48) and
// -K_0*2^(s-48) yields t = (x*inv - K_0)*2^(s-48) exactly, and floor and
// the int32 conversion (|result| < 2^31) keep it exact.  For n = 1 on a tie
// row the value is floor(t - 2^(s-48)): t is a multiple of 2^(s-48) < 1, so
// that is floor(t) - 1 when t is an integer and floor(t) otherwise.
// The 24-bit saturation never acts on a row of 192 int8 values: with
// a = sigma 2^(s-16) (sigma the row's standard deviation), |x*2^s - mean| <=
// 2^16 a sqrt(191) + 1/2 (Samuelson's bound, mean within 1/2), var within 9
// of a^2 (the roundings of mean, e2 and mean^2), so sd >= max(a, 65.47) - 1,
// inv / 2^48 <= 1/sd + 2^-49, and |norm| <= 2^16 * 13.83 * 65.47 / 64.47 +
// 1 < 2^20.  So the element form needs no clamp; the exact form keeps it
// (and the CPU test checks the bound on random and extreme rows).
// The element form without the tie step rounds instead of flooring: with
// u = 2^(s-48), t' = t + u/2 - 1/2 = ((2 N + 1) - 2^(48-s)) u/2 (N = x*inv -
// K_0, |N| < 2^51) is an exact double, never a whole or half integer, so
// round-to-nearest(t') = floor(t), and adding 1.5 * 2^52 (|t'| < 2^31) leaves
// that integer in the low word of the sum: one fma and one add per element.
struct LnRow {
  double inv;   // inv * 2^(s-48)
  double add;   // -K_0 * 2^(s-48)
  double addm;  // add + u/2 - 1/2
  int xt;
  bool tie;  // some x <= xt needs the tie correction
  bool neg_var;
};

// The LnRow fields from mean, inv and C = 2^47 - mean*inv given as
// C = c2*2^48 + low, 0 <= low < 2^48: -K_0 = floor(C / 2^s) = c2*2^(48-s) +
// (low >> s).  K_1 differs from K_0 when 2^s divides low, and then matters
// only for an x <= xt whose t is an integer, x*inv = K_0 (mod 2^(48-s)):
// with inv = 2^e io (io odd), such x exist when 2^e divides K_0 mod
// 2^(48-s) and are x = (K_0 / 2^e) io^-1 (mod 2^(48-s-e)) (all x once
// e >= 48 - s); tie marks a row where one of them lies in [-128, xt].
__host__ __device__ __forceinline__ void ln_row_fill(LnRow &r, double mean, double inv, i64 c2,
                                                     i64 low, int s) {
  const i64 f = c2 * (1ll << (48 - s)) + (low >> s);
  r.inv = ldexp(inv, s - 48);
  r.add = ldexp((double)f, s - 48);
  r.addm = ldexp((double)(2 * f + 1 - (1ll << (48 - s))), s - 49);
  const double xt = floor(ldexp(mean - 1.0, -s));
  r.xt = xt > 127.0 ? 127 : (xt < -129.0 ? -129 : (int)xt);
  r.tie = false;
  if ((low & ((1ll << s) - 1)) == 0 && r.xt >= -128) {
    const int sh = 48 - s;
    const u64 mm = (1ull << sh) - 1, k0 = (u64)(-f) & mm, iv = (u64)inv;
    const int e = __builtin_ctzll(iv);
    if (e >= sh) {
      r.tie = k0 == 0;
    } else if ((k0 & ((1ull << e) - 1)) == 0) {
      const u64 io = iv >> e, pm = (1ull << (sh - e)) - 1;
      u64 ii = io;  // io^-1 mod 2^64: each step doubles the correct low bits
#pragma unroll
      for (int k = 0; k < 5; ++k) ii *= 2 - io * ii;
      const u64 rr = ((k0 >> e) * ii) & pm;
      r.tie = -128 + (i64)((rr + 128) & pm) <= r.xt;
    }
  }
}

// round_div(2^48, d) for 1 <= d < 2^32: double estimate, exact correction.
__host__ __device__ __forceinline__ u64 recip48(u64 d) {
  const u64 num = 1ull << 48;
  u64 q = (u64)((double)num / (double)d);
  while (q * d > num) --q;
  while ((q + 1) * d <= num) ++q;
  const u64 r = num - q * d;
  return 2 * r >= d ? q + 1 : q;
}

// Per-row constants from the row sums sx = sum x, sxx = sum x^2, in 64- and
// 128-bit integers (the form ln_row_consts_e is checked against).
__host__ __device__ __forceinline__ LnRow ln_row_consts(int sx, int sxx, int s, int t) {
  LnRow r;
  const i64 mean = round_div_pos((i64)sx * (1ll << s), 192);
  const i64 e2 = round_div_pos((i64)sxx * (1ll << t), 192);
  const u64 m = mean < 0 ? (u64)(-mean) : (u64)mean;  // < 2^37
  const u64 mh = m >> 16, ml = m & 0xFFFFull;
  const i64 mean_sq = (i64)(mh * mh + ((((mh * ml) << 17) + ml * ml + (1ull << 31)) >> 32));
  i64 var = e2 - mean_sq;
  r.neg_var = var < 0;
  if (var < 0) var = 0;
  const u64 sd = isqrt_u64((u64)var + 4295u);
  const u64 inv = recip48(sd);  // < 2^42
  const i128 C = ((i128)1 << 47) - (i128)mean * (i128)inv;
  const i128 c2 = C >> 48;
  ln_row_fill(r, (double)mean, (double)inv, (i64)c2, (i64)(C - c2 * ((i128)1 << 48)), s);
  return r;
}

// ln_row_consts from double-precision steps that are exact by their error
// bounds, for sx = sum x and sxx = sum x^2 of 192 int8 values, s in
// [16, 28] and t = 2 s - 32.  E supplies two estimates that the code
// corrects exactly: a float square root and a double reciprocal (the
// hardware's v_sqrt_f32 / v_rcp_f64 on the device).
//   mean = round_div(sx 2^s, 192) = floor((sx 2^(s-6) + 1) / 3): n / 3 has
//     fractional part 0, 1/3 or 2/3 (no ties); the product with the double
//     nearest 1/3 is within 2^-17 of n / 3, so adding 2^-10 before the floor
//     gives it exactly;
//   e2 = floor((sxx 2^t + 96) / 192) the same way (fractions in steps of
//     1/192, error below 2^-13);
//   mean_sq = floor((mean^2 + 2^31) / 2^32) from u = |mean| 2^-16: u^2 =
//     hi + lo exactly (fma), and u^2 - floor(hi) is a multiple of 2^-32
//     below 2, so its double sum is exact;
//   sd = isqrt(var + 4295) from the float estimate (within one), corrected
//     by the exact sign of sd^2 - x and (sd + 1)^2 - x;
//   inv = round_div(2^48, sd) from the reciprocal estimate after one Newton
//     step: the floor is within one, and the exact remainder fixes it and
//     decides the rounding;
//   C = 2^47 - mean inv from 24-bit halves of mean and inv and 64-bit
//     products with carries.
template <typename E>
__host__ __device__ __forceinline__ LnRow ln_row_consts_e(int sx, int sxx, int s, int t) {
#pragma clang fp contract(off)
  LnRow r;
  const double third = 1.0 / 3.0;
  const double nm = ldexp((double)sx, s - 6) + 1.0;
  const double mean = floor(fma(nm, third, 0x1p-10));
  const double n2 = ldexp((double)sxx, t) + 96.0;
  const double e2 = floor(fma(n2, third * 0x1p-6, 0x1p-10));
  const double u = fabs(mean) * 0x1p-16;
  const double hi = u * u, lo = fma(u, u, -hi), fh = floor(hi);
  const double mean_sq = fh + (((hi - fh) + lo) >= 0.5 ? 1.0 : 0.0);
  double var = e2 - mean_sq;
  r.neg_var = var < 0.0;
  if (var < 0.0) var = 0.0;
  const double x = var + 4295.0;
  double sd = floor((double)E::sqrt_est((float)x));
  {
    const double d = fma(sd, sd, -x);  // sd^2 - x, exact
    sd = d > 0.0 ? sd - 1.0 : ((d + 2.0 * sd + 1.0) <= 0.0 ? sd + 1.0 : sd);
  }
  double rc = E::rcp_est(sd);
  rc = fma(rc, fma(-sd, rc, 1.0), rc);
  double inv = floor(0x1p48 * rc);
  double rem = fma(-inv, sd, 0x1p48);  // exact
  if (rem < 0.0) {
    inv -= 1.0;
    rem += sd;
  } else if (rem >= sd) {
    inv += 1.0;
    rem -= sd;
  }
  if (2.0 * rem >= sd) inv += 1.0;
  // C = 2^47 - mean inv with mean = m2 2^24 + m1, inv = i1 2^24 + i0
  const double m2d = floor(mean * 0x1p-24), i1d = floor(inv * 0x1p-24);
  const int m2 = (int)m2d, m1 = (int)fma(-m2d, 0x1p24, mean);
  const int i1 = (int)i1d, i0 = (int)fma(-i1d, 0x1p24, inv);
  const i64 p0 = (i64)((u64)(unsigned)m1 * (unsigned)i0);
  const i64 p1 = (i64)m2 * i0 + (i64)m1 * i1;
  const i64 p2 = (i64)m2 * i1;
  const i64 t0 = (1ll << 47) - p0;
  const i64 t1 = (t0 >> 24) - p1;
  ln_row_fill(r, mean, inv, (t1 >> 24) - p2, ((t1 & 0xFFFFFF) << 24) | (t0 & 0xFFFFFF), s);
  return r;
}

// The device's estimates for ln_row_consts_e.
struct LnEstHw {
  __device__ static float sqrt_est(float x) { return __builtin_amdgcn_sqrtf(x); }
  __device__ static double rcp_est(double x) { return __builtin_amdgcn_rcp(x); }
};

// norm_q16 of one element.  EXACT: the tie correction (and the 24-bit
// saturation, which cannot act on a 192-channel row); without EXACT the
// caller has found that no row it handles ties.
template <bool EXACT>
__host__ __device__ __forceinline__ int ln_norm(int x, const LnRow &r) {
  if (!EXACT) {  // within 24 bits (the bound above)
    const double y = fma((double)x, r.inv, r.addm) + 0x1.8p52;
    return (int)(unsigned)__builtin_bit_cast(unsigned long long, y);
  }
  const double t = fma((double)x, r.inv, r.add);
  const double f = floor(t);
  int v = (int)f;
  if (r.tie && x <= r.xt && t == f) v -= 1;
  return v < -(1 << 23) ? -(1 << 23) : (v > (1 << 23) - 1 ? (1 << 23) - 1 : v);
}

// One row of the int32 LayerNorm by a group of LPR lanes (4 or 8; sub =
// lane % LPR owns channels (192 / LPR) * sub onwards): w, gm, bt hold the
// lane's input, gamma and beta bytes packed four per word; out receives the
// packed int8 outputs.  All LPR lanes of the group call it together
// (LPR-lane shuffles).  Returns the row's negative-variance flag.
struct Ln32 {
  const int8_t *gamma, *beta;
  int8_t *out;
  int s, t, bs, os;  // x_scale + 32, 2*x_scale + 32, beta shift, output shift
};

// Lane src's row constants (the fields ln_norm<EXACT> reads).
template <bool EXACT>
__device__ __forceinline__ LnRow ln_row_shfl(const LnRow &m, int src) {
  LnRow c;
  c.inv = __shfl(m.inv, src);
  if (EXACT) {
    c.add = __shfl(m.add, src);
    c.xt = __shfl(m.xt, src);
    c.tie = __shfl((int)m.tie, src) != 0;
  } else {
    c.addm = __shfl(m.addm, src);
  }
  return c;
}

// The NW words of one lane's elements of a row with constants r: gamma,
// beta << bs and the output requant, packed four to a word.
template <bool EXACT, int NW>
__device__ __forceinline__ void ln32_elems(const int (&w)[NW], const int (&gm)[NW],
                                           const int (&bt)[NW], const Ln32 &ln, const LnRow &r,
                                           int (&out)[NW]) {
  const int rnd = 1 << (ln.os - 1);
  int ov[4 * NW];
#pragma unroll
  for (int j = 0; j < 4 * NW; ++j) {
    const int sh = 8 * (j & 3);
    const int xv = (int)(int8_t)(w[j >> 2] >> sh);
    const int g = (int)(int8_t)(gm[j >> 2] >> sh);
    const int b = (int)(int8_t)(bt[j >> 2] >> sh);
    // norm and gamma both fit 24 bits: one 24-bit multiply-add
    const int a = __mul24(ln_norm<EXACT>(xv, r), g) + b * (1 << ln.bs);
    const int o = (a + rnd + (a >> 31)) >> ln.os;
    ov[j] = min(max(o, -128), 127);
  }
#pragma unroll
  for (int q = 0; q < NW; ++q)
    out[q] = (int)pack_lo4(ov[4 * q], ov[4 * q + 1], ov[4 * q + 2], ov[4 * q + 3]);
}

template <int LPR>
__device__ __forceinline__ bool ln32_row(const int (&w)[48 / LPR], const int (&gm)[48 / LPR],
                                         const int (&bt)[48 / LPR], const Ln32 &ln,
                                         int (&out)[48 / LPR]) {
  constexpr int NW = 48 / LPR;  // words (4 channels each) per lane
  int sx = 0, sxx = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    sx = __builtin_amdgcn_sdot4(w[q], 0x01010101, sx, false);
    sxx = __builtin_amdgcn_sdot4(w[q], w[q], sxx, false);
  }
#pragma unroll
  for (int off = 1; off < LPR; off <<= 1) {
    sx += __shfl_xor(sx, off);
    sxx += __shfl_xor(sxx, off);
  }
  const LnRow r = ln_row_consts_e<LnEstHw>(sx, sxx, ln.s, ln.t);
  if (__any(r.tie))
    ln32_elems<true, NW>(w, gm, bt, ln, r, out);
  else
    ln32_elems<false, NW>(w, gm, bt, ln, r, out);
  return r.neg_var;
}

// gamma/beta bytes of lane sub (192 / LPR channels) as packed words.
template <int LPR>
__device__ __forceinline__ void ln32_params(const Ln32 &ln, int sub, int (&gm)[48 / LPR],
                                            int (&bt)[48 / LPR]) {
  const int2 *gp = reinterpret_cast<const int2 *>(ln.gamma + sub * (192 / LPR));
  const int2 *bp = reinterpret_cast<const int2 *>(ln.beta + sub * (192 / LPR));
#pragma unroll
  for (int q = 0; q < 24 / LPR; ++q) {
    const int2 a = gp[q], c = bp[q];
    gm[2 * q] = a.x; gm[2 * q + 1] = a.y;
    bt[2 * q] = c.x; bt[2 * q + 1] = c.y;
  }
}

__device__ __forceinline__ int sat_q016(i64 v) { return v < 0 ? 0 : (v > 65536 ? 65536 : (int)v); }

}  // namespace hv
