// hv_norm_attn.hip -- integer LayerNorm, fused varlen attention and the
// element-wise evaluators of the golden model's nonlinear primitives.
#include "hv_device.h"
#include <type_traits>

#include "hv_internal.h"

namespace hv {

// ---------------------------------------------------------------------------
// LayerNorm (nonlinear.layernorm, nonlinear.py:136-186), D = 192.
// Sixteen lanes per row (four rows per wavefront, 12 channels per lane), so
// the per-row reductions, isqrt and reciprocal division run SIMD across rows.
// Exact 64-bit fast paths, selected per launch from the exponents:
//  * normalise (x_exp <= -1): |x_q32 - mean| < 2^39 and inv_std < 2^42, so
//    rsa(d * inv, 48) = (|d|*inv_hi + ((|d|*inv_lo + 2^47) >> 24)) >> 24
//    with inv = inv_hi*2^24 + inv_lo, every term below 2^64;
//  * gamma/beta alignment (shifts gs <= 30, bs <= 54): |aligned| < 2^62.
// Other exponents take the 128-bit route (mean^2 < 2^78 always does).
// ---------------------------------------------------------------------------
template <bool FAST_NORM, bool FAST_ALIGN>
__global__ __launch_bounds__(256) void k_layernorm(const int8_t *__restrict__ x,
                                                   const int8_t *__restrict__ gamma,
                                                   const int8_t *__restrict__ beta,
                                                   int8_t *__restrict__ y, int rows,
                                                   const int32_t *rows_dev, int x_exp,
                                                   int g_exp, int b_exp, int out_exp,
                                                   uint8_t *neg_var, LnWarn lw) {
  const int sub = threadIdx.x & 15;  // lane within the row group
  const int R = rows_dev ? min(*rows_dev, rows) : rows;
  // Grid-stride over rows: the grid is sized for the chip, not for the
  // largest possible row count.
  for (int row = blockIdx.x * 16 + (threadIdx.x >> 4); row < R; row += gridDim.x * 16) {
  const int *xr = reinterpret_cast<const int *>(x + (size_t)row * 192) + sub * 3;
  int w[3] = {xr[0], xr[1], xr[2]};
  int xv[12];
#pragma unroll
  for (int j = 0; j < 12; ++j) xv[j] = (int)(int8_t)(w[j >> 2] >> (8 * (j & 3)));
  const int sh = x_exp + 32;               // [0, 32]
  const int sq_shift = -(2 * x_exp + 32);  // round_shift_away shift of x^2
  i64 sx = 0, ss = 0;
#pragma unroll
  for (int j = 0; j < 12; ++j) {
    sx += (i64)xv[j];
    const i64 x2 = (i64)(xv[j] * xv[j]);
    ss += sq_shift >= 0 ? rsa_pos(x2, sq_shift) : x2 * (1ll << (-sq_shift));
  }
  sx *= (1ll << sh);
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
    sx += __shfl_xor(sx, off);
    ss += __shfl_xor(ss, off);
  }
  const i64 mean = round_div_pos(sx, 192);
  const i64 e2 = round_div_pos(ss, 192);
  const i128 mean_sq = rsa128((i128)mean * mean, 32);
  i128 var = (i128)e2 - mean_sq;
  const bool neg = var < 0;
  if (neg) var = 0;
  const u64 std_q16 = isqrt_u64((u64)var + 4295u);
  const i64 inv = round_div_pos(1ll << 48, (i64)std_q16);
  const u64 inv_hi = (u64)inv >> 24, inv_lo = (u64)inv & 0xFFFFFFull;
  const int common = (g_exp - 16) < b_exp ? (g_exp - 16) : b_exp;
  const int gs = g_exp - 16 - common, bs = b_exp - common, os = out_exp - common;
  const int c0 = sub * 12;
  int out[3] = {0, 0, 0};
#pragma unroll
  for (int j = 0; j < 12; ++j) {
    const i64 d = (i64)xv[j] * (1ll << sh) - mean;
    i64 norm;
    if (FAST_NORM) {
      const u64 ad = d < 0 ? (u64)(-d) : (u64)d;
      const u64 r = (ad * inv_hi + ((ad * inv_lo + (1ull << 47)) >> 24)) >> 24;
      if (d < 0) norm = r > (1ull << 23) ? -(1ll << 23) : -(i64)r;
      else norm = r > (1ull << 23) - 1 ? (1ll << 23) - 1 : (i64)r;
    } else {
      norm = sat128(rsa128((i128)d * inv, 48), 24);
    }
    const int c = c0 + j;
    int o;
    if (FAST_ALIGN) {
      const i64 al = (norm * gamma[c]) * (1ll << gs) + (i64)beta[c] * (1ll << bs);
      o = (int)requant_shift(al, os, 8);
    } else {
      const i128 al = (i128)(norm * gamma[c]) * ((i128)1 << gs) + (i128)beta[c] * ((i128)1 << bs);
      o = (int)requant128(al, os, 8);
    }
    out[j >> 2] |= (o & 0xFF) << (8 * (j & 3));
  }
  int *yr = reinterpret_cast<int *>(y + (size_t)row * 192) + sub * 3;
  yr[0] = out[0];
  yr[1] = out[1];
  yr[2] = out[2];
  if (neg_var && sub == 0) neg_var[row] = neg ? 1 : 0;
  if (neg && lw.img_warn && sub == 0) ln_warn_row(lw.offsets, lw.batch, lw.img_warn, row);
  }  // row loop
}

// One row's 24 outputs of this lane, packed four to a word.
template <bool EXACT>
__device__ __forceinline__ void ln32_elems24(const int (&w)[6], const int (&g)[24],
                                             const int (&bb)[24], const LnRow &c, int rnd, int os,
                                             int (&out)[6]) {
  int ov[24];
#pragma unroll
  for (int j = 0; j < 24; ++j) {
    const int xv = __builtin_amdgcn_sbfe(w[j >> 2], 8 * (j & 3), 8);
    const int a = __mul24(ln_norm<EXACT>(xv, c), g[j]) + bb[j];  // both within 24 bits
    const int o = (a + rnd + (a >> 31)) >> os;
    ov[j] = min(max(o, -128), 127);
  }
#pragma unroll
  for (int q = 0; q < 6; ++q)
    out[q] = (int)pack_lo4(ov[4 * q], ov[4 * q + 1], ov[4 * q + 2], ov[4 * q + 3]);
}

// int32 LayerNorm for input scales in [-16, -4] with gamma at the common
// exponent (g_exp - 16 <= b_exp), beta shift bs <= 22 and output shift os in
// [1, 29] (LnRow in hv_device.h).  Eight lanes per row, 24 channels each,
// and R rows per 8-lane group: the row sums are all-reduced over the group,
// lane j works out the constants (mean, 2^48 / std, the fma operands of
// LnRow) of row j % R and the group reads each row's constants from its
// lane, so a row's set-up runs once per R rows of the group instead of once
// per row.  Gamma and beta << bs stay in registers per lane; each element
// costs one double fma, floor and conversion for norm_q16, one 24-bit
// multiply-add for gamma/beta and the requant.  R (4 or 1) follows the live
// row count, so small batches keep enough groups in flight.  EXACT: the
// element form with the rounding-tie correction (LnRow); returns whether
// this lane met a row that needs it.
template <int R, bool EXACT>
__device__ __forceinline__ bool ln32_groups(const int8_t *__restrict__ x, const Ln32 &ln, int nrows,
                                            int grp, int ngroups, int sub, const int (&g)[24],
                                            const int (&bb)[24], uint8_t *neg_var, const LnWarn &lw) {
  const int lane = threadIdx.x & 63, base = lane & ~7;
  const int rnd = 1 << (ln.os - 1);
  bool exact_seen = false;
  for (int row0 = grp * R; row0 < nrows; row0 += ngroups * R) {
    int w[R][6];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row < nrows) {
        const int2 *xr = reinterpret_cast<const int2 *>(x + (size_t)row * 192 + sub * 24);
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          const int2 v = xr[q];
          w[r][2 * q] = v.x;
          w[r][2 * q + 1] = v.y;
        }
      } else {
#pragma unroll
        for (int q = 0; q < 6; ++q) w[r][q] = 0;
      }
    }
    int sx[R], sxx[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sx[r] = 0;
      sxx[r] = 0;
#pragma unroll
      for (int q = 0; q < 6; ++q) {
        sx[r] = __builtin_amdgcn_sdot4(w[r][q], 0x01010101, sx[r], false);
        sxx[r] = __builtin_amdgcn_sdot4(w[r][q], w[r][q], sxx[r], false);
      }
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        sx[r] += __shfl_xor(sx[r], off);
        sxx[r] += __shfl_xor(sxx[r], off);
      }
    // this lane's row of the R: sub % R
    int msx = sx[0], msxx = sxx[0];
#pragma unroll
    for (int r = 1; r < R; ++r) {
      msx = (sub % R) == r ? sx[r] : msx;
      msxx = (sub % R) == r ? sxx[r] : msxx;
    }
    const LnRow mine = ln_row_consts_e<LnEstHw>(msx, msxx, ln.s, ln.t);
    if (sub < R && row0 + sub < nrows) {
      if (neg_var) neg_var[row0 + sub] = mine.neg_var ? 1 : 0;
      if (mine.neg_var && lw.img_warn) ln_warn_row(lw.offsets, lw.batch, lw.img_warn, row0 + sub);
    }
    exact_seen |= mine.tie && row0 + sub % R < nrows;  // (rows past the end read as zeros)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int out[6];
      ln32_elems24<EXACT>(w[r], g, bb, R == 1 ? mine : ln_row_shfl<EXACT>(mine, base + r), rnd,
                          ln.os, out);
      if (row0 + r < nrows) {
        int2 *yr = reinterpret_cast<int2 *>(ln.out + (size_t)(row0 + r) * 192 + sub * 24);
#pragma unroll
        for (int q = 0; q < 3; ++q) yr[q] = int2{out[2 * q], out[2 * q + 1]};
      }
    }
  }
  return exact_seen;
}

__global__ __launch_bounds__(256) void k_layernorm32(const int8_t *__restrict__ x, Ln32 ln,
                                                     int rows, const int32_t *rows_dev,
                                                     uint8_t *neg_var, LnWarn lw) {
  const int sub = threadIdx.x & 7;
  const int grp = (int)((blockIdx.x * 256u + threadIdx.x) >> 3), ngroups = gridDim.x * 32;
  // gamma and beta << bs of this lane's 24 channels, before the row count
  // arrives
  int g[24], bb[24];
  {
    const int2 *gp = reinterpret_cast<const int2 *>(ln.gamma + sub * 24);
    const int2 *bp = reinterpret_cast<const int2 *>(ln.beta + sub * 24);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int2 a = gp[q], c = bp[q];
      const int gw[2] = {a.x, a.y}, bw[2] = {c.x, c.y};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        g[8 * q + k] = __builtin_amdgcn_sbfe(gw[k >> 2], 8 * (k & 3), 8);
        bb[8 * q + k] = __builtin_amdgcn_sbfe(bw[k >> 2], 8 * (k & 3), 8) * (1 << ln.bs);
      }
    }
  }
  const int nrows = rows_dev ? min(*rows_dev, rows) : rows;
  // measured on MI355X: four rows per group at 50K rows (11.1 against
  // 12.2 us with one), one row per group below about 30K, where the
  // launch is latency-bound and more groups in flight win
  // A wavefront that met a row with a rounding tie runs its rows again in
  // the corrected element form (rare; same outputs for the other rows).
  if (nrows >= 32768) {
    if (__any(ln32_groups<4, false>(x, ln, nrows, grp, ngroups, sub, g, bb, neg_var, lw)))
      ln32_groups<4, true>(x, ln, nrows, grp, ngroups, sub, g, bb, neg_var, lw);
  } else {
    if (__any(ln32_groups<1, false>(x, ln, nrows, grp, ngroups, sub, g, bb, neg_var, lw)))
      ln32_groups<1, true>(x, ln, nrows, grp, ngroups, sub, g, bb, neg_var, lw);
  }
}

// The int32 LayerNorm applies (and *ln is filled) when the input scale is in
// [-16, -4], gamma sits at the common exponent, beta's shift is at most 22
// and the output shift in [1, 29]; pointers must be 8-byte aligned.
bool ln32_setup(const int8_t *g, const int8_t *b, int8_t *y, int x_exp, int g_exp, int b_exp,
                int out_exp, Ln32 *ln) {
  const int common = (g_exp - 16) < b_exp ? (g_exp - 16) : b_exp;
  const int gs = g_exp - 16 - common, bs = b_exp - common, os = out_exp - common;
  if (!(x_exp >= -16 && x_exp <= -4 && gs == 0 && bs <= 22 && os >= 1 && os <= 29)) return false;
  if (((uintptr_t)g & 7) || ((uintptr_t)b & 7) || ((uintptr_t)y & 7)) return false;
  *ln = Ln32{g, b, y, x_exp + 32, 2 * x_exp + 32, bs, os};
  return true;
}

int launch_layernorm(const int8_t *x, const int8_t *g, const int8_t *b, int8_t *y, int rows,
                     const int32_t *rows_dev, int x_exp, int g_exp, int b_exp, int out_exp,
                     uint8_t *neg_var, const LnWarn &lw, hipStream_t s) {
  if (x_exp < -32 || x_exp > 0)
    return fail(HV_EVALUE, HV_ERR_DIMENSION,
                "layernorm input scale must be in [-32, 0] (got %d)", x_exp);
  if (rows <= 0) return HV_OK;
  if (((uintptr_t)x & 3) || ((uintptr_t)y & 3))
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "layernorm: rows must be 4-byte aligned");
  const int common = (g_exp - 16) < b_exp ? (g_exp - 16) : b_exp;
  Ln32 ln;
  if (((uintptr_t)x & 7) == 0 && ln32_setup(g, b, y, x_exp, g_exp, b_exp, out_exp, &ln)) {
    // eight lanes per row, 32 row groups per workgroup
    const int blocks = (rows + 31) / 32;
    hv_launch(k_layernorm32, dim3(blocks < 256 * 8 ? blocks : 256 * 8), dim3(256), 0, s, x, ln,
              rows, rows_dev, neg_var, lw);
    return check_hip(hipGetLastError(), "k_layernorm32 launch");
  }
  const bool fast_norm = x_exp <= -1;
  const bool fast_align = (g_exp - 16 - common) <= 30 && (b_exp - common) <= 54;
  const int blocks = (rows + 15) / 16;
  const dim3 grid(blocks < 256 * 8 ? blocks : 256 * 8), block(256);
  if (fast_norm && fast_align)
    hv_launch((k_layernorm<true, true>), grid, block, 0, s, x, g, b, y, rows, rows_dev,
                       x_exp, g_exp, b_exp, out_exp, neg_var, lw);
  else if (fast_norm)
    hv_launch((k_layernorm<true, false>), grid, block, 0, s, x, g, b, y, rows,
                       rows_dev, x_exp, g_exp, b_exp, out_exp, neg_var, lw);
  else if (fast_align)
    hv_launch((k_layernorm<false, true>), grid, block, 0, s, x, g, b, y, rows,
                       rows_dev, x_exp, g_exp, b_exp, out_exp, neg_var, lw);
  else
    hv_launch((k_layernorm<false, false>), grid, block, 0, s, x, g, b, y, rows,
                       rows_dev, x_exp, g_exp, b_exp, out_exp, neg_var, lw);
  return check_hip(hipGetLastError(), "k_layernorm launch");
}

// ---------------------------------------------------------------------------
// Fused attention core of mhsa (transformer.py:228-266) for one (image,
// head): score = requant(Q K^T, 2*qkv, score, 32), q16 = sat24(rsa(score,
// -(score+13))), attention softmax to UQ0.8, context = requant(P V,
// prob+qkv, ctx, 8) written in head-concat layout (layout.py:132-155).
//
// The wavefront computes S^T = K Q^T with v_mfma_i32_16x16x64_i8 (A = 16
// keys from LDS, B = 16 queries), so lane l owns query l%16 and keys
// 16*kt + 4*(l/16) + i: row max/sum need two cross-lane steps and one
// reciprocal per lane.  The UQ0.8 probabilities stay in registers: packed
// four per dword they are exactly the B operand of ctx^T = V^T P^T once V^T
// is stored in LDS with the matching key order (key 16t + 4g + i of a
// 64-key chunk at byte 16g + 4t + i).  P is unsigned and the MFMA signed,
// so the bytes enter as P - 128 and the product is corrected by 128 times
// the per-channel key sum of V; |ctx| <= 197*128*255 < 2^23.  Lane l then holds four consecutive context
// channels of query l%16 and stores them as one dword.  V^T is built with
// 4x4 byte transposes in registers (dword LDS stores).
// ---------------------------------------------------------------------------
static constexpr int kMaxKeys = 208;   // 13 key tiles of 16
static constexpr int kKStride = 80;    // LDS row strides: the 16 lanes of a
static constexpr int kVStride = 272;   // fragment read hit disjoint banks

__device__ __forceinline__ int vt_pos(int k) {
  return (k & ~63) | (((k >> 2) & 3) << 4) | (((k >> 4) & 3) << 2) | (k & 3);
}

// q16 = sat24(rsa(requant(acc, 2*qkv, score, 32), -(score+13))).  Modes
// chosen on the host (|acc| <= 64*128*128 = 2^20): 0 = rsa(acc, s) then
// sat24 (s in [1, 30]), 1 = sat24(acc << s) with s <= 10, 2 = the general
// two-step form.
__device__ __noinline__ int attn_q16_general(int acc, int score_shift, int q16_shift) {
  return (int)requant_shift(requant_shift(acc, score_shift, 32), q16_shift, 24);
}

template <int MODE>
__device__ __forceinline__ int attn_q16(int acc, const AttnArgs &g) {
  int r;
  if (MODE == 0) {
    // a right shift by s >= 1 of |acc| <= 2^20 stays inside 24 bits
    return (acc + g.q16_rnd + (acc >> 31)) >> g.q16_s;
  } else if (MODE == 1) {
    r = acc * (1 << g.q16_s);
  } else {
    return attn_q16_general(acc, g.score_shift, g.q16_shift);
  }
  return min(max(r, -(1 << 23)), (1 << 23) - 1);
}

__device__ __noinline__ int attn_score_ckpt(int acc, int score_shift) {
  return (int)requant_shift(acc, score_shift, 32);
}

__device__ __noinline__ int attn_ctx_general(int v, int ctx_shift) {
  return (int)requant_shift(v, ctx_shift, 8);
}

// Exact int8 requant of acc + bias (64-bit), out of line: the fused QKV's
// form for biases beyond the int32 bound.
__device__ __noinline__ int attn_requant8(int acc, int bias, int shift) {
  return (int)requant_shift((i64)acc + bias, shift, 8);
}

// int8 requant of one fused-QKV tile (gemm_writeback, gemm.py:117-139):
// lane l's 16 outputs, the int32 form when every lane's biases allow it.
template <bool LA>
__device__ __forceinline__ v4i qkv_epi(const AttnArgs &g, const v16i &acc, const v4i (&b4)[4],
                                       const Rq &rq, bool all_narrow) {
  bool fast = all_narrow;
  if (!all_narrow) {
    int bmax = b4[0][0], bmin = bmax;
#pragma unroll
    for (int j = 1; j < 16; ++j) {
      bmax = max(bmax, b4[j >> 2][j & 3]);
      bmin = min(bmin, b4[j >> 2][j & 3]);
    }
    fast = __all(bmax <= g.qkv_acc_lim && bmin >= -g.qkv_acc_lim);
  }
  int o[16];
  if (fast) {
#pragma unroll
    for (int j = 0; j < 16; ++j) o[j] = rq_dir_nowrap<LA>(acc[j] + b4[j >> 2][j & 3], rq);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) o[j] = attn_requant8(acc[j], b4[j >> 2][j & 3], g.qkv_shift);
  }
  v4i w;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    w[q] = (int)((unsigned)(o[4 * q] & 0xFF) | ((unsigned)(o[4 * q + 1] & 0xFF) << 8) |
                 ((unsigned)(o[4 * q + 2] & 0xFF) << 16) | ((unsigned)o[4 * q + 3] << 24));
  return w;
}

// Q, K and V of head h over the image's N rows (the fused QKV GEMM and its
// requant, transformer.py:211-227, split per head as qkv_unpack does,
// layout.py:92-131) into LDS: Q and K as rows (Qs, Ks), V transposed in
// the P V key order (Vt).  V takes the product with the operands swapped:
// each lane then holds one channel (the weight packing's channel of its
// column) over four runs of four consecutive keys, and each run is one
// dword of Vt, and adds its keys' sum to the channel's 128 sum_k V[k]
// in vsum (LDS atomics; vsum zeroed before).  Units of one row tile of 32
// and one of Q, K, V (its two column tiles of 32): Q and K over the row
// tiles that hold key tiles, V over those that hold keys.  The head's
// biases sit in LDS (bias_s, loaded by the caller).  Keys from the last V
// tile to the 64-key chunk end are stored as zero; Q and K rows past the
// key tiles are not stored.
__device__ __forceinline__ void qkv_load_w(v4i (&w)[6], const int8_t *wqkv, int ctg, int lane) {
#pragma unroll
  for (int kt = 0; kt < 6; ++kt)
    w[kt] = *reinterpret_cast<const v4i *>(wqkv + (size_t)(ctg * 6 + kt) * 1024 + lane * 16);
}

__device__ __forceinline__ void qkv_load_a(v4i (&a)[6], const int8_t *rows) {
#pragma unroll
  for (int kt = 0; kt < 6; ++kt) a[kt] = *reinterpret_cast<const v4i *>(rows + kt * 32);
}

// One unit: row tile rt of group p (0 Q, 1 K, 2 V; ISV: p == 2) from the A
// fragments a and the group's weight fragments w.  NARROW: every bias of
// the tensor within the accumulator bound, so the requant never takes the
// general (called) form and no call runs with the prefetched operands
// live; Q and K then start their accumulators at the bias.  Rows from N to
// the tile end hold the product of row N - 1 (the A rows are clamped) and
// are stored unmasked: the scores of those keys are masked to -2^30
// (P = 0), so in (P - 128) V + 128 sum_k V[k] each such key adds
// -128 V[k] + 128 V[k] = 0 whatever its V, its K row only meets masked
// scores, and Q rows from N on are never read.
template <bool LA, bool NARROW, bool ISV>
__device__ __forceinline__ void qkv_unit(const AttnArgs &g, const v4i (&w)[2][6],
                                         const v4i (&a)[6], int p, int rt, int8_t *Qs,
                                         int8_t *Ks, int8_t *Vt, int *vsum, const int *bias_s,
                                         int rows_k, int lane, const Rq &rq) {
  const int l32 = lane & 31, hh = lane >> 5;
  if constexpr (ISV) {
    // channel of this lane's column under the weight packing
    const int pj = 16 * ((l32 >> 2) & 1) + 4 * (l32 >> 3) + (l32 & 3);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      v16i acc = v16i{0};
#pragma unroll
      for (int kt = 0; kt < 6; ++kt)
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[kt], w[c][kt], acc, 0, 0, 0);
      const int bias = bias_s[128 + c * 32 + pj];
      if (NARROW || __all(bias <= g.qkv_acc_lim && bias >= -g.qkv_acc_lim)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = rq_dir_nowrap<LA>(acc[j] + bias, rq);
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = attn_requant8(acc[j], bias, g.qkv_shift);
      }
      int8_t *vrow = Vt + (c * 32 + pj) * kVStride;
      int vs = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int t0 = rt * 32 + 8 * k + 4 * hh;  // keys t0 .. t0 + 3
        const unsigned wd = pack_lo4(acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3]);
        vs = __builtin_amdgcn_sdot4((int)wd, 0x01010101, vs, false);
        *reinterpret_cast<unsigned *>(vrow + vt_pos(t0)) = wd;
      }
      atomicAdd(&vsum[c * 32 + pj], vs * 128);
      __builtin_amdgcn_sched_barrier(0);  // one column tile's registers at a time
    }
    return;
  }
  const int r = rt * 32 + l32;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    // this lane's 16 channels c*32 + 16*hh + j
    const int *bc = bias_s + p * 64 + c * 32 + 16 * hh;
    v16i acc = NARROW ? *reinterpret_cast<const v16i *>(bc) : v16i{0};
#pragma unroll
    for (int kt = 0; kt < 6; ++kt)
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[c][kt], a[kt], acc, 0, 0, 0);
    v4i o;
    if (NARROW) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = (int)pack_lo4(rq_dir_nowrap<LA>(acc[4 * q], rq), rq_dir_nowrap<LA>(acc[4 * q + 1], rq),
                             rq_dir_nowrap<LA>(acc[4 * q + 2], rq),
                             rq_dir_nowrap<LA>(acc[4 * q + 3], rq));
    } else {
      v4i b4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) b4[q] = *reinterpret_cast<const v4i *>(bc + 4 * q);
      o = qkv_epi<LA>(g, acc, b4, rq, false);
    }
    const int ch = c * 32 + 16 * hh;  // channel within the head
    if (r < rows_k) *reinterpret_cast<v4i *>(&(p == 0 ? Qs : Ks)[r * kKStride + ch]) = o;
    __builtin_amdgcn_sched_barrier(0);  // one column tile's registers at a time
  }
}

// Wavefront p < 3 runs group p (0 Q, 1 K, 2 V) over all its row tiles
// with the group's weights loaded once; the three wavefronts walk the row
// tiles in step, so the A rows of one tile are fetched from L2 about once
// and served from L1 to the other two.  The next tile's A rows load into
// the other of two register sets while the current one multiplies (the
// last tile reloads its own rows).
template <bool LA, bool NARROW, bool ISV>
__device__ __forceinline__ void qkv_rows(const AttnArgs &g, const v4i (&w)[2][6], int p,
                                         int8_t *Qs, int8_t *Ks, int8_t *Vt, int *vsum,
                                         const int *bias_s, int row0, int N, int lane) {
  const int rows_k = ((N + 15) >> 4) * 16;
  const int nrt = ISV ? (N + 31) >> 5 : (rows_k + 31) >> 5;  // row tiles of the group
  const Rq rq = rq_setup(g.qkv_shift, -128, 127);
  const int8_t *ln1 = g.ln1 + (size_t)row0 * 192 + 16 * (lane >> 5);
  auto a_rows = [&](int rt) {
    return ln1 + (size_t)min(min(rt, nrt - 1) * 32 + (lane & 31), N - 1) * 192;
  };
  v4i a0[6], a1[6];
  qkv_load_a(a0, a_rows(0));
#pragma unroll 1
  for (int rt = 0; rt < nrt; rt += 2) {
    qkv_load_a(a1, a_rows(rt + 1));
    qkv_unit<LA, NARROW, ISV>(g, w, a0, p, rt, Qs, Ks, Vt, vsum, bias_s, rows_k, lane, rq);
    if (rt + 1 >= nrt) break;
    qkv_load_a(a0, a_rows(rt + 2));
    qkv_unit<LA, NARROW, ISV>(g, w, a1, p, rt + 1, Qs, Ks, Vt, vsum, bias_s, rows_k, lane, rq);
  }
}

template <bool LA, bool NARROW>
__device__ __forceinline__ void qkv_units(const AttnArgs &g, const v4i (&w)[2][6], int8_t *Qs,
                                          int8_t *Ks, int8_t *Vt, int *vsum, const int *bias_s,
                                          int row0, int N, int wave, int lane) {
  if (wave == 2)
    qkv_rows<LA, NARROW, true>(g, w, 2, Qs, Ks, Vt, vsum, bias_s, row0, N, lane);
  else if (wave < 2)
    qkv_rows<LA, NARROW, false>(g, w, wave, Qs, Ks, Vt, vsum, bias_s, row0, N, lane);
}

template <bool LA>
__device__ __forceinline__ void qkv_head(const AttnArgs &g, const v4i (&w)[2][6], int8_t *Qs,
                                         int8_t *Ks, int8_t *Vt, int *vsum, const int *bias_s,
                                         int row0, int N, int wave, int lane) {
  if (tensor_narrow(g.bqkv_max, g.qkv_acc_lim))
    qkv_units<LA, true>(g, w, Qs, Ks, Vt, vsum, bias_s, row0, N, wave, lane);
  else
    qkv_units<LA, false>(g, w, Qs, Ks, Vt, vsum, bias_s, row0, N, wave, lane);
  // keys of the last 64-key chunk past the V tiles: zero (four keys of one
  // channel per dword)
  const int nv = (N + 31) >> 5, kz = nv * 32, runs = (((N + 63) >> 6) * 64 - kz) >> 2;
  for (int i = threadIdx.x; i < runs * 64; i += blockDim.x)
    *reinterpret_cast<unsigned *>(Vt + (i & 63) * kVStride + vt_pos(kz + 4 * (i >> 6))) = 0u;
}

// The query tiles of one wavefront for an image of NT key tiles (N in
// (16 (NT - 1), 16 NT]): straight-line code per tile count, so the score
// MFMAs issue back to back and only the last tile masks padded keys.
// FQ: the queries come from Qs in LDS (fused QKV), else from qkv.
template <int MODE, bool CKPT, int NT, bool FQ>
__device__ __forceinline__ void attn_tiles(const AttnArgs &g, const int8_t *Ks, const int8_t *Vt,
                                           const int *vsum, const int8_t *qkv, const int8_t *Qs,
                                           int b, int h, int N, int row0, int wave, int lane) {
  constexpr int NC = (NT + 3) / 4;  // PV chunks of 64 keys
  const int ql = lane & 15, grp = lane >> 4;
  const int kvalid = N - 16 * (NT - 1) - 4 * grp;  // valid keys i < kvalid in the last tile
  // Query tiles round-robin over the wavefronts, rotated by workgroup so
  // the wavefront that gets the extra tile sits on a different SIMD in
  // neighbouring workgroups.
  for (int qt = (wave + blockIdx.x) & 3; qt < NT; qt += 4) {
    const int q = qt * 16 + ql;  // this lane's query
    v4i qb = v4i{0};
    if (q < N)
      qb = FQ ? *reinterpret_cast<const v4i *>(&Qs[q * kKStride + grp * 16])
              : *reinterpret_cast<const v4i *>(qkv + (size_t)q * 576 + h * 64 + grp * 16);
    // S^T tiles: lane holds keys 16 kt + 4 grp + i of query ql.
    v4i st[NT];
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
      const v4i ka = *reinterpret_cast<const v4i *>(&Ks[(kt * 16 + ql) * kKStride + grp * 16]);
      st[kt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, qb, v4i{0}, 0, 0, 0);
    }
    // Q8.16 scores; padded keys (only in the last tile) get -2^30, below
    // every score, so their exponential is exactly zero.
    int mx = -(1 << 30);
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (CKPT && g.score && q < N && kt * 16 + 4 * grp + i < N)
          g.score[(((size_t)b * 3 + h) * 197 + q) * 197 + kt * 16 + 4 * grp + i] =
              attn_score_ckpt(st[kt][i], g.score_shift);
        int v = attn_q16<MODE>(st[kt][i], g);
        if (kt == NT - 1) v = i < kvalid ? v : -(1 << 30);
        st[kt][i] = v;
      }
      mx = max(mx, max(max(st[kt][0], st[kt][1]), max(st[kt][2], st[kt][3])));
    }
    mx = max(mx, __shfl_xor(mx, 16));
    mx = max(mx, __shfl_xor(mx, 32));
    // exp(max(q - mx, -17 * 45426)) with mx folded into the constants
    const int qlo = mx - 17 * 45426;
    i64 k1 = (16ll << 32) + 94549ll * mx;
    unsigned c1s = ((unsigned)(88670 - 16 * 45426) - (unsigned)mx) << 8;
    // opaque to the compiler, which otherwise re-expands q * -94549 + k1
    // into a 64-bit (mx - q) product
    asm volatile("" : "+v"(k1), "+v"(c1s));
    unsigned sum = 0;
#pragma unroll
    for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned e = softmax_exp_qm(max(st[kt][i], qlo), k1, c1s);
        st[kt][i] = (int)e;
        sum += e;
      }
    }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    const unsigned r256 = softmax_recip24(sum) << 8;  // sum <= 197 * 65554 < 2^24
    v4i pk[NC];
    // The bytes P - 128 (softmax_prob_m128), packed by byte permutes.  No
    // exponential exceeds exp(0) = kSoftmaxExp0, so when no lane's
    // probability at exp(0) reaches the clamp the clamp is left out.
    auto probs = [&](auto clamp_c) {
      constexpr bool CLAMP = decltype(clamp_c)::value;
#pragma unroll
      for (int kc = 0; kc < NC; ++kc) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int kt = kc * 4 + t;
          unsigned w = 0x80808080u;  // keys past the tiles: P = 0
          if (kt < NT) {
            unsigned pm[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              pm[i] = (unsigned)(CLAMP ? softmax_prob_m128((unsigned)st[kt][i], r256)
                                       : softmax_prob_m128_raw((unsigned)st[kt][i], r256));
              if (CKPT && g.prob && q < N && kt * 16 + 4 * grp + i < N)
                g.prob[(((size_t)b * 3 + h) * 197 + q) * 197 + kt * 16 + 4 * grp + i] =
                    (uint8_t)(pm[i] + 128);
            }
            w = pack_lo4(pm[0], pm[1], pm[2], pm[3]);
          }
          pk[kc][t] = (int)w;
          // keeps the scheduler from hoisting every tile's 64-bit products
          // at once (register pressure, spills)
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    if (CKPT || !__all(softmax_prob_m128_raw(kSoftmaxExp0, r256) <= 127))
      probs(std::true_type{});
    else
      probs(std::false_type{});
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      v4i acc = v4i{0};
#pragma unroll
      for (int kc = 0; kc < NC; ++kc) {
        const v4i va = *reinterpret_cast<const v4i *>(&Vt[(dt * 16 + ql) * kVStride + kc * 64 + grp * 16]);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(va, pk[kc], acc, 0, 0, 0);
      }
      if (q < N) {
        const v4i cs = *reinterpret_cast<const v4i *>(&vsum[dt * 16 + 4 * grp]);
        int o[4];
        if (g.ctx_fast) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int v = acc[i] + cs[i];
            o[i] = min(max((v + g.ctx_rnd + (v >> 31)) >> g.ctx_shift, -128), 127);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = attn_ctx_general(acc[i] + cs[i], g.ctx_shift);
        }
        *reinterpret_cast<int *>(g.ctx + (size_t)(row0 + q) * 192 + h * 64 + dt * 16 + 4 * grp) =
            (int)pack_lo4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// At most 168 VGPRs (three workgroups per CU): the 768 items of a 256-image
// batch then run in one round.  FQ: fused QKV (qkv_head), FQL its requant
// shifting left.
template <int MODE, bool CKPT, bool FQ, bool FQL>
__global__ __launch_bounds__(256, 3) void k_attention(AttnArgs g) {
  __shared__ __attribute__((aligned(16))) int8_t Ks[kMaxKeys * kKStride];
  __shared__ __attribute__((aligned(16))) int8_t Vt[64 * kVStride];
  __shared__ __attribute__((aligned(16))) int vsum[64];  // 128 * sum_k V[k][d]
  __shared__ __attribute__((aligned(16))) int8_t Qs[FQ ? kMaxKeys * kKStride : 16];
  // the head's QKV biases: group p, column tile c, column j at p*64 + c*32 + j
  __shared__ __attribute__((aligned(64))) int bias_s[FQ ? 192 : 16];

  // The grid is a multiple of 8 and workgroups go round-robin over the 8
  // XCDs, so XCD x runs logical items [x*T8, (x+1)*T8): the three heads of
  // an image share one XCD's L2 and each row of QKV is fetched once.
  const int T = 3 * g.batch, T8 = (T + 7) >> 3;
  const int L = (blockIdx.x & 7) * T8 + (blockIdx.x >> 3);
  if (L >= T) return;
  const int b = L / 3, h = L - 3 * b;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // FQ: wavefront p < 3's weight fragments of Q, K or V and the head's
  // biases load before the row offsets, whose latency they share
  v4i w[2][6];
  int bias_v = 0;
  if constexpr (FQ) {
    if (wave < 3) {
      qkv_load_w(w[0], g.wqkv, wave * 6 + h * 2, lane);
      qkv_load_w(w[1], g.wqkv, wave * 6 + h * 2 + 1, lane);
    }
    if (tid < 192) bias_v = g.bqkv[((tid >> 6) * 6 + h * 2 + ((tid >> 5) & 1)) * 32 + (tid & 31)];
  }
  const int row0 = g.offsets[b];
  const int N = g.offsets[b + 1] - row0;
  // Images with a token count outside [1, 197] or rows outside the
  // buffers are skipped (reported by the block's image check).
  if (N <= 0 || N > HV_MAX_TOKENS || row0 < 0 || row0 > g.rows_cap - N) return;
  const int n16 = (N + 15) >> 4;  // key / query tiles
  const int n64 = (N + 63) >> 6;  // PV chunks of 64 keys
  const int8_t *qkv = FQ ? nullptr : g.qkv + (size_t)row0 * 576;

  if constexpr (FQ) {
    if (tid < 64) vsum[tid] = 0;
    if (tid < 192) bias_s[tid] = bias_v;
    __syncthreads();
    qkv_head<FQL>(g, w, Qs, Ks, Vt, vsum, bias_s, row0, N, wave, lane);
  } else {
  for (int i = tid; i < n16 * 16 * 4; i += 256) {
    const int r = i >> 2, c = (i & 3) * 16;
    v4i v = v4i{0};
    if (r < N) v = *reinterpret_cast<const v4i *>(qkv + (size_t)r * 576 + 192 + h * 64 + c);
    *reinterpret_cast<v4i *>(&Ks[r * kKStride + c]) = v;
  }
  // V^T: item (key quad kq, 16-channel group dg); keys beyond N are zero.
  for (int i = tid; i < n64 * 64; i += 256) {
    const int kq = i >> 2, dg = i & 3;
    v4i rows[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 4 * kq + j;
      rows[j] = r < N ? *reinterpret_cast<const v4i *>(qkv + (size_t)r * 576 + 384 + h * 64 + dg * 16)
                      : v4i{0};
    }
    const int pos = vt_pos(4 * kq);
#pragma unroll
    for (int dq = 0; dq < 4; ++dq)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        unsigned col = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) col |= (((unsigned)rows[j][dq] >> (8 * e)) & 0xFFu) << (8 * j);
        *reinterpret_cast<unsigned *>(&Vt[(dg * 16 + dq * 4 + e) * kVStride + pos]) = col;
      }
  }
  }
  __syncthreads();
  // The probabilities enter P V as the signed bytes P - 128: P V =
  // (P - 128) V + 128 sum_k V[k], one MFMA per tile instead of two.  The
  // per-channel sums run over the padded keys too (with FQ qkv_head has
  // added them up), so a padded key's P = 0 cancels whatever its V.
  if constexpr (!FQ) {
    if (tid < 64) {
      const int *row = reinterpret_cast<const int *>(&Vt[tid * kVStride]);
      int sv = 0;
      for (int w = 0; w < n64 * 16; ++w)
        sv = __builtin_amdgcn_sdot4(row[w], 0x01010101, sv, false);
      vsum[tid] = sv * 128;
    }
    __syncthreads();
  }

  switch (n16) {
#define HV_ATTN_CASE(n) \
    case n: attn_tiles<MODE, CKPT, n, FQ>(g, Ks, Vt, vsum, qkv, Qs, b, h, N, row0, wave, lane); \
      break;
    HV_ATTN_CASE(1) HV_ATTN_CASE(2) HV_ATTN_CASE(3) HV_ATTN_CASE(4) HV_ATTN_CASE(5)
    HV_ATTN_CASE(6) HV_ATTN_CASE(7) HV_ATTN_CASE(8) HV_ATTN_CASE(9) HV_ATTN_CASE(10)
    HV_ATTN_CASE(11) HV_ATTN_CASE(12) HV_ATTN_CASE(13)
#undef HV_ATTN_CASE
    default: break;
  }
}

int launch_attention(const AttnArgs &a_in, hipStream_t s) {
  if (a_in.batch <= 0) return HV_OK;
  AttnArgs a = a_in;
  // |Q K^T| <= 64*128*128 = 2^20.  With score_shift <= 0 and 2^20 << -score_shift
  // < 2^31 the int32 requant never saturates, and rsa(acc << s1, s2) equals
  // rsa(acc, s2 - s1) (or a left shift by s1 - s2), exact in int32.
  const int s1 = -a.score_shift, s2 = a.q16_shift;
  a.q16_mode = 2;
  a.q16_s = 0;
  a.q16_rnd = 0;
  if (a.score_shift <= 0 && s1 <= 10) {
    if (s2 >= s1) {
      a.q16_mode = 0;
      a.q16_s = s2 - s1 > 30 ? 30 : s2 - s1;
      if (a.q16_s == 0) a.q16_mode = 1;  // plain saturation
      a.q16_rnd = a.q16_s > 0 ? 1 << (a.q16_s - 1) : 0;
    } else if (s1 - s2 <= 10) {
      a.q16_mode = 1;
      a.q16_s = s1 - s2;
    }
  }
  // |ctx| < 2^23: the int32 requant is exact for shifts in [1, 30].
  a.ctx_fast = a.ctx_shift >= 1 && a.ctx_shift <= 30;
  a.ctx_rnd = a.ctx_fast ? 1 << (a.ctx_shift - 1) : 0;
  const bool ck = a.score || a.prob;
  const dim3 grid((a.batch * 3 + 7) / 8 * 8), block(256);
  if (a.ln1) {
    // fused QKV: no checkpoints, the int32-form shift range
    if (ck || !a.wqkv || !a.bqkv || a.qkv_shift < -30 || a.qkv_shift > 30 ||
        (((uintptr_t)a.ln1 | (uintptr_t)a.wqkv | (uintptr_t)a.bqkv) & 15))
      return fail(HV_EVALUE, HV_ERR_DIMENSION, "attention: fused QKV arguments");
    const bool left = a.qkv_shift <= 0;
    auto go = [&](auto k) { hv_launch(k, grid, block, 0, s, a); };
    switch (a.q16_mode * 2 + (left ? 1 : 0)) {
      case 0: go(k_attention<0, false, true, false>); break;
      case 1: go(k_attention<0, false, true, true>); break;
      case 2: go(k_attention<1, false, true, false>); break;
      case 3: go(k_attention<1, false, true, true>); break;
      case 4: go(k_attention<2, false, true, false>); break;
      default: go(k_attention<2, false, true, true>); break;
    }
    return check_hip(hipGetLastError(), "k_attention launch");
  }
  if (a.q16_mode == 0 && !ck) hv_launch((k_attention<0, false, false, false>), grid, block, 0, s, a);
  else if (a.q16_mode == 0) hv_launch((k_attention<0, true, false, false>), grid, block, 0, s, a);
  else if (a.q16_mode == 1 && !ck) hv_launch((k_attention<1, false, false, false>), grid, block, 0, s, a);
  else if (a.q16_mode == 1) hv_launch((k_attention<1, true, false, false>), grid, block, 0, s, a);
  else if (!ck) hv_launch((k_attention<2, false, false, false>), grid, block, 0, s, a);
  else hv_launch((k_attention<2, true, false, false>), grid, block, 0, s, a);
  return check_hip(hipGetLastError(), "k_attention launch");
}

// ---------------------------------------------------------------------------
// Softmax over ragged rows (nonlinear.softmax_scaled / _attention /
// _selector, nonlinear.py:109-133): one wavefront per row (<= 256 entries),
// four rows per workgroup.  Rows of at most 255 entries sum to below 2^24
// (each exponential <= exp(0) = 65554), so their reciprocal takes the
// 32-bit form; longer rows the 64-bit one.  att / sel may be NULL.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_softmax_rows(const int32_t *x, const int32_t *offsets,
                                                      int rows, uint8_t *att, int32_t *sel) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int o = offsets[row], n = offsets[row + 1] - o;
  if (n <= 0 || n > 256) return;
  int v[4];
  int mx = -(1 << 30) * 2;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    v[j] = c < n ? x[o + c] : 0;
    if (c < n) mx = v[j] > mx ? v[j] : mx;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int t = __shfl_xor(mx, off);
    mx = t > mx ? t : mx;
  }
  unsigned e[4], sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    e[j] = c < n ? softmax_exp(v[j] - mx) : 0u;
    sum += e[j];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  const unsigned recip = n <= 255 ? softmax_recip24(sum) : softmax_recip(sum);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    if (c < n) {
      const unsigned ratio = softmax_ratio(e[j], recip);
      if (att) att[o + c] = (uint8_t)prob_u8(ratio);
      if (sel) sel[o + c] = (int32_t)(ratio > 65536u ? 65536u : ratio);
    }
  }
}

int launch_softmax_rows(const int32_t *x, const int32_t *offsets, int rows, uint8_t *att,
                        int32_t *sel, hipStream_t s) {
  if (rows <= 0) return HV_OK;
  hv_launch(k_softmax_rows, dim3((rows + 3) / 4), dim3(256), 0, s, x, offsets, rows, att, sel);
  return check_hip(hipGetLastError(), "k_softmax_rows launch");
}

// ---------------------------------------------------------------------------
// Element-wise primitive evaluator.
// ---------------------------------------------------------------------------
__global__ void k_primitive(int op, const int64_t *in, int64_t *out, int64_t n, int a, int b,
                            int c) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const i64 v = in[i];
  i64 r = 0;
  switch (op) {
    case HV_PRIM_REQUANT: r = requant_shift(v, b - a, c); break;
    case HV_PRIM_GELU: r = gelu_q16((int)v); break;
    case HV_PRIM_PLAN: r = plan_sigmoid((int)v); break;
    case HV_PRIM_RSA: r = a >= 0 ? rsa_pos(v, a) : (i64)((u64)v << (-a)); break;
  }
  out[i] = r;
}

int launch_primitive(int op, const int64_t *in, int64_t *out, int64_t n, int a, int b, int c,
                     hipStream_t s) {
  if (op == HV_PRIM_GELU_POST || op == HV_PRIM_GELU_TABLE)
    return launch_gelu_post(op == HV_PRIM_GELU_TABLE, in, out, n, a, s);
  if (op < 0 || op > HV_PRIM_RSA) return fail(HV_EVALUE, HV_ERR_OPCODE, "unknown primitive %d", op);
  if (op == HV_PRIM_REQUANT && (c < 2 || c > 63))
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "requant bits must be in [2, 63]");
  if (n <= 0) return HV_OK;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return fail(HV_EVALUE, HV_ERR_DIMENSION, "too many elements");
  hv_launch(k_primitive, dim3((unsigned)blocks), dim3(256), 0, s, op, in, out, n, a, b,
                     c);
  return check_hip(hipGetLastError(), "k_primitive launch");
}

}  // namespace hv
