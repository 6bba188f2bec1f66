/*
 * hv_oracle.c -- CPU restatement of the HeatViT-T integer golden model
 * (reference: verification/heatvit_ref/{fixed,gemm,nonlinear,layout,
 * transformer,selector,model}.py).
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker for the HIP path and the
 * "port" CPU baseline.  The product library never links or calls it.
 *
 * Width discipline.  The golden model uses unbounded Python integers.  Each
 * quantity below is carried in int64 when its reachable range provably fits
 * (bounds noted inline) and in __int128 otherwise (LayerNorm's mean^2 and
 * normalise product, exponent-aligned adds).  Left shifts that may leave
 * the target range go through sat_shl(), which saturates exactly like
 * Python's shift-then-clamp.  gcc implements >> on negative signed values as
 * an arithmetic (floor) shift, matching Python's >>.
 */
#include "hv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef __int128 i128;

/* ------------------------------------------------------------------ */
/* fixed.py                                                            */
/* ------------------------------------------------------------------ */

static i128 shl128(i128 v, int s) { return v * ((i128)1 << s); }

/* fixed.round_shift_away (fixed.py:15-25): s<0 is a left shift; s>0 rounds
 * half away from zero on the magnitude.  Callers keep |v| < 2^125 and
 * left shifts in range. */
static i128 rsa128(i128 v, int shift) {
  if (shift < 0) return shl128(v, -shift);
  if (shift == 0) return v;
  if (shift > 126) return 0; /* |v| < 2^125 <= 2^(shift-1) rounds to 0 */
  i128 mag = v < 0 ? -v : v;
  i128 r = (mag + ((i128)1 << (shift - 1))) >> shift;
  return v < 0 ? -r : r;
}

/* fixed.sat_signed (fixed.py:28-34), bits <= 64. */
static int64_t sat128(i128 v, int bits) {
  i128 hi = ((i128)1 << (bits - 1)) - 1;
  i128 lo = -hi - 1;
  if (v > hi) return (int64_t)hi;
  if (v < lo) return (int64_t)lo;
  return (int64_t)v;
}

/* sat_signed(v << sl, bits) without forming an out-of-range product. */
static int64_t sat_shl(i128 v, int sl, int bits) {
  i128 hi = ((i128)1 << (bits - 1)) - 1;
  i128 lo = -hi - 1;
  if (v == 0) return 0;
  if (sl >= bits) return v > 0 ? (int64_t)hi : (int64_t)lo;
  if (v > (hi >> sl)) return (int64_t)hi;
  if (v < (lo >> sl)) return (int64_t)lo;
  return (int64_t)shl128(v, sl);
}

/* fixed.requant (fixed.py:37-45). */
static int64_t requant128(i128 v, int src_exp, int dst_exp, int bits) {
  int shift = dst_exp - src_exp;
  if (shift >= 0) return sat128(rsa128(v, shift), bits);
  return sat_shl(v, -shift, bits);
}

void hvo_requant_array(const int64_t *v, int64_t *out, int64_t n, int src_exp, int dst_exp,
                       int bits) {
  for (int64_t i = 0; i < n; i++) out[i] = requant128(v[i], src_exp, dst_exp, bits);
}

int64_t hvo_round_shift_away(int64_t value, int shift) {
  return (int64_t)rsa128(value, shift);
}

int64_t hvo_sat_signed(int64_t value, int bits) { return sat128(value, bits); }

int64_t hvo_requant(int64_t value, int src_exp, int dst_exp, int bits) {
  return requant128(value, src_exp, dst_exp, bits);
}

/* fixed.round_div (fixed.py:57-70): the sign comes from the numerator
 * alone; the magnitude is |num| / |den| rounded half away. */
static int64_t round_div64(int64_t num, int64_t den) {
  int neg = num < 0;
  uint64_t un = neg ? (uint64_t)0 - (uint64_t)num : (uint64_t)num;
  uint64_t ud = den < 0 ? (uint64_t)0 - (uint64_t)den : (uint64_t)den;
  uint64_t q = un / ud, r = un % ud;
  if (2 * (unsigned __int128)r >= ud) q += 1;
  return neg ? -(int64_t)q : (int64_t)q;
}

int hvo_round_div(int64_t num, int64_t den, int64_t *out) {
  if (den == 0) return HVO_EVALUE;
  *out = round_div64(num, den);
  return HVO_OK;
}

/* fixed.udiv (fixed.py:48-54). */
int hvo_udiv(uint64_t num, uint64_t den, uint64_t *quot, uint64_t *rem) {
  if (den == 0) return HVO_EVALUE;
  *quot = num / den;
  *rem = num % den;
  return HVO_OK;
}

/* fixed.isqrt (fixed.py:73-80): floor square root by bitwise restoration
 * (digit-by-digit), exact over the whole uint64 range. */
uint64_t hvo_isqrt(uint64_t x, uint64_t *rem) {
  uint64_t root = 0, bit = (uint64_t)1 << 62, n = x;
  while (bit > n) bit >>= 2;
  while (bit != 0) {
    if (n >= root + bit) {
      n -= root + bit;
      root = (root >> 1) + bit;
    } else {
      root >>= 1;
    }
    bit >>= 2;
  }
  if (rem) *rem = x - root * root;
  return root;
}

/* ------------------------------------------------------------------ */
/* nonlinear.py                                                        */
/* ------------------------------------------------------------------ */

/* nonlinear.gelu (nonlinear.py:60-80), ShiftGELU in Q8.16. */
int32_t hvo_gelu(int32_t x32) {
  int64_t x = x32;
  int64_t ip = x + (x >> 1) + (x >> 3) + (x >> 4);
  int64_t ip2 = ip + (ip >> 1) - (ip >> 4);
  int64_t a = ip2 < 0 ? -ip2 : ip2;
  int64_t q = a >> 16, r = a & 0xFFFF;
  int64_t frac = (r * 11 + 15) >> 4;
  int64_t e;
  if (ip2 < 0) {
    int64_t ib = 65536 - frac;
    e = q <= 16 ? ib >> q : 0;
  } else {
    int64_t ib = 65536 + frac;
    const int64_t cap = (1 << 23) - 1;
    if (q <= 7) {
      e = ib << q;
      if (e > cap) e = cap;
    } else {
      e = cap;
    }
  }
  int64_t den = 65536 + e;
  int64_t sig = ((e << 16) + (den >> 1)) / den;
  return (int32_t)sat128(rsa128((i128)x * sig, 16), 24);
}

void hvo_gelu_array(const int32_t *x, int32_t *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = hvo_gelu(x[i]);
}

/* nonlinear.plan_sigmoid (nonlinear.py:83-95). */
int32_t hvo_plan_sigmoid(int32_t x) {
  int64_t ax = x < 0 ? -(int64_t)x : x;
  int64_t y;
  if (ax >= 327680)
    y = 65536;
  else if (ax >= 155648)
    y = (ax >> 5) + 55296;
  else if (ax >= 65536)
    y = (ax >> 3) + 40960;
  else
    y = (ax >> 2) + 32768;
  return (int32_t)(x < 0 ? 65536 - y : y);
}

/* nonlinear._softmax_exp (nonlinear.py:98-106); x_tilde <= 0. */
static int64_t softmax_exp(int64_t xt) {
  int64_t z = (-xt) / 45426;
  int64_t p = xt + z * 45426;
  int64_t s = p + 88670;
  int64_t square = (int64_t)rsa128((i128)s * s, 16);
  int64_t e = (int64_t)rsa128((i128)23495 * square, 16) + 22544;
  return z >= 63 ? 0 : e >> z;
}

int64_t hvo_softmax_exp(int64_t xt) { return softmax_exp(xt); }

/* nonlinear.softmax_scaled (nonlinear.py:109-121). */
int hvo_softmax_scaled(const int32_t *x, int n, int32_t delta2, int32_t *out) {
  if (n <= 0) return HVO_EVALUE;
  int64_t mx = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  int64_t *e = (int64_t *)malloc(sizeof(int64_t) * (size_t)n);
  int64_t sum = 0;
  for (int i = 0; i < n; i++) {
    e[i] = softmax_exp((int64_t)x[i] - mx);
    sum += e[i];
  }
  if (sum == 0) {
    free(e);
    return HVO_EVALUE;
  }
  int64_t recip = round_div64((int64_t)1 << 32, sum);
  for (int i = 0; i < n; i++) {
    int64_t ratio = (int64_t)rsa128((i128)e[i] * recip, 16);
    out[i] = (int32_t)rsa128((i128)ratio * delta2, 16);
  }
  free(e);
  return HVO_OK;
}

/* nonlinear.softmax_selector (nonlinear.py:124-127). */
int hvo_softmax_selector(const int32_t *x, int n, int32_t *out) {
  int rc = hvo_softmax_scaled(x, n, 65536, out);
  if (rc) return rc;
  for (int i = 0; i < n; i++)
    if (out[i] > 65536) out[i] = 65536;
  return HVO_OK;
}

/* nonlinear.softmax_attention (nonlinear.py:130-133), delta2 = 65536. */
int hvo_softmax_attention(const int32_t *x, int n, uint8_t *out) {
  int32_t *s = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
  int rc = hvo_softmax_scaled(x, n, 65536, s);
  if (rc == HVO_OK)
    for (int i = 0; i < n; i++) {
      int64_t v = (int64_t)rsa128(s[i], 8);
      out[i] = (uint8_t)(v > 255 ? 255 : v);
    }
  free(s);
  return rc;
}

/* nonlinear.layernorm (nonlinear.py:136-186), D = 192.
 * Bounds: x_q32 < 2^39, sum_x < 2^47, sum_square < 2^54 (int64);
 * mean^2 < 2^78 and (x_q32 - mean) * inv_std < 2^82 (int128). */
int hvo_layernorm(const int8_t *x, const int8_t *gamma, const int8_t *beta,
                  int x_exp, int gamma_exp, int beta_exp, int out_exp,
                  int8_t *out, int *negative_variance) {
  if (x_exp < -32 || x_exp > 0) return HVO_EVALUE;
  int64_t xq[HVO_D];
  int64_t sum_x = 0, sum_sq = 0;
  for (int c = 0; c < HVO_D; c++) {
    xq[c] = (int64_t)x[c] * ((int64_t)1 << (x_exp + 32));
    sum_x += xq[c];
    sum_sq += (int64_t)rsa128((i128)x[c] * x[c], -(2 * x_exp + 32));
  }
  int64_t mean = round_div64(sum_x, HVO_D);
  int64_t e2 = round_div64(sum_sq, HVO_D);
  i128 mean_sq = rsa128((i128)mean * mean, 32);
  i128 var = (i128)e2 - mean_sq;
  if (negative_variance) *negative_variance = var < 0;
  if (var < 0) var = 0;
  uint64_t std_q16 = hvo_isqrt((uint64_t)var + 4295, NULL);
  int64_t inv = round_div64((int64_t)1 << 48, (int64_t)std_q16);
  int common = gamma_exp - 16 < beta_exp ? gamma_exp - 16 : beta_exp;
  for (int c = 0; c < HVO_D; c++) {
    int64_t norm = sat128(rsa128((i128)(xq[c] - mean) * inv, 48), 24);
    i128 aligned = shl128((i128)norm * gamma[c], gamma_exp - 16 - common) +
                   shl128((i128)beta[c], beta_exp - common);
    out[c] = (int8_t)requant128(aligned, common, out_exp, 8);
  }
  return HVO_OK;
}

/* ------------------------------------------------------------------ */
/* gemm.py                                                             */
/* ------------------------------------------------------------------ */

/* gemm.gemm / gemm.gemm_numpy (gemm.py:58-120).  With |a| <= 255 and
 * |b| <= 128 every partial sum stays below 2^31 while k <= 65792, so int32
 * accumulation equals the int64 one and the overflow check cannot fire;
 * longer k takes the int64 route and checks as gemm_numpy does. */
int hvo_gemm(const void *a_, const int8_t *b, const int32_t *bias, int m, int n,
             int k, int transpose_b, int a_unsigned, int64_t *acc) {
  const int8_t *as = (const int8_t *)a_;
  const uint8_t *au = (const uint8_t *)a_;
  if (k <= 65792) {
    int32_t *row = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
    for (int r = 0; r < m; r++) {
      if (!transpose_b) {
        for (int c = 0; c < n; c++) row[c] = 0;
        for (int kk = 0; kk < k; kk++) {
          int32_t av = a_unsigned ? (int32_t)au[(size_t)r * k + kk]
                                  : (int32_t)as[(size_t)r * k + kk];
          const int8_t *brow = b + (size_t)kk * n;
          for (int c = 0; c < n; c++) row[c] += av * (int32_t)brow[c];
        }
      } else {
        for (int c = 0; c < n; c++) {
          const int8_t *brow = b + (size_t)c * k;
          int32_t s = 0;
          if (a_unsigned)
            for (int kk = 0; kk < k; kk++)
              s += (int32_t)au[(size_t)r * k + kk] * (int32_t)brow[kk];
          else
            for (int kk = 0; kk < k; kk++)
              s += (int32_t)as[(size_t)r * k + kk] * (int32_t)brow[kk];
          row[c] = s;
        }
      }
      for (int c = 0; c < n; c++)
        acc[(size_t)r * n + c] = (int64_t)row[c] + (bias ? bias[c] : 0);
    }
    free(row);
    return HVO_OK;
  }
  for (int r = 0; r < m; r++)
    for (int c = 0; c < n; c++) {
      int64_t s = 0;
      for (int kk = 0; kk < k; kk++) {
        int64_t av = a_unsigned ? au[(size_t)r * k + kk] : as[(size_t)r * k + kk];
        int64_t bv = transpose_b ? b[(size_t)c * k + kk] : b[(size_t)kk * n + c];
        s += av * bv;
      }
      if (s < -((int64_t)1 << 31) || s > ((int64_t)1 << 31) - 1) return HVO_EOVERFLOW;
      acc[(size_t)r * n + c] = s + (bias ? bias[c] : 0);
    }
  return HVO_OK;
}

/* gemm.gemm_writeback (gemm.py:123-139). */
int hvo_gemm_writeback(const int64_t *acc, int count, int src_exp, int dst_exp,
                       int bits, void *out) {
  if (bits == 8) {
    int8_t *o = (int8_t *)out;
    for (int i = 0; i < count; i++) o[i] = (int8_t)requant128(acc[i], src_exp, dst_exp, 8);
    return HVO_OK;
  }
  if (bits == 32) {
    int32_t *o = (int32_t *)out;
    for (int i = 0; i < count; i++) o[i] = (int32_t)requant128(acc[i], src_exp, dst_exp, 32);
    return HVO_OK;
  }
  return HVO_EVALUE;
}

/* ------------------------------------------------------------------ */
/* transformer.py / layout.py                                          */
/* ------------------------------------------------------------------ */

/* transformer._align_add_requant (transformer.py:96-101). */
static int8_t align_add(int64_t main, int main_exp, int64_t aux, int aux_exp,
                        int out_exp) {
  int common = main_exp < aux_exp ? main_exp : aux_exp;
  i128 s = shl128(main, main_exp - common) + shl128(aux, aux_exp - common);
  return (int8_t)requant128(s, common, out_exp, 8);
}

/* layout.patchify (layout.py:31-72): raster patch order, within-patch
 * flatten (in_row, in_col, channel); patches [(H/P)*(W/P)][P*P*3]. */
int hvo_patchify(const int8_t *image, int W, int H, int P, int8_t *patches) {
  if (W <= 0 || P <= 0 || W % P || H <= 0 || H % P) return HVO_EVALUE;
  int pc_n = W / P, pr_n = H / P, kdim = P * P * 3;
  for (int pr = 0; pr < pr_n; pr++)
    for (int pc = 0; pc < pc_n; pc++) {
      int8_t *v = patches + (size_t)(pr * pc_n + pc) * kdim;
      for (int ir = 0; ir < P; ir++)
        for (int ic = 0; ic < P; ic++)
          for (int ch = 0; ch < 3; ch++)
            v[(ir * P + ic) * 3 + ch] =
                image[((size_t)(pr * P + ir) * W + pc * P + ic) * 3 + ch];
    }
  return HVO_OK;
}

/* p2_export_weights.real_image_list (tools/p2/p2_export_weights.py:246-251):
 * float CHW [3][H][W] -> int8 NHWC, q = clamp(round(x / 2^exp), -128, 127)
 * with torch.round's ties-to-even (rintf in the default rounding mode) on
 * the float32 quotient.  NaN (an undefined int8 cast there) gives 0. */
int hvo_quantize_image(const float *chw, int W, int H, int input_exp, int8_t *nhwc) {
  if (W <= 0 || H <= 0 || input_exp < -32 || input_exp > 31) return HVO_EVALUE;
  const float step = ldexpf(1.0f, input_exp);
  for (int y = 0; y < H; y++)
    for (int x = 0; x < W; x++)
      for (int ch = 0; ch < 3; ch++) {
        float v = rintf(chw[((size_t)ch * H + y) * W + x] / step);
        int q = v != v ? 0 : v < -128.f ? -128 : v > 127.f ? 127 : (int)v;
        nhwc[((size_t)y * W + x) * 3 + ch] = (int8_t)q;
      }
  return HVO_OK;
}

/* transformer.patch_embedding (transformer.py:104-145) over hvo_patchify. */
int hvo_patch_embedding(const int8_t *image, const hvo_patch *p, int8_t *out) {
  int W = p->width, H = p->height, P = p->patch;
  if (W <= 0 || P <= 0 || W % P || H % P) return HVO_EVALUE;
  int pc_n = W / P, pr_n = H / P, np = pc_n * pr_n, kdim = P * P * 3;
  if (np + 1 != HVO_TOKENS) return HVO_EVALUE;
  int8_t *patches = (int8_t *)malloc((size_t)np * kdim);
  hvo_patchify(image, W, H, P, patches);
  int64_t *acc = (int64_t *)malloc(sizeof(int64_t) * (size_t)np * HVO_D);
  int rc = hvo_gemm(patches, p->weight, p->bias, np, HVO_D, kdim, 0, 0, acc);
  if (rc == HVO_OK) {
    int src = p->image_exp + p->weight_exp;
    for (int c = 0; c < HVO_D; c++)
      out[c] = align_add(p->cls[c], p->cls_exp, p->pos[c], p->pos_exp, p->tokens_exp);
    for (int i = 0; i < np; i++)
      for (int c = 0; c < HVO_D; c++) {
        int64_t e = requant128(acc[(size_t)i * HVO_D + c], src, p->activation_exp, 8);
        out[(size_t)(i + 1) * HVO_D + c] =
            align_add(e, p->activation_exp, p->pos[(size_t)(i + 1) * HVO_D + c],
                      p->pos_exp, p->tokens_exp);
      }
  }
  free(acc);
  free(patches);
  return rc;
}

/* LayerNorm over n rows; *warn (when given) gets HVO_WARN_LN_NEGATIVE_VARIANCE
 * ORed in when any row's variance was negative (the engine's warning bit 2,
 * heatvit_pkg.sv:122; the golden model returns the flag per row and its
 * callers drop it, model.py:63, transformer.py:211, 338). */
static int layernorm_rows(const int8_t *x, int n, const int8_t *g, const int8_t *b,
                          int xe, int ge, int be, int oe, int8_t *out, int32_t *warn) {
  for (int r = 0; r < n; r++) {
    int neg = 0;
    int rc = hvo_layernorm(x + (size_t)r * HVO_D, g, b, xe, ge, be, oe,
                           out + (size_t)r * HVO_D, &neg);
    if (rc) return rc;
    if (neg && warn) *warn |= HVO_WARN_LN_NEGATIVE_VARIANCE;
  }
  return HVO_OK;
}

/* transformer.mhsa (transformer.py:201-284) + layout.qkv_unpack /
 * head_concat (layout.py:92-155): Q, K, V of head h are columns
 * [kind*192 + h*64, +64) of the fused [N][576] QKV. */
static int mhsa(const int8_t *x, int n, const hvo_block *p, int8_t *msa,
                hvo_block_ckpt *ck) {
  int rc;
  size_t nn = (size_t)n * n;
  int8_t *ln1 = (int8_t *)malloc((size_t)n * HVO_D);
  int8_t *fused = (int8_t *)malloc((size_t)n * 576);
  int8_t *concat = (int8_t *)malloc((size_t)n * HVO_D);
  int64_t *acc = (int64_t *)malloc(sizeof(int64_t) * ((size_t)n * 576 > nn ? (size_t)n * 576 : nn));
  int8_t *qh = (int8_t *)malloc((size_t)n * 64), *kh = (int8_t *)malloc((size_t)n * 64),
         *vh = (int8_t *)malloc((size_t)n * 64);
  int32_t *score = (int32_t *)malloc(sizeof(int32_t) * nn);
  int32_t *q16 = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
  uint8_t *prob = (uint8_t *)malloc(nn);
  int8_t *ctx = (int8_t *)malloc((size_t)n * 64);

  rc = layernorm_rows(x, n, p->ln1_gamma, p->ln1_beta, p->x_exp, p->gamma1_exp,
                      p->beta1_exp, p->ln1_out_exp, ln1, ck ? ck->warnings : NULL);
  if (rc) goto done;
  rc = hvo_gemm(ln1, p->wqkv, p->bqkv, n, 576, HVO_D, 0, 0, acc);
  if (rc) goto done;
  hvo_gemm_writeback(acc, n * 576, p->ln1_out_exp + p->wqkv_exp, p->qkv_out_exp, 8, fused);

  for (int h = 0; h < HVO_HEADS; h++) {
    for (int t = 0; t < n; t++)
      for (int l = 0; l < 64; l++) {
        qh[t * 64 + l] = fused[(size_t)t * 576 + 0 * 192 + h * 64 + l];
        kh[t * 64 + l] = fused[(size_t)t * 576 + 1 * 192 + h * 64 + l];
        vh[t * 64 + l] = fused[(size_t)t * 576 + 2 * 192 + h * 64 + l];
      }
    rc = hvo_gemm(qh, kh, NULL, n, n, 64, 1, 0, acc);
    if (rc) goto done;
    hvo_gemm_writeback(acc, (int)nn, 2 * p->qkv_out_exp, p->score_exp, 32, score);
    /* q16 = sat24(rsa(score, -(score_exp + 13))) (transformer.py:236-254) */
    for (int r = 0; r < n; r++) {
      for (int c = 0; c < n; c++) {
        int s = -(p->score_exp + 13);
        int64_t v = score[(size_t)r * n + c];
        q16[c] = (int32_t)(s >= 0 ? sat128(rsa128(v, s), 24) : sat_shl(v, -s, 24));
      }
      rc = hvo_softmax_attention(q16, n, prob + (size_t)r * n);
      if (rc) goto done;
    }
    rc = hvo_gemm(prob, vh, NULL, n, 64, n, 0, 1, acc);
    if (rc) goto done;
    hvo_gemm_writeback(acc, n * 64, p->prob_exp + p->qkv_out_exp, p->context_out_exp, 8, ctx);
    for (int t = 0; t < n; t++)
      for (int l = 0; l < 64; l++) concat[(size_t)t * HVO_D + h * 64 + l] = ctx[t * 64 + l];
    if (ck) {
      if (ck->score) memcpy(ck->score + (size_t)h * nn, score, sizeof(int32_t) * nn);
      if (ck->prob) memcpy(ck->prob + (size_t)h * nn, prob, nn);
      if (ck->context) memcpy(ck->context + (size_t)h * n * 64, ctx, (size_t)n * 64);
    }
  }
  rc = hvo_gemm(concat, p->wproj, p->bproj, n, HVO_D, HVO_D, 0, 0, acc);
  if (rc) goto done;
  hvo_gemm_writeback(acc, n * HVO_D, p->context_out_exp + p->wproj_exp, p->msa_out_exp, 8, msa);
  if (ck) {
    if (ck->ln1) memcpy(ck->ln1, ln1, (size_t)n * HVO_D);
    if (ck->fused_qkv) memcpy(ck->fused_qkv, fused, (size_t)n * 576);
    if (ck->concat) memcpy(ck->concat, concat, (size_t)n * HVO_D);
    if (ck->msa) memcpy(ck->msa, msa, (size_t)n * HVO_D);
  }
done:
  free(ln1); free(fused); free(concat); free(acc); free(qh); free(kh); free(vh);
  free(score); free(q16); free(prob); free(ctx);
  return rc;
}

/* transformer.ffn (transformer.py:328-384). */
static int ffn(const int8_t *y, int n, const hvo_block *p, int8_t *z, hvo_block_ckpt *ck) {
  int rc;
  int8_t *ln2 = (int8_t *)malloc((size_t)n * HVO_D);
  int8_t *hidden = (int8_t *)malloc((size_t)n * HVO_FFN);
  int8_t *fo = (int8_t *)malloc((size_t)n * HVO_D);
  int64_t *acc = (int64_t *)malloc(sizeof(int64_t) * (size_t)n * HVO_FFN);
  rc = layernorm_rows(y, n, p->ln2_gamma, p->ln2_beta, p->ffn_x_exp, p->gamma2_exp,
                      p->beta2_exp, p->ln2_out_exp, ln2, ck ? ck->warnings : NULL);
  if (rc) goto done;
  rc = hvo_gemm(ln2, p->w1, p->b1, n, HVO_FFN, HVO_D, 0, 0, acc);
  if (rc) goto done;
  {
    int src = p->ln2_out_exp + p->w1_exp;
    for (size_t i = 0; i < (size_t)n * HVO_FFN; i++) {
      int32_t q = (int32_t)requant128(acc[i], src, -16, 24);
      hidden[i] = (int8_t)requant128(hvo_gelu(q), -16, p->hidden_out_exp, 8);
    }
  }
  rc = hvo_gemm(hidden, p->w2, p->b2, n, HVO_D, HVO_FFN, 0, 0, acc);
  if (rc) goto done;
  hvo_gemm_writeback(acc, n * HVO_D, p->hidden_out_exp + p->w2_exp, p->ffn_out_exp, 8, fo);
  for (size_t i = 0; i < (size_t)n * HVO_D; i++)
    z[i] = align_add(y[i], p->ffn_x_exp, fo[i], p->ffn_out_exp, p->out_exp);
  if (ck) {
    if (ck->ln2) memcpy(ck->ln2, ln2, (size_t)n * HVO_D);
    if (ck->hidden) memcpy(ck->hidden, hidden, (size_t)n * HVO_FFN);
    if (ck->ffn_out) memcpy(ck->ffn_out, fo, (size_t)n * HVO_D);
  }
done:
  free(ln2); free(hidden); free(fo); free(acc);
  return rc;
}

/* transformer.transformer_block (transformer.py:401-431). */
int hvo_transformer_block(const int8_t *x, int n, const hvo_block *p, int8_t *z,
                          hvo_block_ckpt *ck) {
  if (n <= 0) return HVO_EVALUE;
  int8_t *msa = (int8_t *)malloc((size_t)n * HVO_D);
  int8_t *y = (int8_t *)malloc((size_t)n * HVO_D);
  int rc = mhsa(x, n, p, msa, ck);
  if (rc == HVO_OK) {
    for (size_t i = 0; i < (size_t)n * HVO_D; i++)
      y[i] = align_add(x[i], p->x_exp, msa[i], p->msa_out_exp, p->ffn_x_exp);
    if (ck && ck->y) memcpy(ck->y, y, (size_t)n * HVO_D);
    rc = ffn(y, n, p, z, ck);
  }
  free(msa);
  free(y);
  return rc;
}

/* ------------------------------------------------------------------ */
/* selector.py                                                         */
/* ------------------------------------------------------------------ */

static int64_t sat_q016(int64_t v) { return v < 0 ? 0 : v > 65536 ? 65536 : v; }

/* selector._gemm_gelu (selector.py:89-99) over rows of a row-major A. */
static void gemm_gelu(const int8_t *a, int m, int k, const int8_t *w, const int32_t *b,
                      int n, int act_exp, int wt_exp, int dst_exp, int8_t *out) {
  int64_t *acc = (int64_t *)malloc(sizeof(int64_t) * (size_t)m * n);
  hvo_gemm(a, w, b, m, n, k, 0, 0, acc);
  int src = act_exp + wt_exp;
  for (size_t i = 0; i < (size_t)m * n; i++)
    out[i] = (int8_t)requant128(hvo_gelu((int32_t)requant128(acc[i], src, -16, 24)), -16,
                                dst_exp, 8);
  free(acc);
}

/* selector.fuse_head_scores (selector.py:392-418): scores [3][C],
 * weights [C][3]; a zero weight sum falls back to the mean of the three
 * scores and raises WARN_HEAD_DEN_ZERO (returned as *warn = 1). */
void hvo_fuse_head_scores(const int32_t *scores, const int32_t *weights, int C,
                          int32_t *fused, int *warn) {
  *warn = 0;
  for (int c = 0; c < C; c++) {
    int64_t num = 0, den = 0;
    for (int h = 0; h < 3; h++) {
      num += (int64_t)scores[(size_t)h * C + c] * weights[c * 3 + h];
      den += weights[c * 3 + h];
    }
    if (den == 0) {
      num = (int64_t)scores[c] + scores[(size_t)C + c] + scores[(size_t)2 * C + c];
      den = 3;
      *warn = 1;
    }
    fused[c] = (int32_t)sat_q016(round_div64(num, den));
  }
}

/* selector.finalize_tokens (selector.py:421-500).  kept_index receives the
 * normal-candidate index (0-based) of every kept token, in order. */
int hvo_finalize_tokens(const int8_t *cls, const int8_t *normal, int n_normal,
                        const int8_t *incoming, const int32_t *scores, int n_scores,
                        int width, int8_t *out, int32_t *kept_index,
                        hvo_selector_state *st) {
  if (width <= 0) return HVO_EVALUE;
  for (int i = 0; i < n_scores; i++)
    if (scores[i] < 0 || scores[i] > 65536) return HVO_EVALUE;
  int64_t pkg_score = 0;
  if (incoming) {
    if (n_normal == 0) return HVO_EVALUE;
    if (n_scores != n_normal + 1) return HVO_EVALUE;
    pkg_score = scores[n_scores - 1];
  } else if (n_scores != n_normal) {
    return HVO_EVALUE;
  }
  memcpy(out, cls, (size_t)width);
  int kept = 0, n_part = 0;
  int64_t den = 0;
  for (int i = 0; i < n_normal; i++) {
    if (scores[i] >= 32768) {
      memcpy(out + (size_t)(1 + kept) * width, normal + (size_t)i * width, (size_t)width);
      if (kept_index) kept_index[kept] = i;
      kept++;
    } else {
      n_part++;
      den += scores[i];
    }
  }
  if (incoming) {
    n_part++;
    den += pkg_score;
  }
  int warnings = 0;
  int exists = n_part > 0;
  if (exists) {
    int8_t *pkg = out + (size_t)(1 + kept) * width;
    if (den == 0) warnings |= HVO_WARN_PACKAGE_DEN_ZERO;
    for (int d = 0; d < width; d++) {
      int64_t num = 0;
      for (int i = 0; i < n_normal; i++)
        if (scores[i] < 32768)
          num += (den == 0 ? 1 : (int64_t)scores[i]) * normal[(size_t)i * width + d];
      if (incoming) num += (den == 0 ? 1 : pkg_score) * incoming[d];
      pkg[d] = (int8_t)sat128(round_div64(num, den == 0 ? n_part : den), 8);
    }
  }
  st->token_count = 1 + kept + exists;
  st->package_present = exists;
  st->kept_normal_count = kept;
  st->pruned_normal_count = n_part - (incoming ? 1 : 0);
  st->warnings = warnings;
  return HVO_OK;
}

/* selector.token_selector (selector.py:503-563) with its stages
 * per_head_local_mlp :253, mean_over_candidates :273, concat_local_global
 * :292, per_head_score_mlp :338 (score_mlp_layers :307), mean_over_head_lanes
 * :358, head_weight_mlp :370, fuse_head_scores :392. */
int hvo_token_selector(const int8_t *tokens, int n, int package_present,
                       const hvo_selector *p, int8_t *out_tokens, int32_t *kept_index,
                       hvo_selector_state *st, hvo_selector_ckpt *ck) {
  if (n < 2) return HVO_EVALUE;
  int C = n - 1, rc = HVO_OK;
  const int8_t *cand = tokens + HVO_D; /* [C][192] = [C][3][64] */
  int8_t *a = (int8_t *)malloc((size_t)C * 64);
  int8_t *local = (int8_t *)malloc((size_t)3 * C * 32);
  int8_t glob[3][32];
  int8_t *lg = (int8_t *)malloc((size_t)C * 64);
  int8_t *h1 = (int8_t *)malloc((size_t)C * 32);
  int8_t *h2 = (int8_t *)malloc((size_t)C * 16);
  int64_t *acc = (int64_t *)malloc(sizeof(int64_t) * (size_t)C * 3);
  int32_t *hs = (int32_t *)malloc(sizeof(int32_t) * 3 * (size_t)C);
  int8_t *stats = (int8_t *)malloc((size_t)C * 3);
  int8_t *hwh = (int8_t *)malloc((size_t)C * 3);
  int32_t *hw = (int32_t *)malloc(sizeof(int32_t) * 3 * (size_t)C);
  int32_t *fused = (int32_t *)malloc(sizeof(int32_t) * (size_t)C);
  int warn_head = 0;

  /* per_head_local_mlp */
  for (int h = 0; h < 3; h++) {
    for (int c = 0; c < C; c++) memcpy(a + (size_t)c * 64, cand + (size_t)c * HVO_D + h * 64, 64);
    gemm_gelu(a, C, 64, p->local_w + (size_t)h * 64 * 32, p->local_b + h * 32, 32, p->in_exp,
              p->local_w_exp, p->local_out_exp, local + (size_t)h * C * 32);
  }
  /* mean_over_candidates */
  for (int h = 0; h < 3; h++)
    for (int j = 0; j < 32; j++) {
      int64_t s = 0;
      for (int c = 0; c < C; c++) s += local[((size_t)h * C + c) * 32 + j];
      glob[h][j] = (int8_t)sat128(round_div64(s, C), 8);
    }
  /* concat_local_global + score MLP + selector softmax */
  for (int h = 0; h < 3; h++) {
    for (int c = 0; c < C; c++) {
      memcpy(lg + (size_t)c * 64, local + ((size_t)h * C + c) * 32, 32);
      memcpy(lg + (size_t)c * 64 + 32, glob[h], 32);
    }
    gemm_gelu(lg, C, 64, p->w1 + (size_t)h * 64 * 32, p->b1 + h * 32, 32, p->concat_out_exp,
              p->score_w1_exp, p->h1_out_exp, h1);
    gemm_gelu(h1, C, 32, p->w2 + (size_t)h * 32 * 16, p->b2 + h * 16, 16, p->h1_out_exp,
              p->score_w2_exp, p->h2_out_exp, h2);
    if (ck && ck->h2) memcpy(ck->h2 + (size_t)h * C * 16, h2, (size_t)C * 16);
    hvo_gemm(h2, p->w3 + (size_t)h * 16 * 2, p->b3 + h * 2, C, 2, 16, 0, 0, acc);
    for (int c = 0; c < C; c++) {
      int32_t q[2], sm[2];
      for (int j = 0; j < 2; j++) {
        int64_t logit = requant128(acc[c * 2 + j], p->h2_out_exp + p->score_w3_exp,
                                   p->logits_out_exp, 8);
        q[j] = (int32_t)requant128(logit, p->logits_out_exp, -16, 24);
      }
      hvo_softmax_selector(q, 2, sm);
      hs[(size_t)h * C + c] = sm[1];
    }
  }
  /* mean_over_head_lanes: raw lane means, relabelled, no rescale */
  for (int c = 0; c < C; c++)
    for (int h = 0; h < 3; h++) {
      int64_t s = 0;
      for (int l = 0; l < 64; l++) s += cand[(size_t)c * HVO_D + h * 64 + l];
      stats[c * 3 + h] = (int8_t)sat128(round_div64(s, 64), 8);
    }
  /* head_weight_mlp */
  gemm_gelu(stats, C, 3, p->hw_w1, p->hw_b1, 3, p->stats_out_exp, p->hw_w1_exp,
            p->hw_hidden_out_exp, hwh);
  hvo_gemm(hwh, p->hw_w2, p->hw_b2, C, 3, 3, 0, 0, acc);
  for (int i = 0; i < C * 3; i++)
    hw[i] = (int32_t)sat_q016(hvo_plan_sigmoid(
        (int32_t)requant128(acc[i], p->hw_hidden_out_exp + p->hw_w2_exp, -16, 24)));
  /* fuse_head_scores */
  hvo_fuse_head_scores(hs, hw, C, fused, &warn_head);
  /* finalize */
  {
    int pp = package_present ? 1 : 0;
    rc = hvo_finalize_tokens(tokens, cand, C - pp, pp ? cand + (size_t)(C - 1) * HVO_D : NULL,
                             fused, C, HVO_D, out_tokens, kept_index, st);
    if (rc == HVO_OK) st->warnings |= warn_head;
  }
  if (ck) {
    if (ck->local) memcpy(ck->local, local, (size_t)3 * C * 32);
    if (ck->global) memcpy(ck->global, glob, sizeof(glob));
    if (ck->head_scores) memcpy(ck->head_scores, hs, sizeof(int32_t) * 3 * (size_t)C);
    if (ck->head_stats) memcpy(ck->head_stats, stats, (size_t)C * 3);
    if (ck->head_weights) memcpy(ck->head_weights, hw, sizeof(int32_t) * 3 * (size_t)C);
    if (ck->fused) memcpy(ck->fused, fused, sizeof(int32_t) * (size_t)C);
  }
  free(a); free(local); free(lg); free(h1); free(h2); free(acc); free(hs);
  free(stats); free(hwh); free(hw); free(fused);
  return rc;
}

/* ------------------------------------------------------------------ */
/* model.py                                                            */
/* ------------------------------------------------------------------ */

/* model.HeatViTModel.infer (model.py:73-123). */
int hvo_model_infer(const int8_t *image, const hvo_model *m, int32_t *logits,
                    int8_t *ckpt, int32_t *ckpt_rows, hvo_selector_state *summary,
                    int32_t *warnings) {
  int32_t warn = 0;
  hvo_block_ckpt bck;
  memset(&bck, 0, sizeof bck);
  bck.warnings = &warn;
  const size_t slot = (size_t)HVO_TOKENS * HVO_D;
  int8_t *x = (int8_t *)malloc(slot), *nx = (int8_t *)malloc(slot);
  int8_t *fln = (int8_t *)malloc(slot);
  int n = HVO_TOKENS, pkg = 0, sel = 0, rc;
  if (ckpt_rows)
    for (int i = 0; i < HVO_CKPT_SLOTS; i++) ckpt_rows[i] = 0;
  rc = hvo_patch_embedding(image, &m->patch, x);
  if (rc) goto done;
  if (ckpt) memcpy(ckpt, x, slot);
  if (ckpt_rows) ckpt_rows[0] = n;
  for (int b = 1; b <= 12; b++) {
    int is_sel = 0;
    for (int s = 0; s < m->n_selectors; s++)
      if (m->selector_blocks[s] == b) is_sel = 1;
    if (is_sel) {
      hvo_selector_state st;
      rc = hvo_token_selector(x, n, pkg, &m->selectors[sel], nx, NULL, &st, NULL);
      if (rc) goto done;
      if (summary) summary[sel] = st;
      warn |= st.warnings;
      n = st.token_count;
      pkg = st.package_present;
      memcpy(x, nx, (size_t)n * HVO_D);
      sel++;
      if (ckpt) memcpy(ckpt + (size_t)sel * slot, x, (size_t)n * HVO_D);
      if (ckpt_rows) ckpt_rows[sel] = n;
    }
    rc = hvo_transformer_block(x, n, &m->blocks[b - 1], nx, &bck);
    if (rc) goto done;
    memcpy(x, nx, (size_t)n * HVO_D);
    if (ckpt) memcpy(ckpt + (size_t)(3 + b) * slot, x, (size_t)n * HVO_D);
    if (ckpt_rows) ckpt_rows[3 + b] = n;
  }
  rc = layernorm_rows(x, n, m->final_gamma, m->final_beta, m->blocks[11].out_exp,
                      m->final_gamma_exp, m->final_beta_exp, m->final_ln_out_exp, fln,
                      &warn);
  if (rc) goto done;
  if (ckpt) memcpy(ckpt + (size_t)16 * slot, fln, (size_t)n * HVO_D);
  if (ckpt_rows) ckpt_rows[16] = n;
  {
    int64_t *acc = (int64_t *)malloc(sizeof(int64_t) * HVO_CLASSES);
    rc = hvo_gemm(fln, m->head_w, m->head_b, 1, HVO_CLASSES, HVO_D, 0, 0, acc);
    if (rc == HVO_OK)
      hvo_gemm_writeback(acc, HVO_CLASSES, m->final_ln_out_exp + m->head_w_exp, -14, 32, logits);
    free(acc);
  }
done:
  free(x); free(nx); free(fln);
  if (warnings) *warnings = warn;
  return rc;
}

int hvo_model_infer_batch(const int8_t *images, int count, const hvo_model *m, int threads,
                          int32_t *logits, int32_t *token_counts, int32_t *status,
                          int32_t *warnings) {
  const size_t img = (size_t)m->patch.width * m->patch.height * 3;
  int worst = HVO_OK;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1) reduction(min : worst)
#endif
  for (int i = 0; i < count; i++) {
    int32_t rows[HVO_CKPT_SLOTS];
    int rc = hvo_model_infer(images + (size_t)i * img, m, logits + (size_t)i * HVO_CLASSES,
                             NULL, rows, NULL, warnings ? warnings + i : NULL);
    if (status) status[i] = rc;
    if (token_counts) {
      /* rows entering blocks 1, 4, 7, 10 */
      token_counts[i * 4 + 0] = rows[4];
      token_counts[i * 4 + 1] = rows[7];
      token_counts[i * 4 + 2] = rows[10];
      token_counts[i * 4 + 3] = rows[13];
    }
    if (rc < worst) worst = rc;
  }
  (void)threads;
  return worst;
}
