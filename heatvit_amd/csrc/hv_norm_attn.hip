// hv_norm_attn.hip -- integer LayerNorm, fused varlen attention and the
// element-wise evaluators of the golden model's nonlinear primitives.
#include "hv_device.h"
#include "hv_internal.h"

namespace hv {

// ---------------------------------------------------------------------------
// LayerNorm (nonlinear.layernorm, nonlinear.py:136-186), D = 192.
// One wavefront per row, three channels per lane; row statistics are exact
// wavefront sums of int64 terms, mean^2 and the normalise product use
// 128-bit arithmetic (mean^2 < 2^78, (x_q32 - mean) * inv_std < 2^82).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_layernorm(const int8_t *__restrict__ x,
                                                   const int8_t *__restrict__ gamma,
                                                   const int8_t *__restrict__ beta,
                                                   int8_t *__restrict__ y, int rows,
                                                   const int32_t *rows_dev, int x_exp,
                                                   int g_exp, int b_exp, int out_exp,
                                                   uint8_t *neg_var) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int R = rows_dev ? min(*rows_dev, rows) : rows;
  if (row >= R) return;
  const int8_t *xr = x + (size_t)row * 192;
  const int sh = x_exp + 32;             // [0, 32]
  const int sq_shift = -(2 * x_exp + 32);  // round_shift_away shift of x^2
  int xv[3];
  i64 xq[3], sx = 0, ss = 0;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    xv[j] = xr[lane + 64 * j];
    xq[j] = (i64)xv[j] * (1ll << sh);
    sx += xq[j];
    const i64 x2 = (i64)(xv[j] * xv[j]);
    ss += sq_shift >= 0 ? rsa_pos(x2, sq_shift) : x2 * (1ll << (-sq_shift));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
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
  const int common = (g_exp - 16) < b_exp ? (g_exp - 16) : b_exp;
  const int gs = g_exp - 16 - common, bs = b_exp - common, os = out_exp - common;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int c = lane + 64 * j;
    const i64 norm = sat128(rsa128((i128)(xq[j] - mean) * inv, 48), 24);
    const i128 al = (i128)(norm * gamma[c]) * ((i128)1 << gs) + (i128)beta[c] * ((i128)1 << bs);
    y[(size_t)row * 192 + c] = (int8_t)requant128(al, os, 8);
  }
  if (neg_var && lane == 0) neg_var[row] = neg ? 1 : 0;
}

int launch_layernorm(const int8_t *x, const int8_t *g, const int8_t *b, int8_t *y, int rows,
                     const int32_t *rows_dev, int x_exp, int g_exp, int b_exp, int out_exp,
                     uint8_t *neg_var, hipStream_t s) {
  if (x_exp < -32 || x_exp > 0)
    return fail(HV_EVALUE, "layernorm input scale must be in [-32, 0] (got %d)", x_exp);
  if (rows <= 0) return HV_OK;
  hipLaunchKernelGGL(k_layernorm, dim3((rows + 3) / 4), dim3(256), 0, s, x, g, b, y, rows,
                     rows_dev, x_exp, g_exp, b_exp, out_exp, neg_var);
  return check_hip(hipGetLastError(), "k_layernorm launch");
}

// ---------------------------------------------------------------------------
// Fused attention core of mhsa (transformer.py:228-266) for one (image,
// head): S = Q K^T (int8 MFMA 16x16x64), score = requant(S, 2*qkv, score,
// 32), q16 = sat24(rsa(score, -(score+13))), attention softmax to UQ0.8,
// context = requant(P V, prob+qkv, ctx, 8) written in head-concat layout
// (layout.py:132-155).  P is unsigned: P V = (P-128) V + 128 * colsum(V) so
// the signed MFMA applies; |acc| <= 197*255*128 < 2^23.
// Workgroup = 4 wavefronts, each owning 16-row query tiles; K rows and V^T
// (keys contiguous per head lane) are staged in LDS once per (image, head).
// ---------------------------------------------------------------------------
static constexpr int kMaxKeys = 208;   // 13 tiles of 16
static constexpr int kKeyPad = 256;    // PV reduction length (4 x 64)
static constexpr int kKStride = 80;    // LDS row strides chosen so that the
static constexpr int kVStride = 272;   // 16 lanes of a fragment read hit
static constexpr int kPStride = 272;   // disjoint banks

__global__ __launch_bounds__(256) void k_attention(AttnArgs g) {
  __shared__ __attribute__((aligned(16))) int8_t Ks[kMaxKeys * kKStride];
  __shared__ __attribute__((aligned(16))) int8_t Vt[64 * kVStride];
  __shared__ __attribute__((aligned(16))) int8_t Ps[4 * 16 * kPStride];
  __shared__ int colsum[64];

  const int b = blockIdx.x / 3, h = blockIdx.x - 3 * (blockIdx.x / 3);
  const int row0 = g.offsets[b];
  const int N = g.offsets[b + 1] - row0;
  if (N <= 0 || N > HV_MAX_TOKENS) return;  // host validates N <= 197
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n16 = (N + 15) >> 4;       // key / query tiles
  const int n64 = (N + 63) >> 6;       // PV K-chunks
  const int8_t *qkv = g.qkv + (size_t)row0 * 576;

  for (int i = tid; i < n16 * 16 * 4; i += 256) {
    const int r = i >> 2, c = (i & 3) * 16;
    v4i v = v4i{0};
    if (r < N) v = *reinterpret_cast<const v4i *>(qkv + (size_t)r * 576 + 192 + h * 64 + c);
    *reinterpret_cast<v4i *>(&Ks[r * kKStride + c]) = v;
  }
  for (int i = tid; i < n64 * 64 * 4; i += 256) {
    const int r = i >> 2, c = (i & 3) * 16;
    v4i v = v4i{0};
    if (r < N) v = *reinterpret_cast<const v4i *>(qkv + (size_t)r * 576 + 384 + h * 64 + c);
    const int8_t *vb = reinterpret_cast<const int8_t *>(&v);
#pragma unroll
    for (int j = 0; j < 16; ++j) Vt[(c + j) * kVStride + r] = vb[j];
  }
  __syncthreads();
  if (tid < 64) {
    int s = 0;
    for (int r = 0; r < N; ++r) s += Vt[tid * kVStride + r];
    colsum[tid] = s;
  }
  __syncthreads();

  int8_t *P = &Ps[wave * 16 * kPStride];
  const int kgrp = (lane >> 4) * 16;  // this lane's 16-byte K fragment
  for (int qt = wave; qt < n16; qt += 4) {
    const int qrow = qt * 16 + (lane & 15);
    v4i qa = v4i{0};
    if (qrow < N) qa = *reinterpret_cast<const v4i *>(qkv + (size_t)qrow * 576 + h * 64 + kgrp);
    // S tiles: lane holds column kt*16 + lane%16 of rows 4*(lane/16) + i.
    int q16[13][4];
    int mx[4] = {-(1 << 30), -(1 << 30), -(1 << 30), -(1 << 30)};
#pragma unroll
    for (int kt = 0; kt < 13; ++kt) {
      if (kt < n16) {
        const v4i kb = *reinterpret_cast<const v4i *>(&Ks[(kt * 16 + (lane & 15)) * kKStride + kgrp]);
        const v4i s = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa, kb, v4i{0}, 0, 0, 0);
        const int col = kt * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = qt * 16 + 4 * (lane >> 4) + i;
          const i64 score = requant_shift(s[i], g.score_shift, 32);
          const int q = (int)requant_shift(score, g.q16_shift, 24);
          q16[kt][i] = q;
          if (col < N) {
            mx[i] = q > mx[i] ? q : mx[i];
            if (g.score && r < N)
              g.score[(((size_t)b * 3 + h) * 197 + r) * 197 + col] = (int32_t)score;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const int o = __shfl_xor(mx[i], off);
        mx[i] = o > mx[i] ? o : mx[i];
      }
    unsigned sum[4] = {0, 0, 0, 0};
#pragma unroll
    for (int kt = 0; kt < 13; ++kt) {
      if (kt < n16) {
        const int col = kt * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const unsigned e = col < N ? softmax_exp(q16[kt][i] - mx[i]) : 0u;
          q16[kt][i] = (int)e;
          sum[i] += e;
        }
      }
    }
    u64 recip[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) sum[i] += __shfl_xor(sum[i], off);
      recip[i] = softmax_recip(sum[i]);
    }
#pragma unroll
    for (int kt = 0; kt < 13; ++kt) {
      if (kt < n16) {
        const int col = kt * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rl = 4 * (lane >> 4) + i;
          const unsigned p = col < N ? prob_u8(softmax_ratio((unsigned)q16[kt][i], recip[i])) : 0u;
          P[rl * kPStride + col] = (int8_t)((int)p - 128);
          const int r = qt * 16 + rl;
          if (g.prob && r < N && col < N)
            g.prob[(((size_t)b * 3 + h) * 197 + r) * 197 + col] = (uint8_t)p;
        }
      }
    }
    // LDS accesses of one wavefront complete in order; the wait plus the
    // compiler barrier keep the P reads below after the writes above.
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      v4i acc = v4i{0};
      for (int kc = 0; kc < n64; ++kc) {
        const v4i pa = *reinterpret_cast<const v4i *>(&P[(lane & 15) * kPStride + kc * 64 + kgrp]);
        const v4i vb = *reinterpret_cast<const v4i *>(&Vt[(dt * 16 + (lane & 15)) * kVStride + kc * 64 + kgrp]);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb, acc, 0, 0, 0);
      }
      const int d = dt * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = qt * 16 + 4 * (lane >> 4) + i;
        if (r < N) {
          const i64 v = (i64)acc[i] + 128ll * colsum[d];
          g.ctx[(size_t)(row0 + r) * 192 + h * 64 + d] = (int8_t)requant_shift(v, g.ctx_shift, 8);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

int launch_attention(const AttnArgs &a, hipStream_t s) {
  if (a.batch <= 0) return HV_OK;
  hipLaunchKernelGGL(k_attention, dim3(a.batch * 3), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "k_attention launch");
}

// ---------------------------------------------------------------------------
// Softmax over ragged rows (nonlinear.softmax_scaled / _attention /
// _selector, nonlinear.py:109-133): one wavefront per row, <= 256 entries.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_softmax_rows(const int32_t *x, const int32_t *offsets,
                                                     uint8_t *att, int32_t *sel) {
  const int row = blockIdx.x, lane = threadIdx.x;
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
  const u64 recip = softmax_recip(sum);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    if (c < n) {
      const unsigned ratio = softmax_ratio(e[j], recip);
      att[o + c] = (uint8_t)prob_u8(ratio);
      sel[o + c] = (int32_t)(ratio > 65536u ? 65536u : ratio);
    }
  }
}

int launch_softmax_rows(const int32_t *x, const int32_t *offsets, int rows, uint8_t *att,
                        int32_t *sel, hipStream_t s) {
  if (rows <= 0) return HV_OK;
  hipLaunchKernelGGL(k_softmax_rows, dim3(rows), dim3(64), 0, s, x, offsets, att, sel);
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
  if (op < 0 || op > HV_PRIM_RSA) return fail(HV_EVALUE, "unknown primitive %d", op);
  if (op == HV_PRIM_REQUANT && (c < 2 || c > 63))
    return fail(HV_EVALUE, "requant bits must be in [2, 63]");
  if (n <= 0) return HV_OK;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return fail(HV_EVALUE, "too many elements");
  hipLaunchKernelGGL(k_primitive, dim3((unsigned)blocks), dim3(256), 0, s, op, in, out, n, a, b,
                     c);
  return check_hip(hipGetLastError(), "k_primitive launch");
}

}  // namespace hv
