// hv_selector.hip -- token selector (selector.token_selector,
// selector.py:503-563) over a ragged batch.
//
// k_selector_head, one workgroup per (image, head): local MLP + head
//   statistic (:253, :358), candidate mean (:273), concat + 64->32->16->2
//   score MLP + 2-way selector softmax (:292, :307, :338).  The MLP layers
//   run as int8 MFMAs over tiles of 16 candidates with the weights and
//   every intermediate in LDS; head scores and statistics go to a
//   workspace.
// k_selector_keep, one wavefront per image: head-weight MLP with PLAN
//   (:370) and the head fuse (:392) per candidate (skipped when the fused
//   scores are given), then the stable keep list (fused >= 32768) and the
//   per-image state of finalize_tokens (:456-500).
// k_selector_compact: finalize_tokens (:421-500) as stream compaction:
//   each image's output offset is the prefix sum of the counts of earlier
//   images; CLS, the kept rows in input order and the package row
//   (score-weighted mean of pruned normals plus the incoming package, or
//   their plain mean when the scores sum to zero) are written there.
//
// GELU layers use the int32 requant/GELU path when the host finds every
// shift in [-30, 30] and each layer's biases satisfy |b| <= 2^30 - 1 -
// K*2^14 (checked per workgroup, uniform); otherwise the exact 64-bit form.
#include <type_traits>

#include "hv_device.h"
#include "hv_internal.h"
#include "gelu_lut.inc"  // generated at build time by gen_gelu_lut.py

namespace hv {

// A GELU layer's step table (gen_gelu_lut.py) when its output shift has one:
// words [off, off + words) of kGeluLut, clamp [qlo, qhi], cb as gelu_table
// takes it; off < 0: the layer evaluates ShiftGELU.
struct SelLut {
  int off, words, qlo, qhi, cb;
};

// Copies a step table into LDS with 16-byte loads, four rounds in flight
// (tables start on 16-byte boundaries and hold a multiple of four words).
// All kHeadThreads threads call it; the caller puts a barrier after it.
__device__ __forceinline__ void sel_stage_lut(const SelLut &t, unsigned *lut, int tid) {
  const v4i *src = reinterpret_cast<const v4i *>(kGeluLut + t.off);
  v4i *dst = reinterpret_cast<v4i *>(lut);
  const int n4 = t.words >> 2;
  for (int base = tid; base < n4; base += 4 * 256) {
    v4i v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = src[min(base + r * 256, n4 - 1)];
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[min(base + r * 256, n4 - 1)] = v[r];
  }
}

static constexpr int kMaxCand = 196;

__device__ __forceinline__ int dot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

__device__ __noinline__ int gelu_exact(int acc, int bias, int sh_in, int sh_out) {
  return gelu_post((i64)acc + bias, sh_in, sh_out);
}

// requant(gelu(requant(acc + bias, src, -16, 24)), -16, dst, 8).
__device__ __forceinline__ int sel_gelu(int acc, int bias, bool fast, const Rq &ra, const Rq &rb,
                                        int sh_in, int sh_out) {
  if (fast) return rq(gelu_q16(rq(acc + bias, ra)), rb);
  return gelu_exact(acc, bias, sh_in, sh_out);
}


// The same with a 64-bit bias (score layer 1 after its global half is
// folded into the bias, below).
__device__ __noinline__ int gelu_exact64(int acc, i64 bias, int sh_in, int sh_out) {
  return gelu_post((i64)acc + bias, sh_in, sh_out);
}

constexpr int kHeadThreads = 256;
constexpr int kCandTiles = (kMaxCand + 15) / 16;  // 13 tiles of 16 candidates
constexpr int kCandPad = kCandTiles * 16;

// One workgroup per (image, head).  The three MLP layers run as int8 MFMAs
// over tiles of 16 candidates, with the weights (output-major, as stored)
// and every intermediate in LDS:
//   local = GELU(x_h [C][64] . Wl [64][32] + bl)          16x16x64, 2 column tiles
//   h1    = GELU(local . W1[0:32] + b1')                  16x16x32, 2 column tiles
//   h2    = GELU(h1 . W2 + b2)                            16x16x32, 1 column tile
// where b1' = b1 + global . W1[32:64] (the global feature is the same for
// every candidate, so the concat's second half is a per-head bias, exact in
// 64 bits).  Result lane l of a tile holds output channel 16 ct + l % 16 of
// candidates 4 (l / 16) + i.  The logits (16 -> 2), the 2-way softmax and
// the lane mean of the head slice (the head statistic) are per candidate.
// The GELU layers with a step table for their output shift read it from
// LDS (staged per layer: local, h1, h2) instead of evaluating ShiftGELU.
__global__ __launch_bounds__(kHeadThreads) void k_selector_head(
    hv_selector_dev p, const int8_t *tokens, const int32_t *offsets, int batch,
    const uint8_t *pkg_in, int32_t *hs_out, int8_t *stats_out, int fast_shifts,
    hv_selector_ckpt ck, SelLut tl, SelLut t1, SelLut t2) {
  static_assert(kHeadThreads == 256, "sel_stage_lut strides");
  __shared__ __attribute__((aligned(16))) unsigned lut[kGeluLutMaxWords];
  __shared__ __attribute__((aligned(16))) int8_t wl[32 * 64];   // local_wt[h] [32][64]
  __shared__ __attribute__((aligned(16))) int8_t w1[32 * 64];   // w1t[h] [32][64]
  __shared__ __attribute__((aligned(16))) int8_t w2[16 * 32];   // w2t[h] [16][32]
  __shared__ int w3[2 * 4];                                     // w3t[h] [2][16] as words
  __shared__ int bl[32], bb2[16];
  __shared__ i64 bb1[32];                                       // b1 + global . W1[32:64]
  __shared__ __attribute__((aligned(16))) int8_t local_s[kCandPad * 32];
  __shared__ __attribute__((aligned(16))) int8_t h1_s[kCandPad * 32];
  __shared__ __attribute__((aligned(16))) int8_t h2_s[kCandPad * 16];
  __shared__ int part[8 * 32];
  __shared__ int glob_s[32];
  __shared__ int fast_s[3];

  // The grid is a multiple of 8 and workgroups go round-robin over the 8
  // XCDs, so XCD x runs logical items [x*T8, (x+1)*T8): the three heads of
  // an image share one XCD's L2.
  const int T = 3 * batch, T8 = (T + 7) >> 3;
  const int L = (blockIdx.x & 7) * T8 + (blockIdx.x >> 3);
  if (L >= T) return;
  const int b = L / 3, h = L - 3 * b, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, col = lane & 15, grp = lane >> 4;
  const int row0 = offsets[b], N = offsets[b + 1] - row0, C = N - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  if (C < 1 || C > kMaxCand || C - pkg < 1 || row0 < 0) return;  // k_selector_keep reports
  const int ntiles = (C + 15) >> 4;

  {
    const v4i *src = reinterpret_cast<const v4i *>(p.local_wt + h * 2048);
    if (tid < 128) reinterpret_cast<v4i *>(wl)[tid] = src[tid];
    src = reinterpret_cast<const v4i *>(p.w1t + h * 2048);
    if (tid >= 128) reinterpret_cast<v4i *>(w1)[tid - 128] = src[tid - 128];
    src = reinterpret_cast<const v4i *>(p.w2t + h * 512);
    if (tid < 32) reinterpret_cast<v4i *>(w2)[tid] = src[tid];
    if (tid >= 64 && tid < 72) w3[tid - 64] = reinterpret_cast<const int *>(p.w3t)[h * 8 + tid - 64];
    if (tid >= 96 && tid < 128) bl[tid - 96] = p.local_b[h * 32 + tid - 96];
    if (tid >= 160 && tid < 176) bb2[tid - 160] = p.b2[h * 16 + tid - 160];
  }
  if (tl.off >= 0) sel_stage_lut(tl, lut, tid);
  __syncthreads();
  // int32 GELU preconditions: |acc| <= K*2^14 for the layer's K.
  const int lim64 = (1 << 30) - 1 - 64 * 16384, lim32 = (1 << 30) - 1 - 32 * 16384;
  if (tid < 2) {
    bool f = fast_shifts != 0;
    if (tid == 0)
      for (int j = 0; j < 32; ++j) f = f && bl[j] <= lim64 && bl[j] >= -lim64;
    else
      for (int j = 0; j < 16; ++j) f = f && bb2[j] <= lim32 && bb2[j] >= -lim32;
    fast_s[tid == 0 ? 0 : 2] = f;
  }

  const int8_t *cand = tokens + (size_t)(row0 + 1) * 192 + h * 64;
  // Local MLP and head statistic.
  {
    const int sh_in = -16 - (p.in_exp + p.local_w_exp), sh_out = p.local_out_exp + 16;
    const Rq ra = rq_setup(sh_in, -(1 << 23), (1 << 23) - 1), rb = rq_setup(sh_out, -128, 127);
    __syncthreads();
    const bool fast = fast_s[0];
    // two tiles per round: both candidate loads in flight, then the eight
    // table lookups staged together
    const int nt = ntiles * 2;
    for (int t0 = wave; t0 < nt; t0 += 8) {
      v4i a[2], acc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tv = min(t0 + 4 * u, nt - 1);
        const int c = min((tv >> 1) * 16 + col, C - 1);
        a[u] = *reinterpret_cast<const v4i *>(cand + (size_t)c * 192 + grp * 16);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tv = min(t0 + 4 * u, nt - 1), ct = tv & 1;
        const v4i wb = *reinterpret_cast<const v4i *>(&wl[(ct * 16 + col) * 64 + grp * 16]);
        acc[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], wb, v4i{0}, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = t0 + 4 * u, rt = t >> 1, ct = t & 1;
        if (t < nt && ct == 0) {
          // lane mean of the candidate's 64 head lanes (selector.py:358-367)
          int sum = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) sum = dot4(a[u][k], 0x01010101, sum);
          sum += __shfl_xor(sum, 16);
          sum += __shfl_xor(sum, 32);
          if (grp == 0 && rt * 16 + col < C) {
            const int8_t stat = (int8_t)sat_bits(round_div_pos(sum, 64), 8);
            const int cc = rt * 16 + col;
            stats_out[((size_t)b * kMaxCand + cc) * 3 + h] = stat;
            if (ck.head_stats) ck.head_stats[((size_t)b * kMaxCand + cc) * 3 + h] = stat;
          }
        }
      }
      if (fast && tl.off >= 0) {
        int qv[8];
        unsigned ov[8];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int j = ((t0 + 4 * u) & 1) * 16 + col;
#pragma unroll
          for (int i = 0; i < 4; ++i) qv[4 * u + i] = rq(acc[u][i] + bl[j], ra);
        }
        gelu_table_u8_n<8>(qv, ov, lut, tl.cb, tl.qlo, tl.qhi);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t = t0 + 4 * u, rt = t >> 1, j = (t & 1) * 16 + col;
          if (t < nt) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              local_s[(rt * 16 + grp * 4 + i) * 32 + j] = (int8_t)ov[4 * u + i];
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t = t0 + 4 * u, rt = t >> 1, j = (t & 1) * 16 + col;
          if (t < nt) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              local_s[(rt * 16 + grp * 4 + i) * 32 + j] =
                  (int8_t)sel_gelu(acc[u][i], bl[j], fast, ra, rb, sh_in, sh_out);
          }
        }
      }
    }
  }
  __syncthreads();
  // score layer 1's table replaces the local layer's (barriers follow)
  if (t1.off >= 0) sel_stage_lut(t1, lut, tid);
  // Global feature = sat8(round_div(sum_c local, C)) and the folded bias of
  // score layer 1.
  {
    const int ch = tid & 31, prt = tid >> 5;
    int sacc = 0;
    for (int c = prt; c < C; c += 8) sacc += local_s[c * 32 + ch];
    part[prt * 32 + ch] = sacc;
  }
  __syncthreads();
  if (tid < 32) {
    int sacc = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) sacc += part[q * 32 + tid];
    const int gv = (int)sat_bits(round_div_pos(sacc, C), 8);
    glob_s[tid] = gv;
    if (ck.global) ck.global[((size_t)b * 3 + h) * 32 + tid] = (int8_t)gv;
  }
  __syncthreads();
  if (tid < 32) {
    i64 v = p.b1[h * 32 + tid];
#pragma unroll 8
    for (int k = 0; k < 32; ++k) v += (i64)glob_s[k] * w1[tid * 64 + 32 + k];
    bb1[tid] = v;
  }
  __syncthreads();
  if (tid == 0) {
    bool f = fast_shifts != 0;
    for (int j = 0; j < 32; ++j) f = f && bb1[j] <= lim32 && bb1[j] >= -lim32;
    fast_s[1] = f;
  }
  // Score layer 1 (local half).
  {
    const int sh_in = -16 - (p.concat_out_exp + p.score_w1_exp), sh_out = p.h1_out_exp + 16;
    const Rq ra = rq_setup(sh_in, -(1 << 23), (1 << 23) - 1), rb = rq_setup(sh_out, -128, 127);
    __syncthreads();
    const bool fast = fast_s[1];
    for (int t = wave; t < ntiles * 2; t += 4) {
      const int rt = t >> 1, ct = t & 1;
      const long a = *reinterpret_cast<const long *>(&local_s[(rt * 16 + col) * 32 + grp * 8]);
      const long wb = *reinterpret_cast<const long *>(&w1[(ct * 16 + col) * 64 + grp * 8]);
      const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, wb, v4i{0}, 0, 0, 0);
      const int j = ct * 16 + col;
      const i64 bias = bb1[j];
      if (fast && t1.off >= 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          h1_s[(rt * 16 + grp * 4 + i) * 32 + j] =
              (int8_t)gelu_table_u8(rq(acc[i] + (int)bias, ra), lut, t1.cb, t1.qlo, t1.qhi);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = fast ? rq(gelu_q16(rq(acc[i] + (int)bias, ra)), rb)
                             : gelu_exact64(acc[i], bias, sh_in, sh_out);
          h1_s[(rt * 16 + grp * 4 + i) * 32 + j] = (int8_t)v;
        }
      }
    }
  }
  __syncthreads();
  if (t2.off >= 0) {  // score layer 2's table
    sel_stage_lut(t2, lut, tid);
    __syncthreads();
  }
  // Score layer 2.
  {
    const int sh_in = -16 - (p.h1_out_exp + p.score_w2_exp), sh_out = p.h2_out_exp + 16;
    const Rq ra = rq_setup(sh_in, -(1 << 23), (1 << 23) - 1), rb = rq_setup(sh_out, -128, 127);
    const bool fast = fast_s[2];
    for (int rt = wave; rt < ntiles; rt += 4) {
      const long a = *reinterpret_cast<const long *>(&h1_s[(rt * 16 + col) * 32 + grp * 8]);
      const long wb = *reinterpret_cast<const long *>(&w2[col * 32 + grp * 8]);
      const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, wb, v4i{0}, 0, 0, 0);
      if (fast && t2.off >= 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          h2_s[(rt * 16 + grp * 4 + i) * 16 + col] =
              (int8_t)gelu_table_u8(rq(acc[i] + bb2[col], ra), lut, t2.cb, t2.qlo, t2.qhi);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          h2_s[(rt * 16 + grp * 4 + i) * 16 + col] =
              (int8_t)sel_gelu(acc[i], bb2[col], fast, ra, rb, sh_in, sh_out);
      }
    }
  }
  __syncthreads();
  // Logits, the 2-way selector softmax (keep = element 1) and checkpoints.
  {
    const int s3 = p.logits_out_exp - (p.h2_out_exp + p.score_w3_exp);
    const int sq = -16 - p.logits_out_exp;
    for (int c = tid; c < C; c += kHeadThreads) {
      const v4i hv = *reinterpret_cast<const v4i *>(&h2_s[c * 16]);
      int qv[2];
#pragma unroll
      for (int lj = 0; lj < 2; ++lj) {
        int acc = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = dot4(hv[k], w3[lj * 4 + k], acc);
        const int logit = (int)requant_shift((i64)acc + p.b3[h * 2 + lj], s3, 8);
        qv[lj] = (int)requant_shift(logit, sq, 24);
      }
      const int mx = qv[0] > qv[1] ? qv[0] : qv[1];
      const unsigned e0 = softmax_exp(qv[0] - mx), e1 = softmax_exp(qv[1] - mx);
      const unsigned ratio = softmax_ratio(e1, softmax_recip24(e0 + e1));
      const int hsv = (int)(ratio > 65536u ? 65536u : ratio);
      hs_out[((size_t)b * 3 + h) * kMaxCand + c] = hsv;
      if (ck.head_scores) ck.head_scores[((size_t)b * 3 + h) * kMaxCand + c] = hsv;
      if (ck.h2)
        *reinterpret_cast<v4i *>(ck.h2 + (((size_t)b * 3 + h) * kMaxCand + c) * 16) = hv;
    }
    if (ck.local) {
      int8_t *dst = ck.local + ((size_t)b * 3 + h) * kMaxCand * 32;
      for (int i = tid; i < C * 2; i += kHeadThreads)
        reinterpret_cast<v4i *>(dst)[i] = reinterpret_cast<const v4i *>(local_s)[i];
    }
  }
}

// Head fuse of one candidate (selector.py:370-418): head-weight MLP (3->3
// GELU, 3->3 PLAN) on the head statistics and the weighted mean of the head
// scores; *warn is set when the weights sum to zero (plain mean then).
__device__ int fuse_candidate(const hv_selector_dev &p, const int8_t *stats, const int32_t *hs,
                              int C, int c, int32_t *weights_out, bool *warn) {
  const int a_in = -16 - (p.stats_out_exp + p.hw_w1_exp), a_out = p.hw_hidden_out_exp + 16;
  const int b_sh = -16 - (p.hw_hidden_out_exp + p.hw_w2_exp);
  int hid[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    // The bias is any int32 and the reference adds it in int64
    // (gemm.py:118-119): the three products (|sum| < 2^16) are summed in
    // 32 bits and the bias added in 64.  The empty asm keeps the compiler
    // from folding bias and products into one 32-bit dot-product
    // accumulation, which wraps for biases near the int32 limits.
    int dot = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) dot += (int)stats[k] * (int)p.hw_w1t[j * 3 + k];
    asm volatile("" : "+v"(dot));
    hid[j] = gelu_post((i64)p.hw_b1[j] + dot, a_in, a_out);
  }
  i64 num = 0, den = 0;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    int dot = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) dot += hid[k] * (int)p.hw_w2t[j * 3 + k];
    asm volatile("" : "+v"(dot));
    const i64 acc = (i64)p.hw_b2[j] + dot;
    const int w = sat_q016(plan_sigmoid((int)requant_shift(acc, b_sh, 24)));
    if (weights_out) weights_out[j] = w;
    num += (i64)hs[j * kMaxCand] * w;
    den += w;
  }
  *warn = den == 0;
  if (den == 0) {
    num = (i64)hs[0] + hs[kMaxCand] + hs[2 * kMaxCand];
    den = 3;
  }
  return sat_q016(round_div_pos(num, den));
}

// Optional head fuse, then the stable keep list of the normal candidates
// (fused >= 32768, input order) and the per-image state {token_count,
// package_present, kept, pruned, warnings} (selector.py:456-500).  One
// workgroup per image, one thread per candidate (at most 196).
__global__ __launch_bounds__(256) void k_selector_keep(const int32_t *offsets,
                                                       const uint8_t *pkg_in, int32_t *fused,
                                                       int32_t *kept_index, int32_t *state,
                                                       hv_selector_dev p, const int32_t *hs,
                                                       const int8_t *stats, int32_t *weights_ck,
                                                       int32_t *img_warn) {
  __shared__ int w_kept[4], w_warn[4], w_bad[4];
  __shared__ i64 w_den[4];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = offsets[b + 1] - offsets[b] - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  int32_t *st = state + (size_t)b * 5;
  if (C < 1 || C > kMaxCand || C - pkg < 1 || offsets[b] < 0) {
    // token_selector needs CLS plus one candidate (selector.py:513-514) and
    // an incoming package needs a normal candidate beside it (:448-449);
    // the state's token count -1 reports the ValueError.
    if (tid == 0) { st[0] = -1; st[1] = 0; st[2] = 0; st[3] = 0; st[4] = 0; }
    return;
  }
  int32_t *f = fused + (size_t)b * kMaxCand;
  const int n_norm = C - pkg;
  const int c = tid;
  const bool in = c < C;
  int fc = 0;
  bool warn = false, bad = false;
  if (hs) {
    if (in) {
      fc = fuse_candidate(p, stats + ((size_t)b * kMaxCand + c) * 3,
                          hs + (size_t)b * 3 * kMaxCand + c, C, c,
                          weights_ck ? weights_ck + ((size_t)b * kMaxCand + c) * 3 : nullptr,
                          &warn);
      f[c] = fc;
    }
  } else {
    // Given scores must be Q0.16 values in [0, 65536] (selector._q016): an
    // image holding any other value is rejected like a bad token count.
    fc = in ? f[c] : 0;
    bad = in && (unsigned)fc > 65536u;
  }
  const bool is_norm = c < n_norm;
  const bool keep = is_norm && fc >= 32768;
  const bool part = (is_norm && !keep) || (pkg && c == C - 1);
  const u64 mask = __ballot(keep);
  i64 d = part ? fc : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off);
  const bool warn_wave = __ballot(warn) != 0;
  if (lane == 0) {
    w_kept[wave] = __popcll(mask);
    w_den[wave] = d;
    w_warn[wave] = warn_wave;
  }
  const bool bad_wave = __ballot(bad) != 0;
  if (lane == 0) w_bad[wave] = bad_wave;
  __syncthreads();
  if (w_bad[0] | w_bad[1] | w_bad[2] | w_bad[3]) {
    if (tid == 0) { st[0] = -1; st[1] = 0; st[2] = 0; st[3] = 0; st[4] = 0; }
    return;
  }
  int before = __popcll(mask & ((1ull << lane) - 1ull)), kept = 0;
  i64 den = 0;
  bool warn_head = false;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    before += w < wave ? w_kept[w] : 0;
    kept += w_kept[w];
    den += w_den[w];
    warn_head = warn_head || w_warn[w];
  }
  int32_t *ki = kept_index + (size_t)b * kMaxCand;
  if (keep) ki[before] = c;
  if (c >= kept && c < kMaxCand) ki[c] = -1;
  if (tid == 0) {
    const int n_part = C - kept;  // pruned normals + the incoming package
    const int exists = n_part > 0;
    st[0] = 1 + kept + exists;
    st[1] = exists;
    st[2] = kept;
    st[3] = n_part - pkg;
    const int warn_bits = (warn_head ? HV_WARN_HEAD_DEN_ZERO : 0) |
                          ((exists && den == 0) ? HV_WARN_PACKAGE_DEN_ZERO : 0);
    st[4] = warn_bits;
    if (img_warn) img_warn[b] |= warn_bits;
  }
}

__global__ __launch_bounds__(256) void k_selector_compact(
    const int8_t *tokens, const int32_t *offsets, const uint8_t *pkg_in, int batch,
    const int32_t *fused, const int32_t *kept_index, const int32_t *state, int8_t *out,
    int32_t *out_offsets, uint8_t *pkg_out, int32_t *token_counts, int stage) {
  __shared__ int red[4];
  __shared__ i64 den_part[4];
  __shared__ int wgt[kMaxCand];
  __shared__ int part_sum[21 * 192];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t *st = state + (size_t)b * 5;
  const int count = st[0], exists = st[1], kept = st[2];
  const int row0 = offsets[b], C = offsets[b + 1] - row0 - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  // Source row of output row r is row0 + 1 + src_k[r]: -1 for the CLS row,
  // then the kept candidates.
  __shared__ int src_k[kMaxCand + 1];
  const int *ki = kept_index + (size_t)b * kMaxCand;
  if (tid <= kMaxCand) src_k[tid] = tid == 0 ? -1 : ki[tid - 1];
  // Output row of this image: the token counts of the images before it.
  int s = 0;
  for (int i = tid; i < b; i += 256) s += max(state[(size_t)i * 5], 0);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const int out0 = red[0] + red[1] + red[2] + red[3];
  if (tid == 0) {
    out_offsets[b] = out0;
    if (b == batch - 1) out_offsets[batch] = out0 + (count > 0 ? count : 0);
    pkg_out[b] = (uint8_t)exists;
    if (token_counts) token_counts[(size_t)b * 4 + stage] = count;
  }
  if (count <= 0) return;
  // CLS and kept rows, 16 bytes per item; four items per thread in flight
  // (items past the end repeat the last one, so no copy is predicated).
  const int n_items = (1 + kept) * 12;
  for (int base = tid; base < n_items; base += 1024) {
    v4i v[4];
    int dst[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = min(base + j * 256, n_items - 1), r = i / 12, chunk = i - r * 12;
      v[j] = reinterpret_cast<const v4i *>(tokens + (size_t)(row0 + 1 + src_k[r]) * 192)[chunk];
      dst[j] = (out0 + r) * 12 + chunk;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) reinterpret_cast<v4i *>(out)[dst[j]] = v[j];
  }
  if (!exists) return;
  // Package row: num[ch] = sum over partitioned candidates of w_c * x_c[ch]
  // with w_c = fused score (or 1 when the scores sum to zero).  |num| <=
  // 196 * 65536 * 128 < 2^31.  Thread (channel group of 16, candidate
  // group g) accumulates candidates g, g + 21, ... (all of its candidate
  // rows loaded at once, weight 0 for kept ones); LDS sums the groups.
  constexpr int kSteps = (kMaxCand + 20) / 21;
  const int cg = tid / 12, chg = tid - cg * 12;
  v4i xv[kSteps];
  if (tid < 12 * 21) {
    const int8_t *cand = tokens + (size_t)(row0 + 1) * 192 + chg * 16;
#pragma unroll
    for (int j = 0; j < kSteps; ++j)
      xv[j] = *reinterpret_cast<const v4i *>(cand + (size_t)min(cg + 21 * j, C - 1) * 192);
  }
  const int32_t *f = fused + (size_t)b * kMaxCand;
  const int n_norm = C - pkg;
  int fv = 0;
  bool part = false;
  if (tid < C) {
    fv = f[tid];
    part = (tid < n_norm && fv < 32768) || (pkg && tid == C - 1);
  }
  i64 d = part ? fv : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off);
  if (lane == 0) den_part[wave] = d;
  __syncthreads();
  const i64 den = den_part[0] + den_part[1] + den_part[2] + den_part[3];
  if (tid < C) wgt[tid] = part ? (den == 0 ? 1 : fv) : 0;
  __syncthreads();
  if (tid < 12 * 21) {
    int acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0;
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const int c = cg + 21 * j;
      const int w = c < C ? wgt[c] : 0;
#pragma unroll
      for (int k = 0; k < 16; ++k) acc[k] += w * (int)(int8_t)(xv[j][k >> 2] >> (8 * (k & 3)));
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) part_sum[cg * 192 + chg * 16 + j] = acc[j];
  }
  __syncthreads();
  const int n_part = C - kept;
  if (tid < 192) {
    int num = 0;
#pragma unroll
    for (int g = 0; g < 21; ++g) num += part_sum[g * 192 + tid];
    out[(size_t)(out0 + 1 + kept) * 192 + tid] =
        (int8_t)sat_bits(round_div_pos(num, den == 0 ? n_part : den), 8);
  }
}

int launch_selector(const SelectorArgs &a, hipStream_t s) {
  if (a.batch <= 0) return HV_OK;
  int rc = HV_OK;
  hv_selector_dev p{};
  if (a.p) {
    if (!a.hs || !a.stats) return fail(HV_EVALUE, HV_ERR_ADDRESS, "selector: missing workspace");
    p = *a.p;
    auto in = [](int v) { return v >= -30 && v <= 30; };
    const int fast = in(-16 - (p.in_exp + p.local_w_exp)) && in(p.local_out_exp + 16) &&
                     in(-16 - (p.concat_out_exp + p.score_w1_exp)) && in(p.h1_out_exp + 16) &&
                     in(-16 - (p.h1_out_exp + p.score_w2_exp)) && in(p.h2_out_exp + 16);
    auto table = [](int so) {
      if (so < kGeluLutSoMin || so > kGeluLutSoMax) return SelLut{-1, 0, 0, 0, 0};
      const GeluLutInfo &t = kGeluLutInfo[so - kGeluLutSoMin];
      return SelLut{t.off, t.words, t.qlo, t.qhi, -4 * (t.qlo >> kGeluCoarseShift)};
    };
    hv_launch(k_selector_head, dim3((a.batch * 3 + 7) / 8 * 8), dim3(kHeadThreads), 0, s, p,
              a.tokens, a.offsets, a.batch, a.pkg_in, a.hs, a.stats, fast, a.ck,
              table(p.local_out_exp + 16), table(p.h1_out_exp + 16), table(p.h2_out_exp + 16));
    if ((rc = check_hip(hipGetLastError(), "k_selector_head launch"))) return rc;
  }
  hv_launch(k_selector_keep, dim3(a.batch), dim3(256), 0, s, a.offsets, a.pkg_in,
                     a.fused, a.kept_index, a.state, p, a.p ? a.hs : nullptr,
                     a.p ? a.stats : nullptr, a.p ? a.ck.head_weights : nullptr, a.img_warn);
  if ((rc = check_hip(hipGetLastError(), "k_selector_keep launch"))) return rc;
  hv_launch(k_selector_compact, dim3(a.batch), dim3(256), 0, s, a.tokens, a.offsets,
                     a.pkg_in, a.batch, a.fused, a.kept_index, a.state, a.out_tokens,
                     a.out_offsets, a.pkg_out, a.token_counts, a.stage);
  return check_hip(hipGetLastError(), "k_selector_compact launch");
}

}  // namespace hv
