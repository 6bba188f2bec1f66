// hv_selector.hip -- token selector (selector.token_selector,
// selector.py:503-563) over a ragged batch.
//
// k_selector_head, one workgroup per (image, head): local MLP + head
//   statistic (:253, :358), candidate mean (:273), concat + 64->32->16->2
//   score MLP + 2-way selector softmax (:292, :307, :338).  Two adjacent
//   lanes own one candidate, each computing half of every layer's outputs
//   and swapping halves by a lane shuffle; the tiny GEMMs (K = 64/32/16)
//   run on v_dot4_i32_i8 from LDS-held, output-major weights.  Head scores
//   and statistics go to a workspace.
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

namespace hv {

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

constexpr int kHeadThreads = 512;  // two lanes per candidate, kMaxCand <= 256

__global__ __launch_bounds__(kHeadThreads) void k_selector_head(hv_selector_dev p, const int8_t *tokens,
                                                       const int32_t *offsets, int batch,
                                                       const uint8_t *pkg_in, int32_t *hs_out,
                                                       int8_t *stats_out, int fast_shifts,
                                                       hv_selector_ckpt ck) {
  __shared__ int wl[32 * 16];   // local_wt[h] [32][64] as int words
  __shared__ int w1[32 * 16];   // w1t[h] [32][64]
  __shared__ int w2[16 * 8];    // w2t[h] [16][32]
  __shared__ int w3[2 * 4];     // w3t[h] [2][16]
  __shared__ int bl[32], bb1[32], bb2[16];
  __shared__ int local_s[kMaxCand * 8];  // [C][32] int8 as words
  __shared__ int glob[8];                 // [32] int8 as words
  __shared__ int hbuf[kHeadThreads];      // partial channel sums of the candidate mean

  // The grid is a multiple of 8 and workgroups go round-robin over the 8
  // XCDs, so XCD x runs logical items [x*T8, (x+1)*T8): the three heads of
  // an image share one XCD's L2.
  const int T = 3 * batch, T8 = (T + 7) >> 3;
  const int L = (blockIdx.x & 7) * T8 + (blockIdx.x >> 3);
  if (L >= T) return;
  const int b = L / 3, h = L - 3 * b, tid = threadIdx.x;
  const int row0 = offsets[b], N = offsets[b + 1] - row0, C = N - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  if (C < 1 || C > kMaxCand || C - pkg < 1 || row0 < 0) return;  // k_selector_keep reports

  {
    const int *src = reinterpret_cast<const int *>(p.local_wt) + h * 512;
    for (int i = tid; i < 512; i += kHeadThreads) wl[i] = src[i];
    src = reinterpret_cast<const int *>(p.w1t) + h * 512;
    for (int i = tid; i < 512; i += kHeadThreads) w1[i] = src[i];
    src = reinterpret_cast<const int *>(p.w2t) + h * 128;
    if (tid < 128) w2[tid] = src[tid];
    src = reinterpret_cast<const int *>(p.w3t) + h * 8;
    if (tid < 8) w3[tid] = src[tid];
    if (tid < 32) bl[tid] = p.local_b[h * 32 + tid];
    if (tid < 32) bb1[tid] = p.b1[h * 32 + tid];
    if (tid < 16) bb2[tid] = p.b2[h * 16 + tid];
  }
  __syncthreads();
  // int32 GELU preconditions: |acc| <= K*2^14 with K = 64 (32 for layer 2).
  bool fast = fast_shifts != 0;
  {
    const int lim64 = (1 << 30) - 1 - 64 * 16384, lim32 = (1 << 30) - 1 - 32 * 16384;
#pragma unroll 4
    for (int j = 0; j < 32; ++j)
      fast = fast && bl[j] <= lim64 && bl[j] >= -lim64 && bb1[j] <= lim64 && bb1[j] >= -lim64;
#pragma unroll 4
    for (int j = 0; j < 16; ++j) fast = fast && bb2[j] <= lim32 && bb2[j] >= -lim32;
  }

  const int8_t *cand = tokens + (size_t)(row0 + 1) * 192;
  // Stage 1: local MLP with GELU and the head lane mean.
  {
    const int sh_in = -16 - (p.in_exp + p.local_w_exp), sh_out = p.local_out_exp + 16;
    const Rq ra = rq_setup(sh_in, -(1 << 23), (1 << 23) - 1), rb = rq_setup(sh_out, -128, 127);
    // LPC lanes per candidate: four when the candidates fit (shorter
    // chains), else two.
    auto stage1 = [&](auto lpc) {
      constexpr int LPC = decltype(lpc)::value, WPL = 8 / LPC;  // output words per lane
      const int sub = tid & (LPC - 1);
      for (int c = tid / LPC; c < C; c += kHeadThreads / LPC) {
        int x[16];
        const v4i *src = reinterpret_cast<const v4i *>(cand + (size_t)c * 192 + h * 64);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const v4i v = src[k];
          x[4 * k] = v[0]; x[4 * k + 1] = v[1]; x[4 * k + 2] = v[2]; x[4 * k + 3] = v[3];
        }
        if (sub == 0) {
          int lane_sum = 0;
#pragma unroll
          for (int k = 0; k < 16; ++k) lane_sum = dot4(x[k], 0x01010101, lane_sum);
          const int8_t stat = (int8_t)sat_bits(round_div_pos(lane_sum, 64), 8);
          stats_out[((size_t)b * kMaxCand + c) * 3 + h] = stat;
          if (ck.head_stats) ck.head_stats[((size_t)b * kMaxCand + c) * 3 + h] = stat;
        }
#pragma unroll 1
        for (int jg = WPL * sub; jg < WPL * sub + WPL; ++jg) {
          int word = 0;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int j = jg * 4 + jj;
            int acc = 0;
            const int *w = &wl[j * 16];
#pragma unroll
            for (int k = 0; k < 16; ++k) acc = dot4(x[k], w[k], acc);
            const int v = sel_gelu(acc, bl[j], fast, ra, rb, sh_in, sh_out);
            word |= (v & 0xFF) << (8 * jj);
          }
          local_s[c * 8 + jg] = word;
          if (ck.local)
            reinterpret_cast<int *>(ck.local + (((size_t)b * 3 + h) * kMaxCand + c) * 32)[jg] = word;
        }
      }
    };
    if (C <= kHeadThreads / 4) stage1(std::integral_constant<int, 4>{});
    else stage1(std::integral_constant<int, 2>{});
  }
  __syncthreads();
  // Stage 2: global feature = sat8(round_div(sum_c local, C)); sixteen
  // partial sums per channel, then one thread per channel.
  {
    constexpr int kParts = kHeadThreads / 32;
    const int8_t *l8 = reinterpret_cast<const int8_t *>(local_s);
    const int ch = tid & 31, part = tid >> 5;
    int s = 0;
    for (int c = part; c < C; c += kParts) s += l8[c * 32 + ch];
    hbuf[tid] = s;
  }
  __syncthreads();
  if (tid < 32) {
    int s = 0;
#pragma unroll
    for (int part = 0; part < kHeadThreads / 32; ++part) s += hbuf[part * 32 + tid];
    const int8_t gv = (int8_t)sat_bits(round_div_pos(s, C), 8);
    reinterpret_cast<int8_t *>(glob)[tid] = gv;
    if (ck.global) ck.global[((size_t)b * 3 + h) * 32 + tid] = gv;
  }
  __syncthreads();
  // Stage 3: score MLP on [local | global] and the 2-way selector softmax.
  {
    const int s1_in = -16 - (p.concat_out_exp + p.score_w1_exp), s1_out = p.h1_out_exp + 16;
    const int s2_in = -16 - (p.h1_out_exp + p.score_w2_exp), s2_out = p.h2_out_exp + 16;
    const int s3 = p.logits_out_exp - (p.h2_out_exp + p.score_w3_exp);
    const int sq = -16 - p.logits_out_exp;
    const Rq r1a = rq_setup(s1_in, -(1 << 23), (1 << 23) - 1), r1b = rq_setup(s1_out, -128, 127);
    const Rq r2a = rq_setup(s2_in, -(1 << 23), (1 << 23) - 1), r2b = rq_setup(s2_out, -128, 127);
    auto stage3 = [&](auto lpc) {
      constexpr int LPC = decltype(lpc)::value;
      constexpr int W1 = 8 / LPC, W2 = 4 / LPC;  // layer-1 / layer-2 words per lane
      const int sub = tid & (LPC - 1), base = (tid & 63) & ~(LPC - 1);
      for (int c = tid / LPC; c < C; c += kHeadThreads / LPC) {
        int lg[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) lg[k] = local_s[c * 8 + k];
#pragma unroll
        for (int k = 0; k < 8; ++k) lg[8 + k] = glob[k];
        // layer 1: this lane's output words, the group's others by shuffle
        int mine[W1];
#pragma unroll 1
        for (int q = 0; q < W1; ++q) {
          int word = 0;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int j = (W1 * sub + q) * 4 + jj;
            int acc = 0;
            const int *w = &w1[j * 16];
#pragma unroll
            for (int k = 0; k < 16; ++k) acc = dot4(lg[k], w[k], acc);
            const int v = sel_gelu(acc, bb1[j], fast, r1a, r1b, s1_in, s1_out);
            word |= (v & 0xFF) << (8 * jj);
          }
          mine[q] = word;
        }
        int h1[8];
#pragma unroll
        for (int o = 0; o < LPC; ++o)
#pragma unroll
          for (int q = 0; q < W1; ++q) h1[o * W1 + q] = __shfl(mine[q], base + o);
        // layer 2
        int mine2[W2];
#pragma unroll 1
        for (int q = 0; q < W2; ++q) {
          int word = 0;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int j = (W2 * sub + q) * 4 + jj;
            int acc = 0;
            const int *w = &w2[j * 8];
#pragma unroll
            for (int k = 0; k < 8; ++k) acc = dot4(h1[k], w[k], acc);
            const int v = sel_gelu(acc, bb2[j], fast, r2a, r2b, s2_in, s2_out);
            word |= (v & 0xFF) << (8 * jj);
          }
          mine2[q] = word;
        }
        int h2[4];
#pragma unroll
        for (int o = 0; o < LPC; ++o)
#pragma unroll
          for (int q = 0; q < W2; ++q) h2[o * W2 + q] = __shfl(mine2[q], base + o);
        if (ck.h2 && sub == 0)
          *reinterpret_cast<v4i *>(ck.h2 + (((size_t)b * 3 + h) * kMaxCand + c) * 16) =
              v4i{h2[0], h2[1], h2[2], h2[3]};
        // layer 3: logit (sub & 1) here; the group's first two lanes hold both
        const int lj = sub & 1;
        int acc = 0;
        const int *w = &w3[lj * 4];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = dot4(h2[k], w[k], acc);
        const int logit = (int)requant_shift((i64)acc + p.b3[h * 2 + lj], s3, 8);
        const int qmine = (int)requant_shift(logit, sq, 24);
        int qv[2];
        qv[0] = __shfl(qmine, base);
        qv[1] = __shfl(qmine, base + 1);
        const int mx = qv[0] > qv[1] ? qv[0] : qv[1];
        const unsigned e0 = softmax_exp(qv[0] - mx), e1 = softmax_exp(qv[1] - mx);
        const unsigned ratio = softmax_ratio(e1, softmax_recip24(e0 + e1));
        const int hsv = (int)(ratio > 65536u ? 65536u : ratio);
        if (sub == 0) {
          hs_out[((size_t)b * 3 + h) * kMaxCand + c] = hsv;
          if (ck.head_scores) ck.head_scores[((size_t)b * 3 + h) * kMaxCand + c] = hsv;
        }
      }
    };
    if (C <= kHeadThreads / 4) stage3(std::integral_constant<int, 4>{});
    else stage3(std::integral_constant<int, 2>{});
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
    hv_launch(k_selector_head, dim3((a.batch * 3 + 7) / 8 * 8), dim3(kHeadThreads), 0, s, p,
              a.tokens, a.offsets, a.batch, a.pkg_in, a.hs, a.stats, fast, a.ck);
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
