// hv_selector.hip -- token selector (selector.token_selector,
// selector.py:503-563) over a ragged batch, one workgroup per image.
//
// k_selector_score: local MLP + head statistics (:253, :358), candidate mean
//   (:273), concat + 64->32->16->2 score MLP + 2-way selector softmax (:292,
//   :307, :338), head-weight MLP with PLAN (:370), head fuse (:392), then the
//   stable keep list (fused >= 32768) and the per-image state.  The tiny
//   per-candidate GEMMs (K = 64/32/16/3) run on v_dot4_i32_i8 from LDS-held,
//   output-major weights; one thread owns one (candidate, head) chain.
// k_selector_keep: the stable keep list and per-image state of
//   finalize_tokens (:456-500) from the fused scores.
// k_selector_compact: finalize_tokens (:421-500) as stream compaction:
//   each image's output offset is the prefix sum of the counts of earlier
//   images; CLS, the kept rows in input order and the package row
//   (score-weighted mean of pruned normals plus the incoming package, or
//   their plain mean when the scores sum to zero) are written there.
#include "hv_device.h"
#include "hv_internal.h"

namespace hv {

static constexpr int kMaxCand = 196;

__device__ __forceinline__ int dot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

__global__ __launch_bounds__(256) void k_selector_score(hv_selector_dev p, const int8_t *tokens,
                                                        const int32_t *offsets,
                                                        const uint8_t *pkg_in, int32_t *fused_out,
                                                        int32_t *kept_index, int32_t *state,
                                                        hv_selector_ckpt ck) {
  __shared__ int wl[3 * 32 * 16];   // local_wt [3][32][64] as int words
  __shared__ int w1[3 * 32 * 16];   // w1t [3][32][64]
  __shared__ int w2[3 * 16 * 8];    // w2t [3][16][32]
  __shared__ int w3[3 * 2 * 4];     // w3t [3][2][16]
  __shared__ int local_s[3 * kMaxCand * 8];  // [3][C][32] int8 as words
  __shared__ int glob[3 * 8];                 // [3][32] int8 as words
  __shared__ int8_t stats[kMaxCand * 3];
  __shared__ int hs[3 * kMaxCand];
  __shared__ int fused_s[kMaxCand];
  __shared__ int warn_head;

  const int b = blockIdx.x, tid = threadIdx.x;
  const int row0 = offsets[b], N = offsets[b + 1] - row0, C = N - 1;
  int32_t *st = state + (size_t)b * 5;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  if (C < 1 || C > kMaxCand || C - pkg < 1) {
    // token_selector needs CLS plus one candidate (selector.py:513-514) and
    // an incoming package needs a normal candidate beside it (:448-449);
    // the state's token count -1 reports the ValueError.
    if (tid == 0) { st[0] = -1; st[1] = 0; st[2] = 0; st[3] = 0; st[4] = 0; }
    return;
  }

  {
    const int *src = reinterpret_cast<const int *>(p.local_wt);
    for (int i = tid; i < 3 * 32 * 16; i += 256) wl[i] = src[i];
    src = reinterpret_cast<const int *>(p.w1t);
    for (int i = tid; i < 3 * 32 * 16; i += 256) w1[i] = src[i];
    src = reinterpret_cast<const int *>(p.w2t);
    for (int i = tid; i < 3 * 16 * 8; i += 256) w2[i] = src[i];
    src = reinterpret_cast<const int *>(p.w3t);
    if (tid < 24) w3[tid] = src[tid];
    if (tid == 0) warn_head = 0;
  }
  __syncthreads();

  const int8_t *cand = tokens + (size_t)(row0 + 1) * 192;
  // Stage 1: per (head, candidate): local MLP with GELU, and the head lane mean.
  {
    const int sh_in = -16 - (p.in_exp + p.local_w_exp), sh_out = p.local_out_exp + 16;
    for (int q = tid; q < 3 * C; q += 256) {
      const int h = q / C, c = q - h * C;
      int x[16];
      const v4i *src = reinterpret_cast<const v4i *>(cand + (size_t)c * 192 + h * 64);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const v4i v = src[k];
        x[4 * k] = v[0]; x[4 * k + 1] = v[1]; x[4 * k + 2] = v[2]; x[4 * k + 3] = v[3];
      }
      int lane_sum = 0;
#pragma unroll
      for (int k = 0; k < 16; ++k) lane_sum = dot4(x[k], 0x01010101, lane_sum);
      stats[c * 3 + h] = (int8_t)sat_bits(round_div_pos(lane_sum, 64), 8);
      if (ck.head_stats) ck.head_stats[((size_t)b * kMaxCand + c) * 3 + h] = stats[c * 3 + h];
      int packed[8];
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        int acc = 0;
        const int *w = &wl[(h * 32 + j) * 16];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = dot4(x[k], w[k], acc);
        const int v = gelu_post((i64)acc + p.local_b[h * 32 + j], sh_in, sh_out);
        if ((j & 3) == 0) packed[j >> 2] = 0;
        packed[j >> 2] |= (v & 0xFF) << (8 * (j & 3));
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) local_s[(h * C + c) * 8 + k] = packed[k];
      if (ck.local) {
        int *dst = reinterpret_cast<int *>(ck.local + (((size_t)b * 3 + h) * kMaxCand + c) * 32);
#pragma unroll
        for (int k = 0; k < 8; ++k) dst[k] = packed[k];
      }
    }
  }
  __syncthreads();
  // Stage 2: global feature = sat8(round_div(sum_c local, C)).
  if (tid < 96) {
    const int h = tid >> 5, j = tid & 31;
    const int8_t *l8 = reinterpret_cast<const int8_t *>(local_s);
    int s = 0;
    for (int c = 0; c < C; ++c) s += l8[(h * C + c) * 32 + j];
    const int8_t gv = (int8_t)sat_bits(round_div_pos(s, C), 8);
    reinterpret_cast<int8_t *>(glob)[h * 32 + j] = gv;
    if (ck.global) ck.global[((size_t)b * 3 + h) * 32 + j] = gv;
  }
  __syncthreads();
  // Stage 3: score MLP on [local | global] and the 2-way selector softmax.
  {
    const int s1_in = -16 - (p.concat_out_exp + p.score_w1_exp), s1_out = p.h1_out_exp + 16;
    const int s2_in = -16 - (p.h1_out_exp + p.score_w2_exp), s2_out = p.h2_out_exp + 16;
    const int s3 = p.logits_out_exp - (p.h2_out_exp + p.score_w3_exp);
    const int sq = -16 - p.logits_out_exp;
    for (int q = tid; q < 3 * C; q += 256) {
      const int h = q / C, c = q - h * C;
      int lg[16];
#pragma unroll
      for (int k = 0; k < 8; ++k) lg[k] = local_s[(h * C + c) * 8 + k];
#pragma unroll
      for (int k = 0; k < 8; ++k) lg[8 + k] = glob[h * 8 + k];
      int h1[8];
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        int acc = 0;
        const int *w = &w1[(h * 32 + j) * 16];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = dot4(lg[k], w[k], acc);
        const int v = gelu_post((i64)acc + p.b1[h * 32 + j], s1_in, s1_out);
        if ((j & 3) == 0) h1[j >> 2] = 0;
        h1[j >> 2] |= (v & 0xFF) << (8 * (j & 3));
      }
      int h2[4];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int acc = 0;
        const int *w = &w2[(h * 16 + j) * 8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc = dot4(h1[k], w[k], acc);
        const int v = gelu_post((i64)acc + p.b2[h * 16 + j], s2_in, s2_out);
        if ((j & 3) == 0) h2[j >> 2] = 0;
        h2[j >> 2] |= (v & 0xFF) << (8 * (j & 3));
      }
      int qv[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        int acc = 0;
        const int *w = &w3[(h * 2 + j) * 4];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = dot4(h2[k], w[k], acc);
        const int logit = (int)requant_shift((i64)acc + p.b3[h * 2 + j], s3, 8);
        qv[j] = (int)requant_shift(logit, sq, 24);
      }
      const int mx = qv[0] > qv[1] ? qv[0] : qv[1];
      const unsigned e0 = softmax_exp(qv[0] - mx), e1 = softmax_exp(qv[1] - mx);
      const unsigned ratio = softmax_ratio(e1, softmax_recip((u64)e0 + e1));
      hs[h * C + c] = (int)(ratio > 65536u ? 65536u : ratio);
      if (ck.head_scores) ck.head_scores[((size_t)b * 3 + h) * kMaxCand + c] = hs[h * C + c];
    }
  }
  __syncthreads();
  // Stage 4: head-weight MLP (3->3 GELU, 3->3 PLAN) and the weighted fuse.
  {
    const int a_in = -16 - (p.stats_out_exp + p.hw_w1_exp), a_out = p.hw_hidden_out_exp + 16;
    const int b_sh = -16 - (p.hw_hidden_out_exp + p.hw_w2_exp);
    for (int c = tid; c < C; c += 256) {
      int hid[3];
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        int acc = p.hw_b1[j];
#pragma unroll
        for (int k = 0; k < 3; ++k) acc += (int)stats[c * 3 + k] * (int)p.hw_w1t[j * 3 + k];
        hid[j] = gelu_post(acc, a_in, a_out);
      }
      i64 num = 0, den = 0;
      int w[3];
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        i64 acc = p.hw_b2[j];
#pragma unroll
        for (int k = 0; k < 3; ++k) acc += (i64)hid[k] * p.hw_w2t[j * 3 + k];
        w[j] = sat_q016(plan_sigmoid((int)requant_shift(acc, b_sh, 24)));
        if (ck.head_weights) ck.head_weights[((size_t)b * kMaxCand + c) * 3 + j] = w[j];
        num += (i64)hs[j * C + c] * w[j];
        den += w[j];
      }
      if (den == 0) {
        num = (i64)hs[c] + hs[C + c] + hs[2 * C + c];
        den = 3;
        atomicOr(&warn_head, 1);
      }
      const int f = sat_q016(round_div_pos(num, den));
      fused_s[c] = f;
      fused_out[(size_t)b * kMaxCand + c] = f;
    }
  }
  __syncthreads();
  // The head-fuse warning travels to k_selector_keep in the state word.
  if (tid == 0) st[4] = warn_head;
}

// Stable keep list of the normal candidates (fused >= 32768, input order)
// and the per-image state {token_count, package_present, kept, pruned,
// warnings} (selector.py:456-500).  One wavefront per image.
__global__ __launch_bounds__(64) void k_selector_keep(const int32_t *offsets,
                                                      const uint8_t *pkg_in,
                                                      const int32_t *fused, int32_t *kept_index,
                                                      int32_t *state, int head_warn_in_state) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int C = offsets[b + 1] - offsets[b] - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  int32_t *st = state + (size_t)b * 5;
  if (C < 1 || C > kMaxCand || C - pkg < 1) {
    if (lane == 0) { st[0] = -1; st[1] = 0; st[2] = 0; st[3] = 0; st[4] = 0; }
    return;
  }
  const int32_t *f = fused + (size_t)b * kMaxCand;
  const int n_norm = C - pkg;
  int kept = 0;
  i64 den = 0;
  for (int base = 0; base < C; base += 64) {
    const int c = base + lane;
    const bool in = c < C;
    const int fc = in ? f[c] : 0;
    const bool is_norm = c < n_norm;
    const bool keep = is_norm && fc >= 32768;
    const bool part = (is_norm && !keep) || (pkg && c == C - 1);
    const u64 mask = __ballot(keep);
    const int before = __popcll(mask & ((1ull << lane) - 1ull));
    if (keep) kept_index[(size_t)b * kMaxCand + kept + before] = c;
    kept += __popcll(mask);
    i64 d = part ? fc : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off);
    den += d;
  }
  for (int i = kept + lane; i < kMaxCand; i += 64) kept_index[(size_t)b * kMaxCand + i] = -1;
  if (lane == 0) {
    const int warn_head = head_warn_in_state ? (st[4] & 1) : 0;
    const int n_part = C - kept;  // pruned normals + the incoming package
    const int exists = n_part > 0;
    st[0] = 1 + kept + exists;
    st[1] = exists;
    st[2] = kept;
    st[3] = n_part - pkg;
    st[4] = warn_head | ((exists && den == 0) ? 2 : 0);
  }
}

__global__ __launch_bounds__(256) void k_selector_compact(
    const int8_t *tokens, const int32_t *offsets, const uint8_t *pkg_in, int batch,
    const int32_t *fused, const int32_t *kept_index, const int32_t *state, int8_t *out,
    int32_t *out_offsets, uint8_t *pkg_out, int32_t *token_counts, int stage) {
  __shared__ int red[256];
  __shared__ long long den_s;
  const int b = blockIdx.x, tid = threadIdx.x;
  int s = 0;
  for (int i = tid; i < b; i += 256) s += max(state[(size_t)i * 5], 0);
  red[tid] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  const int out0 = red[0];
  const int32_t *st = state + (size_t)b * 5;
  const int count = st[0], exists = st[1], kept = st[2];
  const int row0 = offsets[b], C = offsets[b + 1] - row0 - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  if (tid == 0) {
    out_offsets[b] = out0;
    if (b == batch - 1) out_offsets[batch] = out0 + (count > 0 ? count : 0);
    pkg_out[b] = (uint8_t)exists;
    if (token_counts) token_counts[(size_t)b * 4 + stage] = count;
  }
  if (count <= 0) return;
  // CLS and kept rows, 16 bytes per thread step.
  const int *ki = kept_index + (size_t)b * kMaxCand;
  for (int i = tid; i < (1 + kept) * 12; i += 256) {
    const int r = i / 12, chunk = i - r * 12;
    const int src = r == 0 ? row0 : row0 + 1 + ki[r - 1];
    reinterpret_cast<v4i *>(out + (size_t)(out0 + r) * 192)[chunk] =
        reinterpret_cast<const v4i *>(tokens + (size_t)src * 192)[chunk];
  }
  if (!exists) return;
  const int32_t *f = fused + (size_t)b * kMaxCand;
  const int n_norm = C - pkg;
  if (tid < 64) {
    long long d = 0;
    for (int c = tid; c < C; c += 64) {
      const bool part = (c < n_norm && f[c] < 32768) || (pkg && c == C - 1);
      d += part ? f[c] : 0;
    }
    for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off);
    if (tid == 0) den_s = d;
  }
  __syncthreads();
  const long long den = den_s;
  const int n_part = C - kept;
  if (tid < 192) {
    long long num = 0;
    const int8_t *cand = tokens + (size_t)(row0 + 1) * 192 + tid;
    for (int c = 0; c < C; ++c) {
      const bool part = (c < n_norm && f[c] < 32768) || (pkg && c == C - 1);
      if (part) num += (den == 0 ? 1ll : (long long)f[c]) * cand[(size_t)c * 192];
    }
    out[(size_t)(out0 + 1 + kept) * 192 + tid] =
        (int8_t)sat_bits(round_div_pos(num, den == 0 ? n_part : den), 8);
  }
}

int launch_selector(const SelectorArgs &a, hipStream_t s) {
  if (a.batch <= 0) return HV_OK;
  int rc = HV_OK;
  if (a.p) {
    hipLaunchKernelGGL(k_selector_score, dim3(a.batch), dim3(256), 0, s, *a.p, a.tokens,
                       a.offsets, a.pkg_in, a.fused, a.kept_index, a.state, a.ck);
    if ((rc = check_hip(hipGetLastError(), "k_selector_score launch"))) return rc;
  }
  hipLaunchKernelGGL(k_selector_keep, dim3(a.batch), dim3(64), 0, s, a.offsets, a.pkg_in,
                     a.fused, a.kept_index, a.state, a.p ? 1 : 0);
  if ((rc = check_hip(hipGetLastError(), "k_selector_keep launch"))) return rc;
  hipLaunchKernelGGL(k_selector_compact, dim3(a.batch), dim3(256), 0, s, a.tokens, a.offsets,
                     a.pkg_in, a.batch, a.fused, a.kept_index, a.state, a.out_tokens,
                     a.out_offsets, a.pkg_out, a.token_counts, a.stage);
  return check_hip(hipGetLastError(), "k_selector_compact launch");
}

}  // namespace hv
