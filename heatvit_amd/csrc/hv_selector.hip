// hv_selector.hip -- token selector (selector.token_selector,
// selector.py:503-563) over a ragged batch.
//
// k_selector_image, one 1024-thread workgroup per image (XCD-major): the
//   three heads' local MLP + head statistic (:253, :358), candidate mean
//   (:273), concat + 64->32->16->2 score MLP + 2-way selector softmax
//   (:292, :307, :338) as int8 MFMAs over tiles of 16 candidates, every
//   weight and intermediate in LDS; then, per candidate, the head-weight
//   MLP with PLAN (:370) and the head fuse (:392); the stable keep list
//   (fused >= 32768) and the per-image state of finalize_tokens (:456-500);
//   and the package token (score-weighted mean of the pruned normals plus
//   the incoming package, or their plain mean when the scores sum to
//   zero), written to a per-image scratch row.  Each candidate row is read
//   from memory by this workgroup only.
// k_selector_keep (finalize_tokens from given fused scores): the keep list
//   and state of one image per workgroup.
// k_selector_compact, one workgroup per image with the same XCD-major
//   order as k_selector_image: the image's output offset (the token counts
//   of the images before it), then CLS, the kept rows in input order and
//   the package row there (stream compaction).
//
// GELU layers use the int32 requant/GELU path when the host finds every
// shift in [-30, 30] and each layer's biases satisfy |b| <= 2^30 - 1 -
// K*2^14 (checked per head, uniform); otherwise the exact 64-bit form.
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
// All NT threads call it; the caller puts a barrier after it.
template <int NT>
__device__ __forceinline__ void sel_stage_lut(const SelLut &t, unsigned *lut, int tid) {
  const v4i *src = reinterpret_cast<const v4i *>(kGeluLut + t.off);
  v4i *dst = reinterpret_cast<v4i *>(lut);
  const int n4 = t.words >> 2;
  for (int base = tid; base < n4; base += 4 * NT) {
    v4i v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = src[min(base + r * NT, n4 - 1)];
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[min(base + r * NT, n4 - 1)] = v[r];
  }
}

// A step table held in registers between its loads and its LDS stores, so
// a layer's table loads can be in flight while the previous layer runs
// (NT threads, at most kLutRegs 16-byte words each).
constexpr int kLutRegs = 4;
template <int NT>
__device__ __forceinline__ void lut_load(const SelLut &t, v4i (&v)[kLutRegs], int tid) {
  static_assert(kGeluLutMaxWords / 4 <= kLutRegs * NT, "one round of table loads");
  const v4i *src = reinterpret_cast<const v4i *>(kGeluLut + t.off);
  const int n4 = t.words >> 2;
#pragma unroll
  for (int r = 0; r < kLutRegs; ++r) v[r] = src[min(tid + r * NT, n4 - 1)];
}
template <int NT>
__device__ __forceinline__ void lut_store(const SelLut &t, const v4i (&v)[kLutRegs],
                                          unsigned *lut, int tid) {
  const int n4 = t.words >> 2;
#pragma unroll
  for (int r = 0; r < kLutRegs; ++r) reinterpret_cast<v4i *>(lut)[min(tid + r * NT, n4 - 1)] = v[r];
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

constexpr int kCandTiles = (kMaxCand + 15) / 16;  // 13 tiles of 16 candidates
constexpr int kCandPad = kCandTiles * 16;

// Image of logical index L = XCD-major order of workgroup blockIdx.x over a
// grid that is a multiple of 8: workgroups go round-robin over the 8 XCDs,
// so XCD x runs images [x * B8, (x + 1) * B8).  -1 past the batch.
__device__ __forceinline__ int xcd_image(int batch) {
  const int B8 = (batch + 7) >> 3;
  const int L = (blockIdx.x & 7) * B8 + (blockIdx.x >> 3);
  return L < batch ? L : -1;
}

// An image the selector takes: CLS plus at least one candidate
// (selector.py:513-514), at most 196 candidates, and with an incoming
// package a normal candidate beside it (:448-449).
__device__ __forceinline__ bool image_ok(int row0, int C, int pkg) {
  return C >= 1 && C <= kMaxCand && C - pkg >= 1 && row0 >= 0;
}

__device__ __forceinline__ void state_invalid(int32_t *st) {
  st[0] = -1; st[1] = 0; st[2] = 0; st[3] = 0; st[4] = 0;
}

// Head fuse (selector.py:370-418), in three steps over one thread per
// candidate and head-weight unit: the head-weight MLP's GELU layer on the
// head statistics (3 -> 3), its PLAN layer (3 -> 3), and the weighted mean
// of the head scores (plain mean, and the warning, when the weights sum to
// zero).  The biases are any int32 and the reference adds them in int64
// (gemm.py:118-119): the three products (|sum| < 2^16) are summed in 32
// bits and the bias added in 64; the empty asm keeps the compiler from
// folding bias and products into one 32-bit dot-product accumulation, which
// wraps for biases near the int32 limits.
__device__ __forceinline__ int fuse_hidden(const hv_selector_dev &p, const int8_t *stats, int j) {
  const int a_in = -16 - (p.stats_out_exp + p.hw_w1_exp), a_out = p.hw_hidden_out_exp + 16;
  int dot = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) dot += (int)stats[k] * (int)p.hw_w1t[j * 3 + k];
  asm volatile("" : "+v"(dot));
  return gelu_post((i64)p.hw_b1[j] + dot, a_in, a_out);
}

__device__ __forceinline__ int fuse_weight(const hv_selector_dev &p, const int *hid, int j) {
  const int b_sh = -16 - (p.hw_hidden_out_exp + p.hw_w2_exp);
  int dot = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) dot += hid[k] * (int)p.hw_w2t[j * 3 + k];
  asm volatile("" : "+v"(dot));
  return sat_q016(plan_sigmoid((int)requant_shift((i64)p.hw_b2[j] + dot, b_sh, 24)));
}

// hs[0], hs[kMaxCand], hs[2 * kMaxCand]: the candidate's head scores; w[0..2]
// its head weights.
__device__ __forceinline__ int fuse_mean(const int32_t *hs, const int *w, bool *warn) {
  i64 num = 0, den = 0;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    num += (i64)hs[j * kMaxCand] * w[j];
    den += w[j];
  }
  *warn = den == 0;
  if (den == 0) {
    num = (i64)hs[0] + hs[kMaxCand] + hs[2 * kMaxCand];
    den = 3;
  }
  return sat_q016(round_div_pos_d(num, den));  // num < 2^35, den < 2^18
}

// The stable keep list and state of one image (selector.py:456-500) from
// the fused scores: thread c (c < 256) holds candidate c's score fc (0 past
// C) and its head-fuse warning; every thread of the NT-thread workgroup
// calls it.  Writes kept_index ki[0 .. kept) = the kept normals (fused >=
// 32768) in input order, ki[kept .. 196) = -1, and the state {token_count,
// package_present, kept, pruned, warnings}; bad (any thread) marks the
// image invalid (state token count -1).  Returns the kept count, or -1 when
// the image is invalid; *den_out receives the sum of the partitioned
// candidates' scores (the package's divisor).
template <int NT>
__device__ __forceinline__ int keep_list(int C, int pkg, int fc, bool warn, bool bad, int32_t *ki,
                                         int32_t *st, i64 *den_out = nullptr) {
  constexpr int NWAVE = NT / 64;
  __shared__ int w_kept[NWAVE], w_flags[NWAVE], w_den[NWAVE];
  const int c = threadIdx.x, lane = c & 63, wave = c >> 6;
  const int n_norm = C - pkg;
  const bool is_norm = c < n_norm;
  const bool keep = is_norm && fc >= 32768;
  const bool part = (is_norm && !keep) || (pkg && c == C - 1);
  const u64 mask = __ballot(keep);
  // valid scores are at most 65536, so a wavefront's sum fits 32 bits (an
  // invalid image is rejected below before the sum is used)
  int d = part ? fc : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off);
  const int flags = (__ballot(warn) != 0 ? 1 : 0) | (__ballot(bad) != 0 ? 2 : 0);
  if (lane == 0) {
    w_kept[wave] = __popcll(mask);
    w_den[wave] = d;
    w_flags[wave] = flags;
  }
  __syncthreads();
  int before = __popcll(mask & ((1ull << lane) - 1ull)), kept = 0, any = 0;
  i64 den = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    before += w < wave ? w_kept[w] : 0;
    kept += w_kept[w];
    den += w_den[w];
    any |= w_flags[w];
  }
  if (any & 2) {
    if (c == 0) state_invalid(st);
    return -1;
  }
  if (den_out) *den_out = den;
  if (keep) ki[before] = c;
  if (c >= kept && c < kMaxCand) ki[c] = -1;
  if (c == 0) {
    const int n_part = C - kept;  // pruned normals + the incoming package
    const int exists = n_part > 0;
    st[0] = 1 + kept + exists;
    st[1] = exists;
    st[2] = kept;
    st[3] = n_part - pkg;
    const int warn_bits = ((any & 1) ? HV_WARN_HEAD_DEN_ZERO : 0) |
                          ((exists && den == 0) ? HV_WARN_PACKAGE_DEN_ZERO : 0);
    st[4] = warn_bits;
  }
  return kept;
}

// Package token of one image (selector.py:470-500): dst[ch] = sat8(
// round_div(sum_c w_c x_c[ch], sum_c w_c)) over the pruned normals and the
// incoming package with w_c = fused score, or their plain mean (w_c = 1,
// divisor n_part) when those scores sum to zero (den: the scores' sum, from
// keep_list).  |num| <= 196 * 65536 *
// 128 < 2^31.  Thread c holds candidate c's fused score fv; thread (channel
// group of 16, candidate group g < G) accumulates candidates g, g + G, ...
// (its candidate rows loaded at once, weight 0 for kept ones) and part_sum
// ([G][192] ints) sums the groups.  Every thread of the NT-thread workgroup
// calls it; cand points at candidate 0's row (16-byte aligned rows, RS
// bytes apart, in memory or LDS).
template <int NT, int RS, int G>
__device__ __forceinline__ void package_row(const int8_t *cand, int C, int pkg, int kept, int fv,
                                            i64 den, int8_t *dst, int *wgt, int *part_sum) {
  constexpr int kSteps = (kMaxCand + G - 1) / G;
  static_assert(12 * G <= NT, "one thread per channel group and candidate group");
  const int tid = threadIdx.x;
  const int cg = tid / 12, chg = tid - cg * 12;
  v4i xv[kSteps];
  if (tid < 12 * G) {
    const int8_t *cp = cand + chg * 16;
#pragma unroll
    for (int j = 0; j < kSteps; ++j)
      xv[j] = *reinterpret_cast<const v4i *>(cp + (size_t)min(cg + G * j, C - 1) * RS);
  }
  const int n_norm = C - pkg;
  const bool part = tid < C && ((tid < n_norm && fv < 32768) || (pkg && tid == C - 1));
  if (tid < C) wgt[tid] = part ? (den == 0 ? 1 : fv) : 0;
  __syncthreads();
  if (tid < 12 * G) {
    int acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0;
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const int c = cg + G * j;
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
    for (int g = 0; g < G; ++g) num += part_sum[g * 192 + tid];
    dst[tid] = (int8_t)sat_bits(round_div_pos_d(num, den == 0 ? n_part : den), 8);
  }
}

// Eight GELU post-ops of a layer from its step table in LDS, packed four
// to a word: q = rsa(v, s) (or v << -s after the pre-clamp) with the
// direction of the launch-uniform shift chosen once; the table's clamp
// [qlo, qhi] lies inside the 24-bit range, so q needs no clamp of its own.
__device__ __forceinline__ void sel_gelu_pack8(const int (&v)[8], const Rq &ra, const unsigned *lut,
                                               const SelLut &t, unsigned (&ow)[2]) {
  int q[8];
  if (ra.s > 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = (v[i] + ra.rnd + (v[i] >> 31)) >> ra.s;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = min(max(v[i], ra.vlo), ra.vhi) << -ra.s;
  }
  gelu_table_pack_n<8>(q, ow, lut, t.cb, t.qlo, t.qhi);
}

constexpr int kImgThreads = 1024, kXsRow = 208;

// One workgroup per image (XCD-major).  Per layer, the (head, tile) units of
// the three heads run over the eight wavefronts; the layer's GELU step table
// (when its output shift has one) is staged once for the three heads:
//   local = GELU(x_h [C][64] . Wl [64][32] + bl)     16x16x64, 2 column tiles
//   h1    = GELU(local . W1[0:32] + b1')             16x16x32, 2 column tiles
//   h2    = GELU(h1 . W2 + b2)                       16x16x32, 1 column tile
// where b1' = b1 + global . W1[32:64] (the global feature is the same for
// every candidate, so the concat's second half is a per-head bias, exact in
// 64 bits).  With the weights as the MFMA's first operand, result lane l of
// a tile holds output channels 16 ct + 4 (l / 16) + i of candidate l % 16,
// stored as one word.  Logits (16 -> 2), the 2-way softmax and the
// lane mean of the head slice (the head statistic) are per candidate; the
// head fuse, the keep list and the package token follow in the same
// workgroup.  The package row goes to pkg_rows[b] for k_selector_compact.
__global__ __launch_bounds__(kImgThreads) void k_selector_image(
    hv_selector_dev p, const int8_t *tokens, const int32_t *offsets, int batch,
    const uint8_t *pkg_in, int fast_shifts, hv_selector_ckpt ck, SelLut tl, SelLut t1, SelLut t2,
    int32_t *fused_out, int32_t *kept_index, int32_t *state, int8_t *pkg_rows,
    int32_t *img_warn) {
  constexpr int NT = kImgThreads;
  __shared__ __attribute__((aligned(16))) unsigned lut[kGeluLutMaxWords];
  __shared__ __attribute__((aligned(16))) int8_t wl[3][32 * 64];   // local_wt[h] [32][64]
  __shared__ __attribute__((aligned(16))) int8_t w1[3][32 * 64];   // w1t[h] [32][64]
  __shared__ __attribute__((aligned(16))) int8_t w2[3][16 * 32];   // w2t[h] [16][32]
  __shared__ int w3[3][8];                                         // w3t[h] [2][16] as words
  __shared__ int bl[3][32], bb2[3][16];
  __shared__ i64 bb1[3][32];                                       // b1 + global . W1[32:64]
  // local [3][208][32], then h2 [3][208][16]; h1 [3][208][32]
  __shared__ __attribute__((aligned(16))) int8_t act_a[3 * kCandPad * 32];
  __shared__ __attribute__((aligned(16))) int8_t act_b[3 * kCandPad * 32];
  __shared__ int hs_s[3 * kMaxCand];                               // head scores [h][c]
  __shared__ int8_t st_s[kMaxCand * 3];                            // head statistics [c][h]
  __shared__ int part[10][96];
  __shared__ int glob_s[3][32];
  __shared__ int fast_s[3][3];
  __shared__ int wgt[kMaxCand];
  // the image's candidate rows, 208-byte stride (conflict-free 16-byte
  // fragment reads of 16 consecutive rows)
  __shared__ __attribute__((aligned(16))) int8_t xs[kMaxCand * kXsRow];

  const int b = xcd_image(batch);
  if (b < 0) return;  // uniform: before any barrier
  constexpr int NW = NT / 64;  // wavefronts; each takes two units per round, NW apart
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, col = lane & 15, grp = lane >> 4;
  const int row0 = offsets[b], N = offsets[b + 1] - row0, C = N - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  int32_t *st = state + (size_t)b * 5;
  if (!image_ok(row0, C, pkg)) {
    if (tid == 0) state_invalid(st);
    return;
  }
  const int ntiles = (C + 15) >> 4;
  const int8_t *cand = tokens + (size_t)(row0 + 1) * 192;
  // Candidate rows into LDS: every 16-byte load of the image in flight at
  // once (items past the end repeat the last one), stored after the weight
  // and table loads below are issued.
  constexpr int kRowItems = (kMaxCand * 12 + NT - 1) / NT;
  v4i rv[kRowItems];
  const int n_items = C * 12;
#pragma unroll
  for (int j = 0; j < kRowItems; ++j)
    rv[j] = reinterpret_cast<const v4i *>(cand)[min(tid + j * NT, n_items - 1)];

  for (int i = tid; i < 3 * 128; i += NT) {  // 16-byte words of the three heads' weights
    const int h = i >> 7, k = i & 127;
    reinterpret_cast<v4i *>(wl[h])[k] = reinterpret_cast<const v4i *>(p.local_wt + h * 2048)[k];
    reinterpret_cast<v4i *>(w1[h])[k] = reinterpret_cast<const v4i *>(p.w1t + h * 2048)[k];
    if (k < 32)
      reinterpret_cast<v4i *>(w2[h])[k] = reinterpret_cast<const v4i *>(p.w2t + h * 512)[k];
  }
  // int32 GELU preconditions per head: |acc| <= K*2^14 for the layer's K
  // (head h's biases sit in one run of lanes of one wavefront: a ballot).
  const int lim64 = (1 << 30) - 1 - 64 * 16384, lim32 = (1 << 30) - 1 - 32 * 16384;
  if (tid < 24) w3[tid >> 3][tid & 7] = reinterpret_cast<const int *>(p.w3t)[tid];
  if (tid >= 64 && tid < 160) {  // local biases: head h in lanes 32 (h % 2) .. +31
    const int v = p.local_b[tid - 64], h = (tid - 64) >> 5;
    bl[h][(tid - 64) & 31] = v;
    const u64 m = __ballot(fast_shifts && v <= lim64 && v >= -lim64);
    if ((tid & 31) == 0) fast_s[h][0] = (unsigned)(m >> (tid & 32)) == 0xFFFFFFFFu;
  }
  if (tid >= 192 && tid < 240) {  // score layer 2 biases: head h in lanes 16 h .. +15
    const int v = p.b2[tid - 192], h = (tid - 192) >> 4;
    bb2[h][(tid - 192) & 15] = v;
    const u64 m = __ballot(fast_shifts && v <= lim32 && v >= -lim32);
    if ((tid & 15) == 0) fast_s[h][2] = ((unsigned)(m >> (16 * h)) & 0xFFFFu) == 0xFFFFu;
  }
  if (tl.off >= 0) sel_stage_lut<NT>(tl, lut, tid);
#pragma unroll
  for (int j = 0; j < kRowItems; ++j) {
    const int i = min(tid + j * NT, n_items - 1), c = i / 12;
    *reinterpret_cast<v4i *>(&xs[c * kXsRow + (i - c * 12) * 16]) = rv[j];
  }
  // score layer 1's table loads in flight during the local layer
  v4i lv[kLutRegs];
  if (t1.off >= 0) lut_load<NT>(t1, lv, tid);
  __syncthreads();

  // Local MLP and head statistics: unit u = h * nt2 + tile, tile = 2 rt + ct;
  // two units per round, both candidate loads in flight, then their eight
  // table lookups staged together.
  {
    const int sh_in = -16 - (p.in_exp + p.local_w_exp), sh_out = p.local_out_exp + 16;
    const Rq ra = rq_setup(sh_in, -(1 << 23), (1 << 23) - 1), rb = rq_setup(sh_out, -128, 127);
    // a second barrier here measured faster than none (three runs, about
    // 1 us per launch)
    __syncthreads();
    const int nt2 = ntiles * 2, nu = 3 * nt2;
    for (int u0 = wave; u0 < nu; u0 += 2 * NW) {
      int hh[2], tv[2];
      bool valid[2], fast[2];
      v4i a[2], acc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int uu = min(u0 + NW * u, nu - 1);
        valid[u] = u0 + NW * u < nu;
        hh[u] = (uu >= nt2 ? 1 : 0) + (uu >= 2 * nt2 ? 1 : 0);  // uu / nt2 (< 3)
        tv[u] = uu - hh[u] * nt2;
        fast[u] = fast_s[hh[u]][0];
        const int c = min((tv[u] >> 1) * 16 + col, C - 1);
        a[u] = *reinterpret_cast<const v4i *>(&xs[c * kXsRow + hh[u] * 64 + grp * 16]);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const v4i wb =
            *reinterpret_cast<const v4i *>(&wl[hh[u]][((tv[u] & 1) * 16 + col) * 64 + grp * 16]);
        // weights as the first operand: lane (col, grp) gets output channels
        // 16 ct + 4 grp + i of candidate 16 rt + col, stored as one word
        acc[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wb, a[u], v4i{0}, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int rt = tv[u] >> 1, cc = rt * 16 + col;
        if (valid[u] && (tv[u] & 1) == 0) {
          // lane mean of the candidate's 64 head lanes (selector.py:358-367)
          int sum = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) sum = dot4(a[u][k], 0x01010101, sum);
          sum += __shfl_xor(sum, 16);
          sum += __shfl_xor(sum, 32);
          if (grp == 0 && cc < C) {
            const int8_t stat = (int8_t)sat_bits(round_div_pos(sum, 64), 8);
            st_s[cc * 3 + hh[u]] = stat;
            if (ck.head_stats) ck.head_stats[((size_t)b * kMaxCand + cc) * 3 + hh[u]] = stat;
          }
        }
      }
      if (fast[0] && fast[1] && tl.off >= 0) {
        int vv[8];
        unsigned ow[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int jb = (tv[u] & 1) * 16 + 4 * grp;
#pragma unroll
          for (int i = 0; i < 4; ++i) vv[4 * u + i] = acc[u][i] + bl[hh[u]][jb + i];
        }
        sel_gelu_pack8(vv, ra, lut, tl, ow);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int rt = tv[u] >> 1, jb = (tv[u] & 1) * 16 + 4 * grp;
          if (valid[u])
            *reinterpret_cast<unsigned *>(&act_a[(hh[u] * kCandPad + rt * 16 + col) * 32 + jb]) =
                ow[u];
        }
      } else {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int rt = tv[u] >> 1, jb = (tv[u] & 1) * 16 + 4 * grp;
          if (valid[u]) {
            unsigned o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              o[i] = (unsigned)(fast[u] && tl.off >= 0
                                    ? (int)gelu_table_u8(rq(acc[u][i] + bl[hh[u]][jb + i], ra),
                                                         lut, tl.cb, tl.qlo, tl.qhi)
                                    : sel_gelu(acc[u][i], bl[hh[u]][jb + i], fast[u], ra, rb,
                                               sh_in, sh_out));
            *reinterpret_cast<unsigned *>(&act_a[(hh[u] * kCandPad + rt * 16 + col) * 32 + jb]) =
                pack_lo4(o[0], o[1], o[2], o[3]);
          }
        }
      }
    }
  }
  __syncthreads();
  // score layer 1's table replaces the local layer's (barriers follow)
  if (t1.off >= 0) lut_store<NT>(t1, lv, lut, tid);
  // Global features = sat8(round_div(sum_c local, C)) per head and channel,
  // five partial sums each; the local checkpoint before act_a is reused.
  if (tid < 10 * 96) {
    const int prt = tid / 96, hc = tid - prt * 96, h = hc >> 5, ch = hc & 31;
    int sacc = 0;
    for (int c = prt; c < C; c += 10) sacc += act_a[(h * kCandPad + c) * 32 + ch];
    part[prt][hc] = sacc;
  }
  if (ck.local)
    for (int i = tid; i < 3 * C * 2; i += NT) {
      const int h = i / (C * 2), k = i - h * C * 2;
      reinterpret_cast<v4i *>(ck.local + ((size_t)b * 3 + h) * kMaxCand * 32)[k] =
          reinterpret_cast<const v4i *>(act_a + h * kCandPad * 32)[k];
    }
  __syncthreads();
  if (tid < 96) {
    int sacc = 0;
#pragma unroll
    for (int q = 0; q < 10; ++q) sacc += part[q][tid];
    const int gv = (int)sat_bits(round_div_pos_d(sacc, C), 8);
    glob_s[tid >> 5][tid & 31] = gv;
    if (ck.global) ck.global[((size_t)b * 3 + (tid >> 5)) * 32 + (tid & 31)] = (int8_t)gv;
  }
  __syncthreads();
  if (tid < 96) {
    // global . W1[32:64] in 32 bits (|sum| <= 32 * 128 * 127), the bias in 64
    const int h = tid >> 5, j = tid & 31;
    const int *wr = reinterpret_cast<const int *>(&w1[h][j * 64 + 32]);
    int dot = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int gp = (glob_s[h][4 * q] & 0xFF) | ((glob_s[h][4 * q + 1] & 0xFF) << 8) |
                     ((glob_s[h][4 * q + 2] & 0xFF) << 16) | (glob_s[h][4 * q + 3] << 24);
      dot = dot4(gp, wr[q], dot);
    }
    const i64 v = (i64)p.b1[h * 32 + j] + dot;
    bb1[h][j] = v;
    const u64 m = __ballot(fast_shifts && v <= lim32 && v >= -lim32);
    if (j == 0) fast_s[h][1] = (unsigned)(m >> (tid & 32)) == 0xFFFFFFFFu;
  }
  // Score layer 1 (local half): unit u = h * nt2 + 2 rt + ct, two units per
  // round with their eight table lookups staged together.
  {
    const int sh_in = -16 - (p.concat_out_exp + p.score_w1_exp), sh_out = p.h1_out_exp + 16;
    const Rq ra = rq_setup(sh_in, -(1 << 23), (1 << 23) - 1), rb = rq_setup(sh_out, -128, 127);
    __syncthreads();
    if (t2.off >= 0) lut_load<NT>(t2, lv, tid);  // score layer 2's table
    const int nt2 = ntiles * 2, nu = 3 * nt2;
    for (int u0 = wave; u0 < nu; u0 += 2 * NW) {
      int hh[2], tv[2];
      bool valid[2], fast[2];
      v4i acc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int uu = min(u0 + NW * u, nu - 1);
        valid[u] = u0 + NW * u < nu;
        hh[u] = (uu >= nt2 ? 1 : 0) + (uu >= 2 * nt2 ? 1 : 0);  // uu / nt2 (< 3)
        tv[u] = uu - hh[u] * nt2;
        fast[u] = fast_s[hh[u]][1];
        const int rt = tv[u] >> 1, ct = tv[u] & 1;
        const long a = *reinterpret_cast<const long *>(
            &act_a[(hh[u] * kCandPad + rt * 16 + col) * 32 + grp * 8]);
        const long wb =
            *reinterpret_cast<const long *>(&w1[hh[u]][(ct * 16 + col) * 64 + grp * 8]);
        // weights first: four channels of one candidate per lane
        acc[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wb, a, v4i{0}, 0, 0, 0);
      }
      if (fast[0] && fast[1] && t1.off >= 0) {
        int vv[8];
        unsigned ow[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int jb = (tv[u] & 1) * 16 + 4 * grp;
#pragma unroll
          for (int i = 0; i < 4; ++i) vv[4 * u + i] = acc[u][i] + (int)bb1[hh[u]][jb + i];
        }
        sel_gelu_pack8(vv, ra, lut, t1, ow);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int jb = (tv[u] & 1) * 16 + 4 * grp;
          if (valid[u])
            *reinterpret_cast<unsigned *>(
                &act_b[(hh[u] * kCandPad + (tv[u] >> 1) * 16 + col) * 32 + jb]) = ow[u];
        }
      } else {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int jb = (tv[u] & 1) * 16 + 4 * grp;
          if (valid[u]) {
            unsigned o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const i64 bias = bb1[hh[u]][jb + i];
              o[i] = (unsigned)(fast[u] && t1.off >= 0
                                    ? (int)gelu_table_u8(rq(acc[u][i] + (int)bias, ra), lut,
                                                         t1.cb, t1.qlo, t1.qhi)
                                : fast[u] ? rq(gelu_q16(rq(acc[u][i] + (int)bias, ra)), rb)
                                          : gelu_exact64(acc[u][i], bias, sh_in, sh_out));
            }
            *reinterpret_cast<unsigned *>(
                &act_b[(hh[u] * kCandPad + (tv[u] >> 1) * 16 + col) * 32 + jb]) =
                pack_lo4(o[0], o[1], o[2], o[3]);
          }
        }
      }
    }
  }
  __syncthreads();
  if (t2.off >= 0) {  // score layer 2's table
    lut_store<NT>(t2, lv, lut, tid);
    __syncthreads();
  }
  // Score layer 2 into act_a ([3][208][16]): unit u = h * ntiles + rt, two
  // units per round.
  {
    const int sh_in = -16 - (p.h1_out_exp + p.score_w2_exp), sh_out = p.h2_out_exp + 16;
    const Rq ra = rq_setup(sh_in, -(1 << 23), (1 << 23) - 1), rb = rq_setup(sh_out, -128, 127);
    const int nu = 3 * ntiles;
    for (int u0 = wave; u0 < nu; u0 += 2 * NW) {
      int hh[2], rt[2];
      bool valid[2], fast[2];
      v4i acc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int uu = min(u0 + NW * u, nu - 1);
        valid[u] = u0 + NW * u < nu;
        hh[u] = (uu >= ntiles ? 1 : 0) + (uu >= 2 * ntiles ? 1 : 0);  // uu / ntiles (< 3)
        rt[u] = uu - hh[u] * ntiles;
        fast[u] = fast_s[hh[u]][2];
        const long a = *reinterpret_cast<const long *>(
            &act_b[(hh[u] * kCandPad + rt[u] * 16 + col) * 32 + grp * 8]);
        const long wb = *reinterpret_cast<const long *>(&w2[hh[u]][col * 32 + grp * 8]);
        acc[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wb, a, v4i{0}, 0, 0, 0);
      }
      if (fast[0] && fast[1] && t2.off >= 0) {
        int vv[8];
        unsigned ow[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) vv[4 * u + i] = acc[u][i] + bb2[hh[u]][4 * grp + i];
        sel_gelu_pack8(vv, ra, lut, t2, ow);
#pragma unroll
        for (int u = 0; u < 2; ++u)
          if (valid[u])
            *reinterpret_cast<unsigned *>(
                &act_a[(hh[u] * kCandPad + rt[u] * 16 + col) * 16 + 4 * grp]) = ow[u];
      } else {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (valid[u]) {
            unsigned o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int bias = bb2[hh[u]][4 * grp + i];
              o[i] = (unsigned)(fast[u] && t2.off >= 0
                                    ? (int)gelu_table_u8(rq(acc[u][i] + bias, ra), lut, t2.cb,
                                                         t2.qlo, t2.qhi)
                                    : sel_gelu(acc[u][i], bias, fast[u], ra, rb, sh_in, sh_out));
            }
            *reinterpret_cast<unsigned *>(
                &act_a[(hh[u] * kCandPad + rt[u] * 16 + col) * 16 + 4 * grp]) =
                pack_lo4(o[0], o[1], o[2], o[3]);
          }
        }
      }
    }
  }
  __syncthreads();
  // Logits, the 2-way selector softmax (keep = element 1) and checkpoints.
  {
    const int s3 = p.logits_out_exp - (p.h2_out_exp + p.score_w3_exp);
    const int sq = -16 - p.logits_out_exp;
    for (int i = tid; i < 3 * C; i += NT) {
      const int h = i / C, c = i - h * C;
      const v4i hv = *reinterpret_cast<const v4i *>(&act_a[(h * kCandPad + c) * 16]);
      int qv[2];
#pragma unroll
      for (int lj = 0; lj < 2; ++lj) {
        int acc = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = dot4(hv[k], w3[h][lj * 4 + k], acc);
        const int logit = (int)requant_shift((i64)acc + p.b3[h * 2 + lj], s3, 8);
        qv[lj] = (int)requant_shift(logit, sq, 24);
      }
      const int mx = qv[0] > qv[1] ? qv[0] : qv[1];
      const unsigned e0 = softmax_exp(qv[0] - mx), e1 = softmax_exp(qv[1] - mx);
      const unsigned ratio = softmax_ratio(e1, softmax_recip24(e0 + e1));
      const int hsv = (int)(ratio > 65536u ? 65536u : ratio);
      hs_s[h * kMaxCand + c] = hsv;
      if (ck.head_scores) ck.head_scores[((size_t)b * 3 + h) * kMaxCand + c] = hsv;
      if (ck.h2)
        *reinterpret_cast<v4i *>(ck.h2 + (((size_t)b * 3 + h) * kMaxCand + c) * 16) = hv;
    }
  }
  __syncthreads();
  // Head fuse: thread j * C + c takes head-weight unit j of candidate c
  // (hidden and weight layers, through LDS: the h1 buffer is free), then
  // thread c < C the mean; keep list and state.
  int *hid_s = reinterpret_cast<int *>(act_b), *hw_s = hid_s + 3 * kMaxCand;
  const int fj = (tid >= C ? 1 : 0) + (tid >= 2 * C ? 1 : 0), fcand = tid - fj * C;
  if (tid < 3 * C) hid_s[fcand * 3 + fj] = fuse_hidden(p, &st_s[fcand * 3], fj);
  __syncthreads();
  if (tid < 3 * C) {
    const int w = fuse_weight(p, &hid_s[fcand * 3], fj);
    hw_s[fcand * 3 + fj] = w;
    if (ck.head_weights) ck.head_weights[((size_t)b * kMaxCand + fcand) * 3 + fj] = w;
  }
  __syncthreads();
  int fc = 0;
  bool warn = false;
  if (tid < C) {
    fc = fuse_mean(&hs_s[tid], &hw_s[tid * 3], &warn);
    fused_out[(size_t)b * kMaxCand + tid] = fc;
  }
  i64 den = 0;
  const int kept =
      keep_list<NT>(C, pkg, fc, warn, false, kept_index + (size_t)b * kMaxCand, st, &den);
  if (tid == 0 && img_warn) img_warn[b] |= st[4];
  if (kept < 0 || C - kept == 0) return;  // uniform; no package row
  // (the step table's LDS is free: its last reader was score layer 2)
  static_assert(36 * 192 <= kGeluLutMaxWords, "package sums fit the table's LDS");
  package_row<NT, kXsRow, 36>(xs, C, pkg, kept, fc, den, pkg_rows + (size_t)b * 192, wgt,
                              reinterpret_cast<int *>(lut));
}

// finalize_tokens from given fused scores (hv_selector_finalize): the keep
// list and state of one image per workgroup, one thread per candidate.
// Given scores must be Q0.16 values in [0, 65536] (selector._q016): an
// image holding any other value is rejected like a bad token count.
__global__ __launch_bounds__(256) void k_selector_keep(const int32_t *offsets,
                                                       const uint8_t *pkg_in, int batch,
                                                       const int32_t *fused, int32_t *kept_index,
                                                       int32_t *state, int32_t *img_warn) {
  const int b = xcd_image(batch);
  if (b < 0) return;
  const int c = threadIdx.x;
  const int row0 = offsets[b], C = offsets[b + 1] - row0 - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  int32_t *st = state + (size_t)b * 5;
  if (!image_ok(row0, C, pkg)) {
    if (c == 0) state_invalid(st);
    return;
  }
  const int fc = c < C ? fused[(size_t)b * kMaxCand + c] : 0;
  const bool bad = c < C && (unsigned)fc > 65536u;
  keep_list<256>(C, pkg, fc, false, bad, kept_index + (size_t)b * kMaxCand, st);
  if (c == 0 && img_warn && st[0] > 0) img_warn[b] |= st[4];
}

// Stream compaction of one image (XCD-major, as k_selector_image): the
// image's output offset (the token counts of the images before it; an image
// with a bad count contributes 0), then CLS, the kept rows and the package
// row there.  The package row comes from pkg_rows (selector forward) or is
// computed here from the given fused scores (finalize).  Each workgroup
// sums the counts before its image itself, one load per thread: a separate
// one-workgroup scan kernel over all counts cost a launch (4.5 us each on
// the pruned batch-256 forward) against that sum.
__global__ __launch_bounds__(256) void k_selector_compact(
    const int8_t *tokens, const int32_t *offsets, const uint8_t *pkg_in, int batch,
    const int32_t *fused, const int32_t *kept_index, const int32_t *state,
    const int8_t *pkg_rows, int8_t *out, int32_t *out_offsets, uint8_t *pkg_out,
    int32_t *token_counts, int stage) {
  __shared__ int wgt[kMaxCand];
  __shared__ int part_sum[21 * 192];
  __shared__ int src_k[kMaxCand + 1];
  __shared__ int red[4];
  const int b = xcd_image(batch);
  if (b < 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t *st = state + (size_t)b * 5;
  const int count = st[0], exists = st[1], kept = st[2];
  int sum = 0;
  for (int i = tid; i < b; i += 256) sum += max(state[(size_t)i * 5], 0);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  const int out0 = red[0] + red[1] + red[2] + red[3];
  if (tid == 0) {
    out_offsets[b] = out0;
    if (b == batch - 1) out_offsets[batch] = out0 + max(count, 0);
    pkg_out[b] = (uint8_t)(count > 0 ? exists : 0);
    if (token_counts) token_counts[(size_t)b * 4 + stage] = count;
  }
  if (count <= 0) return;  // uniform
  const int row0 = offsets[b], C = offsets[b + 1] - row0 - 1;
  const int pkg = pkg_in ? (pkg_in[b] ? 1 : 0) : 0;
  // Source row of output row r is row0 + 1 + src_k[r]: -1 for the CLS row,
  // then the kept candidates.
  const int *ki = kept_index + (size_t)b * kMaxCand;
  if (tid <= kMaxCand) src_k[tid] = tid == 0 ? -1 : ki[tid - 1];
  __syncthreads();
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
  int8_t *prow = out + (size_t)(out0 + 1 + kept) * 192;
  if (pkg_rows) {
    if (tid < 12)
      reinterpret_cast<v4i *>(prow)[tid] =
          reinterpret_cast<const v4i *>(pkg_rows + (size_t)b * 192)[tid];
    return;
  }
  // the partitioned candidates' score sum (finalize's scores are checked
  // to lie in [0, 65536], so a wavefront's sum fits 32 bits)
  const int fv = tid < C ? fused[(size_t)b * kMaxCand + tid] : 0;
  const bool part = tid < C && ((tid < C - pkg && fv < 32768) || (pkg && tid == C - 1));
  int d = part ? fv : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off);
  if (lane == 0) red[wave] = d;
  __syncthreads();
  const i64 den = (i64)red[0] + red[1] + red[2] + red[3];
  package_row<256, 192, 21>(tokens + (size_t)(row0 + 1) * 192, C, pkg, kept, fv, den, prow, wgt,
                            part_sum);
}

int launch_selector(const SelectorArgs &a, hipStream_t s) {
  if (a.batch <= 0) return HV_OK;
  int rc = HV_OK;
  const dim3 grid((a.batch + 7) / 8 * 8);
  if (a.p) {
    if (!a.pkg_rows)
      return fail(HV_EVALUE, HV_ERR_ADDRESS, "selector: missing workspace");
    const hv_selector_dev p = *a.p;
    auto in = [](int v) { return v >= -30 && v <= 30; };
    const int fast = in(-16 - (p.in_exp + p.local_w_exp)) && in(p.local_out_exp + 16) &&
                     in(-16 - (p.concat_out_exp + p.score_w1_exp)) && in(p.h1_out_exp + 16) &&
                     in(-16 - (p.h1_out_exp + p.score_w2_exp)) && in(p.h2_out_exp + 16);
    auto table = [](int so) {
      if (so < kGeluLutSoMin || so > kGeluLutSoMax) return SelLut{-1, 0, 0, 0, 0};
      const GeluLutInfo &t = kGeluLutInfo[so - kGeluLutSoMin];
      return SelLut{t.off, t.words, t.qlo, t.qhi, -4 * (t.qlo >> kGeluCoarseShift)};
    };
    hv_launch(k_selector_image, grid, dim3(kImgThreads), 0, s, p, a.tokens, a.offsets, a.batch,
              a.pkg_in, fast, a.ck, table(p.local_out_exp + 16), table(p.h1_out_exp + 16),
              table(p.h2_out_exp + 16), a.fused, a.kept_index, a.state, a.pkg_rows, a.img_warn);
    if ((rc = check_hip(hipGetLastError(), "k_selector_image launch"))) return rc;
  } else {
    hv_launch(k_selector_keep, grid, dim3(256), 0, s, a.offsets, a.pkg_in, a.batch, a.fused,
              a.kept_index, a.state, a.img_warn);
    if ((rc = check_hip(hipGetLastError(), "k_selector_keep launch"))) return rc;
  }
  hv_launch(k_selector_compact, grid, dim3(256), 0, s, a.tokens, a.offsets, a.pkg_in, a.batch,
            a.fused, a.kept_index, a.state, a.p ? a.pkg_rows : nullptr, a.out_tokens,
            a.out_offsets, a.pkg_out, a.token_counts, a.stage);
  return check_hip(hipGetLastError(), "k_selector_compact launch");
}

}  // namespace hv
