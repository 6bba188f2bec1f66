// hv_gemm.hip -- int8 GEMM on CDNA4 MFMA with the golden model's fused
// writebacks (gemm.gemm_numpy + gemm.gemm_writeback, gemm.py:93-139).
//
// Tiling: a 256-thread workgroup owns a (64*MT) x (64*NT) output tile; its
// four wavefronts form a 2x2 grid, each computing MT x NT tiles of 32x32
// with v_mfma_i32_32x32x32_i8 (int32 accumulation is exact: |acc| <=
// K*128*128 < 2^31 for K <= 131071, so gemm_numpy's overflow check cannot
// fire).  A rows are read straight from HBM/L2 as 16-byte lane fragments;
// weights come pre-packed in MFMA operand order ("mfma32", see
// include/heatvit_hip.h) so every B fragment load is one coalesced 1 KiB
// wavefront read.  The K loop is software-pipelined one step deep.
//
// Epilogues (per output element v = acc + bias, int64):
//   EPI_I8/I32   requant(v, src, dst, 8|32)                     gemm.py:123-139
//   EPI_GELU     requant(gelu(requant(v, src, -16, 24)), -16, dst, 8)
//                                                    transformer.py:349-358
//   EPI_RESIDUAL t = requant(v, src, mid, 8); out = align_add(res, t)
//                                                    transformer.py:96-101
//   EPI_PATCH    t = requant(v, img+w, act, 8); out = align_add(t, pos[p+1])
//                into row b*197 + 1 + p                transformer.py:120-145
#include "hv_device.h"
#include "hv_internal.h"

namespace hv {

enum { EPI_I8 = HV_EPI_I8, EPI_I32 = HV_EPI_I32, EPI_GELU = HV_EPI_GELU,
       EPI_RES = HV_EPI_RESIDUAL, EPI_PATCH = 4 };

static constexpr int kPatchesPerImage = 196;
static constexpr int kTokens = 197;
static constexpr int kImageBytes = 224 * 224 * 3;

template <int AMODE>
__device__ __forceinline__ const int8_t *a_row(const GemmArgs &g, int r) {
  if (AMODE == A_GATHER) return g.a + (size_t)g.a_rows[r] * g.lda;
  return g.a + (size_t)r * g.lda;
}

// Patch gather (layout.patchify, layout.py:31-72): patch p = pr*14 + pc of
// image b; column k = (in_row*16 + in_col)*3 + ch maps to image byte
// ((pr*16 + in_row)*224 + pc*16)*3 + (k % 48).  A 16-byte fragment never
// crosses an in_row boundary (48 = 3*16).
__device__ __forceinline__ const int8_t *patch_ptr(const int8_t *images, int r, int k) {
  const int b = r / kPatchesPerImage, p = r - b * kPatchesPerImage;
  const int pr = p / 14, pc = p - pr * 14;
  const int in_row = k / 48, rem = k - in_row * 48;
  return images + (size_t)b * kImageBytes + ((pr * 16 + in_row) * 224 + pc * 16) * 3 + rem;
}

template <int MT, int NT, int EPI, int AMODE, int KTC>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g, int n_blocks) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = g.m_dev ? min(*g.m_dev, g.m) : g.m;
  const int nb = blockIdx.x % n_blocks, mb = blockIdx.x / n_blocks;
  constexpr int BM = 64 * MT, BN = 64 * NT;
  if (M <= 0 || mb * BM >= M) return;
  const int m0 = mb * BM + wm * 32 * MT;
  const int n32t = (g.n + 31) >> 5;
  const int ntile0 = (nb * BN >> 5) + wn * NT;
  const int KT = KTC ? KTC : (g.k >> 5);  // K/32 steps; compile-time for K = 192, 768
  const int khalf = (lane >> 5) * 16;

  int arow[MT];
  const int8_t *ap[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    int r = m0 + mt * 32 + (lane & 31);
    r = r < M ? r : M - 1;
    arow[mt] = r;
    if (AMODE != A_PATCH) ap[mt] = a_row<AMODE>(g, r) + khalf;
  }
  const int8_t *bp[NT];
  bool nvalid[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int t = ntile0 + nt;
    nvalid[nt] = t < n32t;
    bp[nt] = g.b + ((size_t)(t < n32t ? t : n32t - 1) * KT) * 1024 + lane * 16;
  }

  v16i acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v16i{0};

  v4i a_cur[MT], b_cur[NT], a_nxt[MT], b_nxt[NT];
  auto load = [&](int kt, v4i *av, v4i *bv) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int8_t *p = AMODE == A_PATCH ? patch_ptr(g.a, arow[mt], kt * 32 + khalf)
                                         : ap[mt] + kt * 32;
      av[mt] = *reinterpret_cast<const v4i *>(p);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bv[nt] = *reinterpret_cast<const v4i *>(bp[nt] + kt * 1024);
  };
  load(0, a_cur, b_cur);
#pragma unroll(KTC ? 6 : 1)
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) load(kt + 1, a_nxt, b_nxt);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur[mt], b_cur[nt], acc[mt][nt],
                                                             0, 0, 0);
    if (kt + 1 < KT) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) a_cur[mt] = a_nxt[mt];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) b_cur[nt] = b_nxt[nt];
    }
  }

  // 32x32 accumulator layout: lane l holds column l%32 and, in element i,
  // row 8*(i/4) + 4*(l/32) + i%4 of the tile.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if (!nvalid[nt]) continue;
    const int col = (ntile0 + nt) * 32 + (lane & 31);
    if (col >= g.n) continue;
    const i64 bias = g.bias ? (i64)g.bias[col] : 0;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = m0 + mt * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (row >= M) continue;
        const i64 v = (i64)acc[mt][nt][i] + bias;
        if (EPI == EPI_I32) {
          reinterpret_cast<int32_t *>(g.c)[(size_t)row * g.ldc + col] =
              (int32_t)requant_shift(v, g.shift_a, 32);
        } else if (EPI == EPI_I8) {
          reinterpret_cast<int8_t *>(g.c)[(size_t)row * g.ldc + col] =
              (int8_t)requant_shift(v, g.shift_a, 8);
        } else if (EPI == EPI_GELU) {
          reinterpret_cast<int8_t *>(g.c)[(size_t)row * g.ldc + col] =
              (int8_t)gelu_post(v, g.shift_a, g.shift_b);
        } else if (EPI == EPI_RES) {
          const int t = (int)requant_shift(v, g.shift_a, 8);
          if (g.aux) g.aux[(size_t)row * g.ldc + col] = (int8_t)t;
          const int r = g.res[(size_t)row * g.ldr + col];
          reinterpret_cast<int8_t *>(g.c)[(size_t)row * g.ldc + col] =
              (int8_t)align_add_i8(r, g.res_exp, t, g.mid_exp, g.out_exp);
        } else {  // EPI_PATCH
          const int t = (int)requant_shift(v, g.shift_a, 8);
          const int b = row / kPatchesPerImage, p = row - b * kPatchesPerImage;
          const int pos = g.pos[(size_t)(p + 1) * 192 + col];
          reinterpret_cast<int8_t *>(g.c)[((size_t)b * kTokens + 1 + p) * g.ldc + col] =
              (int8_t)align_add_i8(t, g.mid_exp, pos, g.res_exp, g.out_exp);
        }
      }
    }
  }
}

template <int MT, int NT, int EPI, int AMODE, int KTC = 0>
static int run(const GemmArgs &g, hipStream_t s) {
  constexpr int BM = 64 * MT, BN = 64 * NT;
  const int n_blocks = (g.n + BN - 1) / BN;
  const long long m_blocks = (g.m + BM - 1) / BM;
  const long long grid = m_blocks * n_blocks;
  if (grid <= 0) return HV_OK;
  if (grid > 0x7fffffff) return fail(HV_EVALUE, "gemm grid too large");
  hipLaunchKernelGGL((k_gemm<MT, NT, EPI, AMODE, KTC>), dim3((unsigned)grid), dim3(256), 0, s,
                     g, n_blocks);
  return check_hip(hipGetLastError(), "k_gemm launch");
}

// Tile choice: N that is a multiple of 192 (QKV 576, FFN1 768, proj/FFN2
// 192) uses 192-wide column blocks; other N (head 1000, tests) 128-wide.
// Large-N GEMMs use 128-row tiles, N = 192 GEMMs 64-row tiles so the grid
// still fills 256 CUs.
template <int EPI, int AMODE, int KTC>
static int dispatch_tiles(const GemmArgs &g, hipStream_t s) {
  // The GELU epilogue needs more registers; 128x128 tiles keep it spill-free.
  if (EPI == EPI_GELU && g.n > 192) return run<2, 2, EPI, AMODE, KTC>(g, s);
  if (g.n % 192 == 0) {
    if (g.n > 192) return run<2, 3, EPI, AMODE, KTC>(g, s);
    return run<1, 3, EPI, AMODE, KTC>(g, s);
  }
  return run<1, 2, EPI, AMODE, KTC>(g, s);
}

// K = 192 (every GEMM but FFN2) and K = 768 (FFN2) get compile-time trip
// counts; other K (tests, tails) take the runtime loop.
template <int EPI>
static int dispatch_k(const GemmArgs &g, int a_mode, hipStream_t s) {
  if (a_mode == A_GATHER) return dispatch_tiles<EPI, A_GATHER, 0>(g, s);
  if (a_mode != A_ROWS) return fail(HV_EVALUE, "gemm: bad A mode %d", a_mode);
  if (g.k == 192) return dispatch_tiles<EPI, A_ROWS, 6>(g, s);
  if (g.k == 768) return dispatch_tiles<EPI, A_ROWS, 24>(g, s);
  return dispatch_tiles<EPI, A_ROWS, 0>(g, s);
}

int launch_gemm(const GemmArgs &g, int a_mode, int epi, hipStream_t s) {
  if (g.k <= 0 || g.k % 32) return fail(HV_EVALUE, "gemm: K=%d must be a positive multiple of 32", g.k);
  if (g.n <= 0) return fail(HV_EVALUE, "gemm: N=%d must be positive", g.n);
  if (g.m < 0) return fail(HV_EVALUE, "gemm: M=%d must be non-negative", g.m);
  if (a_mode != A_PATCH && (g.lda % 16 || ((uintptr_t)g.a & 15)))
    return fail(HV_EVALUE, "gemm: A must be 16-byte aligned with lda %% 16 == 0");
  if (g.k > 131071) return fail(HV_EOVERFLOW, "gemm: K=%d may overflow int32", g.k);
  switch (epi) {
    case EPI_I8: return dispatch_k<EPI_I8>(g, a_mode, s);
    case EPI_I32: return dispatch_k<EPI_I32>(g, a_mode, s);
    case EPI_GELU: return dispatch_k<EPI_GELU>(g, a_mode, s);
    case EPI_RES: return dispatch_k<EPI_RES>(g, a_mode, s);
    default: return fail(HV_EVALUE, "gemm: bad epilogue %d", epi);
  }
}

// CLS rows: row b*197 = align_add(cls @ cls_exp, pos[0] @ pos_exp -> tokens)
// (transformer.py:127-135).
__global__ void k_cls_rows(const int8_t *cls, const int8_t *pos, int8_t *x, int cls_exp,
                           int pos_exp, int tokens_exp) {
  const int b = blockIdx.x, c = threadIdx.x;
  if (c < 192)
    x[(size_t)b * kTokens * 192 + c] =
        (int8_t)align_add_i8(cls[c], cls_exp, pos[c], pos_exp, tokens_exp);
}

int launch_patch_embed(const hv_patch_dev &p, const int8_t *images, int batch, int8_t *x,
                       hipStream_t s) {
  if (batch <= 0) return HV_OK;
  if ((uintptr_t)images & 15) return fail(HV_EVALUE, "patch: images must be 16-byte aligned");
  GemmArgs g{};
  g.a = images;
  g.b = p.weight_p;
  g.bias = p.bias;
  g.c = x;
  g.pos = p.pos;
  g.m = batch * kPatchesPerImage;
  g.n = 192;
  g.k = 768;
  g.ldc = 192;
  g.shift_a = p.activation_exp - (p.image_exp + p.weight_exp);
  g.mid_exp = p.activation_exp;
  g.res_exp = p.pos_exp;
  g.out_exp = p.tokens_exp;
  int rc = run<1, 3, EPI_PATCH, A_PATCH, 24>(g, s);
  if (rc) return rc;
  hipLaunchKernelGGL(k_cls_rows, dim3(batch), dim3(192), 0, s, p.cls, p.pos, x, p.cls_exp,
                     p.pos_exp, p.tokens_exp);
  return check_hip(hipGetLastError(), "k_cls_rows launch");
}

}  // namespace hv
