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
static constexpr long long kGridCap = 256 * 8;  // workgroups: 256 CUs x 8 resident
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
  constexpr int BM = 64 * MT, BN = 64 * NT;
  const int live_tiles = ((M + BM - 1) / BM) * n_blocks;
  // Grid-stride over output tiles: the grid is sized for the chip, not for
  // the largest possible M, so pruned batches launch no idle workgroups.
  for (int tile_id = blockIdx.x; tile_id < live_tiles; tile_id += gridDim.x) {
  const int nb = tile_id % n_blocks, mb = tile_id / n_blocks;
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
  auto step = [&](int kt) {
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
  };
  load(0, a_cur, b_cur);
  if constexpr (KTC > 0) {
#pragma unroll
    for (int kt = 0; kt < KTC; ++kt) step(kt);
  } else {
    for (int kt = 0; kt < KT; ++kt) step(kt);
  }

  // Epilogue.  Each wavefront stages one 32x32 int32 accumulator tile at a
  // time in its LDS slice (MFMA layout: lane l holds column l%32 and, in
  // element i, row 8*(i/4) + 4*(l/32) + i%4), then lane l finishes row l/2,
  // columns 16*(l%2) + 4*g .. +3 for g = 0..3: four outputs per group with
  // one bias/residual vector load and one packed store.  With |acc| <=
  // K*2^14 and |bias| <= acc_lim, v = acc + bias stays below 2^30 and the
  // epilogue's requants are exact in int32 (requant_i32); other columns take
  // the 64-bit forms.
  __shared__ int stage[4][32 * 36];
  int *T = stage[wave];
  const int er = lane >> 1, ec0 = (lane & 1) * 16;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        T[(8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) * 36 + (lane & 31)] = acc[mt][nt][i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int row = m0 + mt * 32 + er;
      if (nvalid[nt] && row < M) {
#pragma unroll 1
        for (int grp = 0; grp < 4; ++grp) {
          const int cl = ec0 + 4 * grp;
          const int col = (ntile0 + nt) * 32 + cl;
          if (col >= g.n) break;
          const v4i a4 = *reinterpret_cast<const v4i *>(&T[er * 36 + cl]);
          const bool full = col + 3 < g.n;
          int bias[4] = {0, 0, 0, 0};
          if (g.bias) {
            if (full && (g.n & 3) == 0) {
              const v4i b4 = *reinterpret_cast<const v4i *>(g.bias + col);
              bias[0] = b4[0]; bias[1] = b4[1]; bias[2] = b4[2]; bias[3] = b4[3];
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j) bias[j] = col + j < g.n ? g.bias[col + j] : 0;
            }
          }
          int rv[4] = {0, 0, 0, 0};
          if (EPI == EPI_RES) {
            const int8_t *rp = g.res + (size_t)row * g.ldr + col;
#pragma unroll
            for (int j = 0; j < 4; ++j) rv[j] = col + j < g.n ? rp[j] : 0;
          }
          size_t orow = (size_t)row;
          if (EPI == EPI_PATCH) {
            const int b = row / kPatchesPerImage, p = row - b * kPatchesPerImage;
            orow = (size_t)b * kTokens + 1 + p;
            const int8_t *pp = g.pos + (size_t)(p + 1) * 192 + col;
#pragma unroll
            for (int j = 0; j < 4; ++j) rv[j] = pp[j];
          }
          int out[4], aux[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool n32 = g.narrow_ok && bias[j] <= g.acc_lim && bias[j] >= -g.acc_lim;
            const int v32 = a4[j] + (n32 ? bias[j] : 0);
            const i64 v = (i64)a4[j] + bias[j];
            if (EPI == EPI_I32) {
              out[j] = (int)requant_shift(v, g.shift_a, 32);
            } else if (EPI == EPI_I8) {
              out[j] = n32 ? requant_i32(v32, g.shift_a, -128, 127)
                           : (int)requant_shift(v, g.shift_a, 8);
            } else if (EPI == EPI_GELU) {
              if (n32) {
                const int q = requant_i32(v32, g.shift_a, -(1 << 23), (1 << 23) - 1);
                out[j] = requant_i32(gelu_q16(q), g.shift_b, -128, 127);
              } else {
                out[j] = gelu_post(v, g.shift_a, g.shift_b);
              }
            } else {  // EPI_RES, EPI_PATCH
              const int t = n32 ? requant_i32(v32, g.shift_a, -128, 127)
                                : (int)requant_shift(v, g.shift_a, 8);
              aux[j] = t;
              out[j] = EPI == EPI_RES ? align_add_pre(rv[j], t, g.da, g.db, g.os, n32)
                                      : align_add_pre(t, rv[j], g.da, g.db, g.os, n32);
            }
          }
          if (EPI == EPI_I32) {
            int32_t *cp = reinterpret_cast<int32_t *>(g.c) + orow * g.ldc + col;
            if (full && ((g.ldc & 3) == 0)) {
              *reinterpret_cast<v4i *>(cp) = v4i{out[0], out[1], out[2], out[3]};
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j)
                if (col + j < g.n) cp[j] = out[j];
            }
          } else {
            int8_t *cp = reinterpret_cast<int8_t *>(g.c) + orow * g.ldc + col;
            const int word = (out[0] & 0xFF) | ((out[1] & 0xFF) << 8) | ((out[2] & 0xFF) << 16) |
                             ((out[3] & 0xFF) << 24);
            if (full && ((g.ldc & 3) == 0)) {
              *reinterpret_cast<int *>(cp) = word;
            } else {
#pragma unroll
              for (int j = 0; j < 4; ++j)
                if (col + j < g.n) cp[j] = (int8_t)out[j];
            }
            if (EPI == EPI_RES && g.aux) {
              int8_t *xp = g.aux + (size_t)row * g.ldc + col;
              const int aw = (aux[0] & 0xFF) | ((aux[1] & 0xFF) << 8) | ((aux[2] & 0xFF) << 16) |
                             ((aux[3] & 0xFF) << 24);
              if (full && ((g.ldc & 3) == 0)) {
                *reinterpret_cast<int *>(xp) = aw;
              } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                  if (col + j < g.n) xp[j] = (int8_t)aux[j];
              }
            }
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  }  // tile loop
}

// Shared host-side set-up of the int32 epilogue preconditions.
void epilogue_limits_pub(GemmArgs &g, int epi) {
  const long long acc_max = (long long)g.k * 128 * 128;  // |A W| bound (int8 x int8)
  const long long lim = (1ll << 30) - 1 - acc_max;
  g.acc_lim = lim > 0 ? (int)lim : -1;
  g.narrow_ok = 1;
  if (epi == EPI_RES || epi == EPI_PATCH) {
    // residual: align_add(res @ res_exp, t @ mid_exp -> out_exp);
    // patch:    align_add(t @ mid_exp, pos @ res_exp -> out_exp)
    const int a_exp = epi == EPI_RES ? g.res_exp : g.mid_exp;
    const int b_exp = epi == EPI_RES ? g.mid_exp : g.res_exp;
    const int c = a_exp < b_exp ? a_exp : b_exp;
    g.da = a_exp - c;
    g.db = b_exp - c;
    g.os = g.out_exp - c;
    g.narrow_ok = g.da <= 21 && g.db <= 21;
  }
}

template <int MT, int NT, int EPI, int AMODE, int KTC = 0>
static int run(const GemmArgs &g, hipStream_t s) {
  constexpr int BM = 64 * MT, BN = 64 * NT;
  const int n_blocks = (g.n + BN - 1) / BN;
  const long long m_blocks = (g.m + BM - 1) / BM;
  long long grid = m_blocks * n_blocks;
  if (grid <= 0) return HV_OK;
  if (grid > kGridCap) grid = kGridCap;
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

int launch_gemm(const GemmArgs &g_in, int a_mode, int epi, hipStream_t s) {
  GemmArgs g = g_in;
  epilogue_limits_pub(g, epi);
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
  g.lda = 0;
  int rc = launch_block_gemm(BG_PATCH, g, nullptr, s);
  if (rc) return rc;
  hipLaunchKernelGGL(k_cls_rows, dim3(batch), dim3(192), 0, s, p.cls, p.pos, x, p.cls_exp,
                     p.pos_exp, p.tokens_exp);
  return check_hip(hipGetLastError(), "k_cls_rows launch");
}

}  // namespace hv
