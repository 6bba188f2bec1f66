// hv_gemm_p.hip -- persistent int8 GEMM for the per-token GEMMs of the
// block (QKV, proj, FFN1, FFN2) and the patch embedding, with an optional
// fused LayerNorm prologue (nonlinear.layernorm on the A rows, which turns
// LN1 -> QKV and LN2 -> FFN1 into one launch each).
//
// Workgroup: NW wavefronts side by side along N; wavefront w owns NT
// column tiles of 32 and all 32*MT rows of the current row tile.  Its B
// fragments (NT x K/32 of the "mfma32" packed weights, 16 bytes per lane
// each) are loaded once into registers and reused for every row tile the
// workgroup visits.  The workgroups stride over row tiles (grid = column
// blocks x row groups), so a pruned batch with few live rows does not pay
// for empty workgroups; the live row count is read from the device.  The A
// row tile is staged in LDS (row stride K+16, conflict-free fragment reads)
// with coalesced 16-byte loads, the next tile's loads are in flight while
// the current one is multiplied, and the epilogue stages each 32x32 int32
// accumulator tile through a per-wavefront LDS slice (see hv_gemm.hip for
// the epilogue semantics).
#include "hv_device.h"
#include "hv_internal.h"

namespace hv {

enum { P_EPI_I8 = HV_EPI_I8, P_EPI_GELU = HV_EPI_GELU, P_EPI_RES = HV_EPI_RESIDUAL,
       P_EPI_PATCH = 4 };

static constexpr int kPPatches = 196;
static constexpr int kPTokens = 197;
static constexpr int kPImage = 224 * 224 * 3;

__device__ __forceinline__ const int8_t *p_patch_ptr(const int8_t *images, int r, int k) {
  const int b = r / kPPatches, p = r - b * kPPatches;
  const int pr = p / 14, pc = p - pr * 14;
  const int in_row = k / 48, rem = k - in_row * 48;
  return images + (size_t)b * kPImage + ((pr * 16 + in_row) * 224 + pc * 16) * 3 + rem;
}

// LayerNorm of one 192-byte row held in LDS, by a group of 16 lanes
// (12 channels each), in place.  Same arithmetic as k_layernorm.
__device__ __forceinline__ void ln_row_lds(int8_t *row, int sub, const LnArgs &ln) {
  int *w = reinterpret_cast<int *>(row) + sub * 3;
  int xv[12];
#pragma unroll
  for (int j = 0; j < 12; ++j) xv[j] = (int)(int8_t)(w[j >> 2] >> (8 * (j & 3)));
  const int sh = ln.x_exp + 32;
  const int sq_shift = -(2 * ln.x_exp + 32);
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
  if (var < 0) var = 0;
  const u64 std_q16 = isqrt_u64((u64)var + 4295u);
  const i64 inv = round_div_pos(1ll << 48, (i64)std_q16);
  const u64 inv_hi = (u64)inv >> 24, inv_lo = (u64)inv & 0xFFFFFFull;
  const int c0 = sub * 12;
  int out[3] = {0, 0, 0};
#pragma unroll
  for (int j = 0; j < 12; ++j) {
    const i64 d = (i64)xv[j] * (1ll << sh) - mean;
    i64 norm;
    if (ln.fast_norm) {
      const u64 ad = d < 0 ? (u64)(-d) : (u64)d;
      const u64 r = (ad * inv_hi + ((ad * inv_lo + (1ull << 47)) >> 24)) >> 24;
      if (d < 0) norm = r > (1ull << 23) ? -(1ll << 23) : -(i64)r;
      else norm = r > (1ull << 23) - 1 ? (1ll << 23) - 1 : (i64)r;
    } else {
      norm = sat128(rsa128((i128)d * inv, 48), 24);
    }
    const int c = c0 + j;
    int o;
    if (ln.fast_align) {
      const i64 al = (norm * ln.gamma[c]) * (1ll << ln.gs) + (i64)ln.beta[c] * (1ll << ln.bs);
      o = (int)requant_shift(al, ln.os, 8);
    } else {
      const i128 al = (i128)(norm * ln.gamma[c]) * ((i128)1 << ln.gs) +
                      (i128)ln.beta[c] * ((i128)1 << ln.bs);
      o = (int)requant128(al, ln.os, 8);
    }
    out[j >> 2] |= (o & 0xFF) << (8 * (j & 3));
  }
  w[0] = out[0];
  w[1] = out[1];
  w[2] = out[2];
}

template <int NW, int NT, int MT, int KT, int EPI, int AMODE, bool LNP>
__global__ __launch_bounds__(NW * 64) void k_gemm_p(GemmArgs g, LnArgs ln, int n_blocks) {
  constexpr int K = KT * 32, LDA = K + 16, BM = MT * 32;
  constexpr int THREADS = NW * 64;
  constexpr int CHUNKS = BM * K / 16;                       // 16-byte A chunks per tile
  constexpr int CPT = (CHUNKS + THREADS - 1) / THREADS;     // chunks per thread
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];
  int8_t *At = lds;                                          // [BM][LDA]
  int *stage = reinterpret_cast<int *>(lds + BM * LDA);      // [NW][32][36]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = g.m_dev ? min(*g.m_dev, g.m) : g.m;
  const int n_tiles = (M + BM - 1) / BM;
  const int nb = blockIdx.x % n_blocks;
  const int groups = gridDim.x / n_blocks;
  int tile = blockIdx.x / n_blocks;
  if (M <= 0 || tile >= n_tiles) return;

  const int n32t = (g.n + 31) >> 5;
  const int ntile0 = nb * NW * NT + wave * NT;
  v4i bfrag[NT][KT];
  bool nvalid[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int t = ntile0 + nt;
    nvalid[nt] = t < n32t;
    const int8_t *bp = g.b + ((size_t)(t < n32t ? t : n32t - 1) * KT) * 1024 + lane * 16;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) bfrag[nt][kt] = *reinterpret_cast<const v4i *>(bp + kt * 1024);
  }

  v4i pre[CPT];
  auto load_tile = [&](int t) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = tid + c * THREADS;
      if (ch < CHUNKS) {
        const int r = ch / (K / 16), k16 = ch - r * (K / 16);
        int row = t * BM + r;
        row = row < M ? row : M - 1;
        const int8_t *src = AMODE == A_PATCH ? p_patch_ptr(g.a, row, k16 * 16)
                                             : g.a + (size_t)row * g.lda + k16 * 16;
        pre[c] = *reinterpret_cast<const v4i *>(src);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = tid + c * THREADS;
      if (ch < CHUNKS) {
        const int r = ch / (K / 16), k16 = ch - r * (K / 16);
        *reinterpret_cast<v4i *>(At + r * LDA + k16 * 16) = pre[c];
      }
    }
  };

  load_tile(tile);
  int *T = stage + wave * (32 * 36);
  const int er = lane >> 1, ec0 = (lane & 1) * 16;
  for (; tile < n_tiles; tile += groups) {
    __syncthreads();  // the previous tile's fragments have been read
    store_tile();
    __syncthreads();
    const int next = tile + groups;
    if (next < n_tiles) load_tile(next);
    if constexpr (LNP) {
      // LayerNorm prologue: groups of 16 lanes normalise the staged rows in place.
      const int sub = tid & 15;
      for (int r = tid >> 4; r < BM; r += THREADS / 16) {
        const int row = tile * BM + r;
        if (row < M) {
          ln_row_lds(At + r * LDA, sub, ln);
          if (ln.out) {
            const int *src = reinterpret_cast<const int *>(At + r * LDA) + sub * 3;
            int *dst = reinterpret_cast<int *>(ln.out + (size_t)row * 192) + sub * 3;
            dst[0] = src[0]; dst[1] = src[1]; dst[2] = src[2];
          }
        }
      }
      __syncthreads();
    }

    v16i acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v16i{0};
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const v4i af = *reinterpret_cast<const v4i *>(At + (mt * 32 + (lane & 31)) * LDA + kt * 32 +
                                                      (lane >> 5) * 16);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bfrag[nt][kt], acc[mt][nt], 0, 0, 0);
      }
    }

    // Epilogue, one 32x32 tile at a time through the wavefront's LDS slice.
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
        const int row = tile * BM + mt * 32 + er;
        if (nvalid[nt] && row < M) {
#pragma unroll 1
          for (int grp = 0; grp < 4; ++grp) {
            const int cl = ec0 + 4 * grp;
            const int col = (ntile0 + nt) * 32 + cl;
            if (col >= g.n) break;
            const v4i a4 = *reinterpret_cast<const v4i *>(&T[er * 36 + cl]);
            const v4i b4 = g.bias ? *reinterpret_cast<const v4i *>(g.bias + col) : v4i{0};
            int rv[4] = {0, 0, 0, 0};
            size_t orow = (size_t)row;
            if (EPI == P_EPI_RES) {
              const int w = *reinterpret_cast<const int *>(g.res + (size_t)row * g.ldr + col);
#pragma unroll
              for (int j = 0; j < 4; ++j) rv[j] = (int)(int8_t)(w >> (8 * j));
            }
            if (EPI == P_EPI_PATCH) {
              const int b = row / kPPatches, p = row - b * kPPatches;
              orow = (size_t)b * kPTokens + 1 + p;
              const int w = *reinterpret_cast<const int *>(g.pos + (size_t)(p + 1) * 192 + col);
#pragma unroll
              for (int j = 0; j < 4; ++j) rv[j] = (int)(int8_t)(w >> (8 * j));
            }
            int word = 0, aword = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int bias = b4[j];
              const bool n32 = g.narrow_ok && bias <= g.acc_lim && bias >= -g.acc_lim;
              const int v32 = a4[j] + (n32 ? bias : 0);
              const i64 v = (i64)a4[j] + bias;
              int o;
              if (EPI == P_EPI_I8) {
                o = n32 ? requant_i32(v32, g.shift_a, -128, 127) : (int)requant_shift(v, g.shift_a, 8);
              } else if (EPI == P_EPI_GELU) {
                if (n32) {
                  const int q = requant_i32(v32, g.shift_a, -(1 << 23), (1 << 23) - 1);
                  o = requant_i32(gelu_q16(q), g.shift_b, -128, 127);
                } else {
                  o = gelu_post(v, g.shift_a, g.shift_b);
                }
              } else {
                const int t = n32 ? requant_i32(v32, g.shift_a, -128, 127)
                                  : (int)requant_shift(v, g.shift_a, 8);
                aword |= (t & 0xFF) << (8 * j);
                o = EPI == P_EPI_RES ? align_add_pre(rv[j], t, g.da, g.db, g.os, n32)
                                     : align_add_pre(t, rv[j], g.da, g.db, g.os, n32);
              }
              word |= (o & 0xFF) << (8 * j);
            }
            *reinterpret_cast<int *>(reinterpret_cast<int8_t *>(g.c) + orow * g.ldc + col) = word;
            if (EPI == P_EPI_RES && g.aux)
              *reinterpret_cast<int *>(g.aux + (size_t)row * g.ldc + col) = aword;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
  }
}

static int g_num_cus = 0;

static int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_num_cus = n;
    else
      g_num_cus = 256;
  }
  return g_num_cus;
}

template <int NW, int NT, int MT, int KT, int EPI, int AMODE, bool LNP>
static int run_p(const GemmArgs &g, const LnArgs &ln, int wgs_per_cu, hipStream_t s) {
  constexpr int BM = MT * 32, K = KT * 32, BN = NW * NT * 32;
  const int n_blocks = (g.n + BN - 1) / BN;
  const int tiles = (g.m + BM - 1) / BM;
  if (tiles <= 0) return HV_OK;
  // Row groups: enough workgroups to fill the chip, tiles shared evenly.
  int target = (num_cus() * wgs_per_cu + n_blocks - 1) / n_blocks;
  if (target < 1) target = 1;
  const int per = (tiles + target - 1) / target;
  const int groups = (tiles + per - 1) / per;
  const size_t lds = (size_t)BM * (K + 16) + (size_t)NW * 32 * 36 * 4;
  auto kern = k_gemm_p<NW, NT, MT, KT, EPI, AMODE, LNP>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return fail(HV_EHIP, "gemm_p: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(n_blocks * groups), dim3(NW * 64), lds, s, g, ln, n_blocks);
  return check_hip(hipGetLastError(), "k_gemm_p launch");
}

void ln_args_setup(LnArgs &ln) {
  const int common = (ln.g_exp - 16) < ln.b_exp ? (ln.g_exp - 16) : ln.b_exp;
  ln.gs = ln.g_exp - 16 - common;
  ln.bs = ln.b_exp - common;
  ln.os = ln.out_exp - common;
  ln.fast_norm = ln.x_exp <= -1;
  ln.fast_align = ln.gs <= 30 && ln.bs <= 54;
}

int launch_block_gemm(int which, const GemmArgs &g_in, const LnArgs *ln_in, hipStream_t s) {
  GemmArgs g = g_in;
  LnArgs ln{};
  if (ln_in) {
    ln = *ln_in;
    if (ln.x_exp < -32 || ln.x_exp > 0)
      return fail(HV_EVALUE, "layernorm input scale must be in [-32, 0] (got %d)", ln.x_exp);
    ln_args_setup(ln);
  }
  if (((uintptr_t)g.a & 15) || (g.lda & 15) || ((uintptr_t)g.c & 3) || (g.ldc & 3) ||
      ((uintptr_t)g.bias & 15) || (g.n & 3))
    return fail(HV_EVALUE, "gemm_p: misaligned operands");
  if (g.m <= 0) return HV_OK;
  switch (which) {
    case BG_QKV:
      epilogue_limits_pub(g, P_EPI_I8);
      return ln_in ? run_p<6, 3, 2, 6, P_EPI_I8, A_ROWS, true>(g, ln, 1, s)
                   : run_p<6, 3, 2, 6, P_EPI_I8, A_ROWS, false>(g, ln, 1, s);
    case BG_FFN1:
      epilogue_limits_pub(g, P_EPI_GELU);
      return ln_in ? run_p<8, 3, 2, 6, P_EPI_GELU, A_ROWS, true>(g, ln, 1, s)
                   : run_p<8, 3, 2, 6, P_EPI_GELU, A_ROWS, false>(g, ln, 1, s);
    case BG_PROJ:
      epilogue_limits_pub(g, P_EPI_RES);
      return run_p<6, 1, 4, 6, P_EPI_RES, A_ROWS, false>(g, ln, 1, s);
    case BG_FFN2:
      epilogue_limits_pub(g, P_EPI_RES);
      return run_p<6, 1, 2, 24, P_EPI_RES, A_ROWS, false>(g, ln, 1, s);
    case BG_PATCH:
      epilogue_limits_pub(g, P_EPI_PATCH);
      return run_p<6, 1, 2, 24, P_EPI_PATCH, A_PATCH, false>(g, ln, 1, s);
    default:
      return fail(HV_EVALUE, "gemm_p: unknown GEMM %d", which);
  }
}

}  // namespace hv
