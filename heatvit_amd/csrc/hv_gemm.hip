// hv_gemm.hip -- int8 GEMM on CDNA4 MFMA with the golden model's fused
// writebacks (gemm.gemm_numpy + gemm.gemm_writeback, gemm.py:93-139).
//
// Orientation: every wavefront computes C^T tiles, W^T A^T, with
// v_mfma_i32_32x32x32_i8 taking the packed weight fragment as its first
// operand and the activation rows as its second.  The "mfma32" packing
// (include/heatvit_hip.h) permutes the 32 columns of each weight tile so
// that result lane l holds, for token row l%32, the 16 contiguous output
// channels 16*(l/32) .. +15 of the tile.  The whole epilogue therefore runs
// in registers: one 16-byte residual load and one 16-byte store per lane
// and tile, four 16-byte bias loads per column tile, no LDS round trip.
// int32 accumulation is exact: |acc| <= K*128*128 < 2^31 for K <= 131071,
// so gemm_numpy's overflow check cannot fire.
//
// Tiling: a 256-thread workgroup is a WM x (4/WM) grid of wavefronts, each
// owning MT x NT 32x32 tiles.  Workgroups stride over the output tiles of
// the live rows (row count read on the device); consecutive tiles of one
// row block (its column blocks) go to the same XCD, so the row block's A
// bytes are fetched into one L2.  For K = 192 all operand fragments of a
// tile are loaded before the first MFMA (one memory latency per tile); for
// K = 768 the loads run in double-buffered chunks of four K steps, and the
// epilogue's bias and residual loads are issued with the first chunk.
//
// Epilogues (per output element v = acc + bias):
//   EPI_I8/I32   requant(v, src, dst, 8|32)                     gemm.py:123-139
//   EPI_GELU     requant(gelu(requant(v, src, -16, 24)), -16, dst, 8)
//                                                    transformer.py:349-358
//   EPI_RESIDUAL t = requant(v, src, mid, 8); out = align_add(res, t)
//                                                    transformer.py:96-101
//   EPI_PATCH    t = requant(v, img+w, act, 8); out = align_add(t, pos[p+1])
//                into row b*197 + 1 + p                transformer.py:120-145
// The GELU epilogue with an output shift so = dst + 16 in [3, 12] looks the
// post-op requant(gelu(q), -16, dst, 8) up in a step table of q instead of
// evaluating it (gen_gelu_lut.py writes the tables and checks each against
// the post-op over the whole 24-bit domain): the table (about 10-13 KB) is
// staged in LDS per workgroup, and one lookup is two LDS reads and a dozen
// integer operations against about forty for the evaluation.
//
// The int32 form of each epilogue is taken when the launch's shifts lie in
// [-30, 30], the align-add shifts are at most 21, and every bias of the
// wavefront's columns satisfies |bias| <= 2^30 - 1 - K*2^14 (so v, the
// aligned sums and every rounding addend stay below 2^31) and, when the
// first requant shifts left by k, |bias| <= ((2^31 - 1) >> k) - K*2^14 (so
// v << k stays inside int32); the other cases call the exact 64/128-bit
// form, kept out of line.
#include <atomic>
#include "hv_device.h"
#include "hv_internal.h"
#include "gelu_lut.inc"  // generated at build time by gen_gelu_lut.py

namespace hv {

enum { EPI_I8 = HV_EPI_I8, EPI_I32 = HV_EPI_I32, EPI_GELU = HV_EPI_GELU,
       EPI_RES = HV_EPI_RESIDUAL, EPI_PATCH = 4 };

static constexpr int kPatchesPerImage = 196;
static constexpr int kTokens = 197;
static constexpr int kImageBytes = 224 * 224 * 3;
// Direct kernel: one workgroup per tile (the grid is not capped), so the
// hardware dispatcher balances the tiles over the resident slots; a capped
// grid with static tile striding left a partial last round per workgroup.
static constexpr int kGridCap = 1 << 20;
static constexpr int kLdsGridCap = 256 * 2;  // LDS-staged kernel: 2 per CU, persistent
// GELU step-table launches: persistent, five workgroups per CU, which the
// 92 VGPRs and the largest table (31 KB of LDS) both allow; each stages the
// table once (two, three, four or eight per CU, or one workgroup per tile,
// were slower)
static constexpr int kLutGridCap = 256 * 5;

template <int AMODE>
__device__ __forceinline__ const int8_t *a_row(const GemmArgs &g, int r) {
  if ((AMODE & 3) == A_GATHER) return g.a + (size_t)g.a_rows[r] * g.lda;
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

// Exact epilogue of one element (64/128-bit), out of line.  Returns
// {output, requantised product (residual forms)}.
typedef int v2i __attribute__((ext_vector_type(2)));
__device__ __noinline__ v2i epi_exact(int epi, int acc, int bias, int res, int shift_a,
                                      int shift_b, int da, int db, int os) {
  const i64 v = (i64)acc + bias;
  if (epi == EPI_I8) return v2i{(int)requant_shift(v, shift_a, 8), 0};
  if (epi == EPI_I32) return v2i{(int)requant_shift(v, shift_a, 32), 0};
  if (epi == EPI_GELU) return v2i{gelu_post(v, shift_a, shift_b), 0};
  const int t = (int)requant_shift(v, shift_a, 8);
  return v2i{epi == EPI_RES ? align_add_pre(res, t, da, db, os, false)
                            : align_add_pre(t, res, da, db, os, false),
             t};
}

// The launch's GELU step table in LDS (gelu_table_u8 in hv_device.h): the
// post-op's int8 value in the low byte.
__device__ __forceinline__ unsigned gelu_lut(int q, const unsigned *lut, int qhi, const GemmArgs &g) {
  return gelu_table_u8(q, lut, g.lut_cb, g.lut_qlo, qhi);
}

// Stages the launch's GELU step table in LDS (all threads, then a barrier).
// Copies the launch's step table into LDS with 16-byte loads, four rounds
// of loads in flight before their LDS writes (one L2 latency per 16 KB, not
// one per word).  Tables start on 16-byte boundaries and hold a multiple of
// four words; blockDim.x is 256.
__device__ __forceinline__ void stage_lut(const GemmArgs &g, unsigned *lut) {
  const v4i *src = reinterpret_cast<const v4i *>(kGeluLut + g.lut_off);
  v4i *dst = reinterpret_cast<v4i *>(lut);
  const int n4 = g.lut_words >> 2;
  for (int base = threadIdx.x; base < n4; base += 1024) {
    v4i v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = src[min(base + r * 256, n4 - 1)];
    // Lanes past the end rewrite the last vector with its own value, so
    // no write is predicated and no load sinks behind one.
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[min(base + r * 256, n4 - 1)] = v[r];
  }
  __syncthreads();
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
  return (int)pack_lo4((unsigned)a, (unsigned)b, (unsigned)c, (unsigned)d);
}


// Epilogue operands that do not depend on the product: the 16 biases of
// each column tile this lane finishes and, for the residual forms, the 16
// residual (or position) bytes of each of its rows.
template <int MT, int NT, int EPI>
__device__ __forceinline__ void epi_operands(const GemmArgs &g, const int (&arow)[MT], int ct0,
                                             int h, v4i (&bias4)[NT][4], v4i (&res4)[MT][NT]) {
  constexpr bool RESLIKE = EPI == EPI_RES || EPI == EPI_PATCH;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int c0 = (ct0 + nt) * 32 + 16 * h;
    if (g.bias && c0 + 16 <= g.n) {
#pragma unroll
      for (int q = 0; q < 4; ++q) bias4[nt][q] = *reinterpret_cast<const v4i *>(g.bias + c0 + 4 * q);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        bias4[nt][j >> 2][j & 3] = g.bias && c0 + j < g.n ? g.bias[c0 + j] : 0;
    }
  }
  if constexpr (RESLIKE) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int c0 = (ct0 + nt) * 32 + 16 * h;
        const int8_t *rp;
        if (EPI == EPI_RES) {
          rp = g.res + (size_t)arow[mt] * g.ldr + c0;
        } else {
          const int p = arow[mt] % kPatchesPerImage;
          rp = g.pos + (size_t)(p + 1) * 192 + c0;
        }
        if (g.vec_res && c0 + 16 <= g.n) {
          res4[mt][nt] = *reinterpret_cast<const v4i *>(rp);
        } else {
          int w[4] = {0, 0, 0, 0};
          for (int j = 0; j < 16 && c0 + j < g.n; ++j) w[j >> 2] |= ((int)rp[j] & 0xFF) << (8 * (j & 3));
          res4[mt][nt] = v4i{w[0], w[1], w[2], w[3]};
        }
      }
  }
}

// Epilogue of one wavefront tile: lane l finishes row r0 + 32*mt + l%32,
// channels c0 .. c0+15 of each column tile.
// lds_out (optional, EPI_RES with 16-byte stores): the output bytes also go
// to lds_out + (32 * mt + l32) * lds_stride + c0.
// BACC: the accumulators started at the bias (the MFMA's C operand), so the
// int32 form adds nothing and the exact form takes the bias back out.
template <int MT, int NT, int EPI, bool FAST, int DIRS, bool BACC = false>
__device__ __forceinline__ void epi_tile(const GemmArgs &g, const v16i (&acc)[MT][NT],
                                         const v4i (&bias4)[NT][4], const v4i (&res4)[MT][NT],
                                         int r0, int ct0, int M, int h, int l32, const Rq &rq_a,
                                         const Rq &rq_b, const unsigned *lut,
                                         int8_t *lds_out = nullptr, int lds_stride = 0) {
  constexpr bool RESLIKE = EPI == EPI_RES || EPI == EPI_PATCH;
  // the table's upper clamp in a vector register: with both bounds in
  // scalar registers the clamp cannot be a single med3
  int qhi = g.lut_qhi;
  if constexpr (EPI == EPI_GELU && (DIRS & 4)) asm("" : "+v"(qhi));
  const bool all_narrow = FAST && tensor_narrow(g.bias_max, g.acc_lim);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int c0 = (ct0 + nt) * 32 + 16 * h;
    // Uniform per wavefront: the int32 form only when every lane qualifies
    // (the whole tensor, or a vote over the lanes' 16 biases each).
    bool fast = all_narrow;
    if (FAST && !all_narrow) {
      int bmax = bias4[nt][0][0], bmin = bmax;
#pragma unroll
      for (int j = 1; j < 16; ++j) {
        bmax = max(bmax, bias4[nt][j >> 2][j & 3]);
        bmin = min(bmin, bias4[nt][j >> 2][j & 3]);
      }
      fast = __all(bmax <= g.acc_lim && bmin >= -g.acc_lim);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = r0 + mt * 32 + l32;
      if (row >= M || c0 >= g.n) continue;
      size_t orow = (size_t)row;
      if (EPI == EPI_PATCH) {
        const int b = row / kPatchesPerImage;
        orow = (size_t)b * kTokens + 1 + (row - b * kPatchesPerImage);
      }
      int o[16], mid[16];
      if (fast) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int v = BACC ? acc[mt][nt][j] : acc[mt][nt][j] + bias4[nt][j >> 2][j & 3];
          constexpr bool LA = DIRS & 1, LB = (DIRS >> 1) & 1;
          if (EPI == EPI_I8) {
            o[j] = rq_dir_nowrap<LA>(v, rq_a);
          } else if (EPI == EPI_I32) {
            // |acc + bias| < 2^30 and a left shift stays inside int32 (the
            // acc_lim bound): the int32 requant needs no saturation
            o[j] = shift_nowrap<LA>(v, rq_a);
          } else if (EPI == EPI_GELU && (DIRS & 4)) {
            // the table's clamp [qlo, qhi] lies inside the 24-bit range
            o[j] = (int)gelu_lut(shift_nowrap<LA>(v, rq_a), lut, qhi, g);
          } else if (EPI == EPI_GELU) {
            o[j] = rq_dir<LB>(gelu_q16(rq_dir_nowrap<LA>(v, rq_a)), rq_b);
          } else if (RESLIKE) {
            const int t8 = rq_dir_nowrap<LA>(v, rq_a);
            const int r8 = (int)(int8_t)(res4[mt][nt][j >> 2] >> (8 * (j & 3)));
            const int s = EPI == EPI_RES ? r8 * (1 << g.da) + t8 * (1 << g.db)
                                         : t8 * (1 << g.da) + r8 * (1 << g.db);
            mid[j] = t8;
            o[j] = rq_dir<LB>(s, rq_b);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int r8 = RESLIKE ? (int)(int8_t)(res4[mt][nt][j >> 2] >> (8 * (j & 3))) : 0;
          const int b = bias4[nt][j >> 2][j & 3];
          const v2i r = epi_exact(EPI, BACC ? acc[mt][nt][j] - b : acc[mt][nt][j], b, r8,
                                  g.shift_a, g.shift_b, g.da, g.db, g.os);
          o[j] = r[0];
          mid[j] = r[1];
        }
      }
      const bool full = g.vec_out && c0 + 16 <= g.n;
      if (EPI == EPI_I32) {
        int32_t *cp = reinterpret_cast<int32_t *>(g.c) + orow * g.ldc + c0;
        if (full) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<v4i *>(cp + 4 * q) = v4i{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (c0 + j < g.n) cp[j] = o[j];
        }
      } else {
        int8_t *cp = reinterpret_cast<int8_t *>(g.c) + orow * g.ldc + c0;
        if (full) {
          const v4i ov = v4i{pack4(o[0], o[1], o[2], o[3]), pack4(o[4], o[5], o[6], o[7]),
                             pack4(o[8], o[9], o[10], o[11]), pack4(o[12], o[13], o[14], o[15])};
          *reinterpret_cast<v4i *>(cp) = ov;
          if (EPI == EPI_RES && lds_out)
            *reinterpret_cast<v4i *>(lds_out + (32 * mt + l32) * lds_stride + c0) = ov;
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (c0 + j < g.n) cp[j] = (int8_t)o[j];
        }
        if (EPI == EPI_RES && g.aux) {
          int8_t *xp = g.aux + orow * g.ldc + c0;
          if (full) {
            *reinterpret_cast<v4i *>(xp) =
                v4i{pack4(mid[0], mid[1], mid[2], mid[3]), pack4(mid[4], mid[5], mid[6], mid[7]),
                    pack4(mid[8], mid[9], mid[10], mid[11]), pack4(mid[12], mid[13], mid[14], mid[15])};
          } else {
#pragma unroll
            for (int j = 0; j < 16; ++j)
              if (c0 + j < g.n) xp[j] = (int8_t)mid[j];
          }
        }
      }
    }
  }
}

template <int MT, int NT, int WM, int EPI, int AMODE, int KTC, bool FAST, int DIRS>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g, int n_blocks) {
  constexpr int WN = 4 / WM;
  constexpr int BM = 32 * MT * WM;  // rows per tile
  constexpr int BT = NT * WN;       // 32-column weight tiles per tile
  constexpr bool RESLIKE = EPI == EPI_RES || EPI == EPI_PATCH;
  // Unsigned A (runtime K only): the MFMA takes s = u - 128 (the byte with
  // its top bit flipped) and a second MFMA per weight tile, with every A
  // byte -128, accumulates corr = -128 * (column sums of W), so
  // sum(u w) = sum(s w) - corr; both stay below 2^31 for K <= 65536.
  constexpr bool AU = (AMODE & A_UNSIGNED) != 0;
  static_assert(!AU || KTC == 0, "unsigned A uses the runtime-K loop");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave - wm * WN;
  const int h = lane >> 5, l32 = lane & 31;
  const int M = g.m_dev ? min(*g.m_dev, g.m) : g.m;
  if (M <= 0) return;
  const int T = ((M + BM - 1) / BM) * n_blocks;
  const int T8 = (T + 7) >> 3;
  const int KT = KTC ? KTC : (g.k >> 5);
  const int n32t = (g.n + 31) >> 5;
  const Rq rq_a = rq_setup(g.shift_a, EPI == EPI_GELU ? -(1 << 23) : -128,
                           EPI == EPI_GELU ? (1 << 23) - 1 : 127);
  const Rq rq_b = rq_setup(EPI == EPI_GELU ? g.shift_b : g.os, -128, 127);
  extern __shared__ __attribute__((aligned(16))) unsigned lut[];
  if constexpr (EPI == EPI_GELU && (DIRS & 4)) stage_lut(g, lut);

  // The grid is a multiple of 8, so t & 7 (the XCD) is fixed per workgroup
  // and XCD x works through logical tiles [x*T8, (x+1)*T8).
  for (int t = blockIdx.x; t < 8 * T8; t += gridDim.x) {
    const int L = (t & 7) * T8 + (t >> 3);
    if (L >= T) continue;
    const int mb = L / n_blocks, nb = L - mb * n_blocks;
    const int r0 = mb * BM + wm * 32 * MT;
    const int ct0 = nb * BT + wn * NT;

    int arow[MT];
    const int8_t *ap[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = min(r0 + mt * 32 + l32, M - 1);
      arow[mt] = r;
      if (AMODE != A_PATCH) ap[mt] = a_row<AMODE>(g, r) + 16 * h;
    }
    const int8_t *bp[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      bp[nt] = g.b + (size_t)min(ct0 + nt, n32t - 1) * KT * 1024 + lane * 16;

    auto load_a = [&](int mt, int kt) -> v4i {
      const int8_t *p = AMODE == A_PATCH ? patch_ptr(g.a, arow[mt], kt * 32 + 16 * h)
                                         : ap[mt] + kt * 32;
      const v4i v = *reinterpret_cast<const v4i *>(p);
      if constexpr (AU) return v ^ (int)0x80808080;
      return v;
    };
    auto load_b = [&](int nt, int kt) -> v4i {
      return *reinterpret_cast<const v4i *>(bp[nt] + kt * 1024);
    };

    v4i bias4[NT][4], res4[MT][NT];
    epi_operands<MT, NT, EPI>(g, arow, ct0, h, bias4, res4);

    v16i acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v16i{0};

    if constexpr (KTC > 0 && KTC <= 8) {
      // Every fragment of the tile in flight at once.
      v4i af[MT][KTC], bf[NT][KTC];
#pragma unroll
      for (int kt = 0; kt < KTC; ++kt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) af[mt][kt] = load_a(mt, kt);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) bf[nt][kt] = load_b(nt, kt);
      }
#pragma unroll
      for (int kt = 0; kt < KTC; ++kt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[nt][kt], af[mt][kt],
                                                                 acc[mt][nt], 0, 0, 0);
    } else if constexpr (KTC > 8) {
      // Double-buffered chunks of KC steps.
      constexpr int KC = 4, NC = KTC / KC;
      static_assert(KTC % (2 * KC) == 0, "K steps must split into chunk pairs");
      v4i a0[MT][KC], b0[NT][KC], a1[MT][KC], b1[NT][KC];
      auto load_chunk = [&](int c, v4i (*av)[KC], v4i (*bv)[KC]) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) av[mt][j] = load_a(mt, c * KC + j);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) bv[nt][j] = load_b(nt, c * KC + j);
        }
      };
      auto mma_chunk = [&](v4i (*av)[KC], v4i (*bv)[KC]) {
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
              acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv[nt][j], av[mt][j],
                                                                   acc[mt][nt], 0, 0, 0);
      };
      load_chunk(0, a0, b0);
#pragma unroll
      for (int c = 0; c < NC; c += 2) {
        load_chunk(c + 1, a1, b1);
        mma_chunk(a0, b0);
        if (c + 2 < NC) load_chunk(c + 2, a0, b0);
        mma_chunk(a1, b1);
      }
    } else {
      // Runtime K: one step of prefetch.
      v4i ac[MT], bc[NT], an[MT], bn[NT];
      v16i corr[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) corr[nt] = v16i{0};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) ac[mt] = load_a(mt, 0);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) bc[nt] = load_b(nt, 0);
      for (int kt = 0; kt < KT; ++kt) {
        if (kt + 1 < KT) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) an[mt] = load_a(mt, kt + 1);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) bn[nt] = load_b(nt, kt + 1);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bc[nt], ac[mt], acc[mt][nt], 0, 0, 0);
        if constexpr (AU) {
          const v4i m128 = v4i{(int)0x80808080, (int)0x80808080, (int)0x80808080,
                               (int)0x80808080};
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            corr[nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bc[nt], m128, corr[nt], 0, 0, 0);
        }
        if (kt + 1 < KT) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) ac[mt] = an[mt];
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) bc[nt] = bn[nt];
        }
      }
      if constexpr (AU) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[mt][nt] -= corr[nt];
      }
    }

    epi_tile<MT, NT, EPI, FAST, DIRS>(g, acc, bias4, res4, r0, ct0, M, h, l32, rq_a, rq_b, lut);
  }
}

// A staged through LDS: for K = 192*NCH the A tile is brought in by K-chunks
// of 192 bytes (6 MFMA K-steps) with fully coalesced 16-byte loads (12
// threads per row), double-buffered in LDS at a 208-byte row stride
// (conflict-free fragment reads).  The next chunk -- or the next tile's
// first chunk -- and its weight fragments are loaded while the current
// chunk's MFMAs run; one barrier per chunk.
template <int MT, int NT, int WM, int EPI, int AMODE, int KTC, bool FAST, int DIRS>
__global__ __launch_bounds__(256) void k_gemm_lds(GemmArgs g, int n_blocks) {
  constexpr int WN = 4 / WM, BM = 32 * MT * WM, BT = NT * WN;
  constexpr int KC = 6, NCH = KTC / KC, ROW = 208;
  constexpr int PIECES = BM * 12, PPT = PIECES / 256;
  static_assert(KTC % KC == 0 && PIECES % 256 == 0, "tile / K shape");
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave - wm * WN;
  const int h = lane >> 5, l32 = lane & 31;
  const int M = g.m_dev ? min(*g.m_dev, g.m) : g.m;
  if (M <= 0) return;
  const int T = ((M + BM - 1) / BM) * n_blocks;
  const int T8 = (T + 7) >> 3;
  const int n32t = (g.n + 31) >> 5;
  const Rq rq_a = rq_setup(g.shift_a, EPI == EPI_GELU ? -(1 << 23) : -128,
                           EPI == EPI_GELU ? (1 << 23) - 1 : 127);
  const Rq rq_b = rq_setup(EPI == EPI_GELU ? g.shift_b : g.os, -128, 127);
  // The grid is a multiple of 8, so t & 7 (the XCD) is fixed per workgroup;
  // XCD x works through logical tiles [x*T8, (x+1)*T8) in order, so the
  // first out-of-range tile ends the sequence.
  auto logical = [&](int t) { return t < 8 * T8 ? (t & 7) * T8 + (t >> 3) : T; };

  int t = blockIdx.x;
  int L = logical(t);
  if (L >= T) return;

  v4i apre[PPT];
  v4i bcur[NT][KC], bnext[NT][KC];
  auto load_step = [&](int Ls, int c) {
    const int mb = Ls / n_blocks, nb = Ls - mb * n_blocks;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int i = tid + j * 256, pr = i / 12, pc = i - pr * 12;
      const int r = min(mb * BM + pr, M - 1);
      const int8_t *src = AMODE == A_PATCH ? patch_ptr(g.a, r, c * 192 + pc * 16)
                                           : g.a + (size_t)r * g.lda + c * 192 + pc * 16;
      apre[j] = *reinterpret_cast<const v4i *>(src);
    }
    const int ct0 = nb * BT + wn * NT;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int8_t *bp = g.b + ((size_t)min(ct0 + nt, n32t - 1) * KTC + c * KC) * 1024 + lane * 16;
#pragma unroll
      for (int kt = 0; kt < KC; ++kt) bnext[nt][kt] = *reinterpret_cast<const v4i *>(bp + kt * 1024);
    }
  };
  auto tile_rows = [&](int Ls, int (&arow)[MT], int &r0, int &ct0) {
    const int mb = Ls / n_blocks, nb = Ls - mb * n_blocks;
    r0 = mb * BM + wm * 32 * MT;
    ct0 = nb * BT + wn * NT;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) arow[mt] = min(r0 + mt * 32 + l32, M - 1);
  };

  int arow[MT], r0, ct0;
  tile_rows(L, arow, r0, ct0);
  v4i bias4[NT][4], res4[MT][NT];
  epi_operands<MT, NT, EPI>(g, arow, ct0, h, bias4, res4);
  load_step(L, 0);

  // One tile per iteration with its K-chunks unrolled, so the accumulators
  // are not carried around the loop (a loop-carried accumulator was copied
  // between VGPRs and AGPRs at every chunk).  The LDS buffers alternate by
  // chunk; the last chunk prefetches the next tile's first.
  int8_t *Ab = As[0], *An = As[1];
  while (true) {
    v16i acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v16i{0};
    int Ln = L;
    bool more = true;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int j = 0; j < PPT; ++j) {
        const int i = tid + j * 256, pr = i / 12, pc = i - pr * 12;
        *reinterpret_cast<v4i *>(Ab + pr * ROW + pc * 16) = apre[j];
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int kt = 0; kt < KC; ++kt) bcur[nt][kt] = bnext[nt][kt];
      __syncthreads();
      // Next step: the following chunk of this tile or the next tile's first.
      if (c == NCH - 1) {
        Ln = logical(t + (int)gridDim.x);
        more = Ln < T;
        if (more) load_step(Ln, 0);
      } else {
        load_step(L, c + 1);
      }
#pragma unroll
      for (int kt = 0; kt < KC; ++kt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const v4i af = *reinterpret_cast<const v4i *>(Ab + (wm * 32 * MT + mt * 32 + l32) * ROW +
                                                        kt * 32 + 16 * h);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bcur[nt][kt], af, acc[mt][nt], 0, 0, 0);
        }
      int8_t *tmp = Ab;
      Ab = An;
      An = tmp;
    }
    epi_tile<MT, NT, EPI, FAST, DIRS>(g, acc, bias4, res4, r0, ct0, M, h, l32, rq_a, rq_b,
                                      nullptr);
    if (!more) break;
    t += gridDim.x;
    L = Ln;
    tile_rows(L, arow, r0, ct0);
    epi_operands<MT, NT, EPI>(g, arow, ct0, h, bias4, res4);
  }
}

// Host-side set-up of the epilogue preconditions.
void epilogue_limits_pub(GemmArgs &g, int epi) {
  // |A W| bound: int8 x int8, or uint8 x int8
  const long long acc_max = (long long)g.k * (g.a_unsigned ? 255 : 128) * 128;
  long long lim = (1ll << 30) - 1 - acc_max;
  if (g.shift_a < 0) {
    // the first requant shifts v = acc + bias left by -shift_a: keep that
    // shift inside int32
    const int sl = -g.shift_a;
    const long long lim_l = sl >= 31 ? -1 : (((1ll << 31) - 1) >> sl) - acc_max;
    lim = lim < lim_l ? lim : lim_l;
  }
  g.acc_lim = lim > 0 ? (int)lim : -1;
  g.narrow_ok = g.acc_lim > 0;
  g.da = g.db = g.os = 0;
  if (epi == EPI_RES || epi == EPI_PATCH) {
    // residual: align_add(res @ res_exp, t @ mid_exp -> out_exp);
    // patch:    align_add(t @ mid_exp, pos @ res_exp -> out_exp)
    const int a_exp = epi == EPI_RES ? g.res_exp : g.mid_exp;
    const int b_exp = epi == EPI_RES ? g.mid_exp : g.res_exp;
    const int c = a_exp < b_exp ? a_exp : b_exp;
    g.da = a_exp - c;
    g.db = b_exp - c;
    g.os = g.out_exp - c;
  }
}

static bool fast_epilogue(const GemmArgs &g, int epi) {
  auto in = [](int s) { return s >= -30 && s <= 30; };
  if (!g.narrow_ok || !in(g.shift_a)) return false;
  switch (epi) {
    case EPI_I8:
    case EPI_I32: return true;
    case EPI_GELU: return in(g.shift_b);
    case EPI_RES:
    case EPI_PATCH: return g.da <= 21 && g.db <= 21 && in(g.os);
    default: return false;
  }
}

// Requant directions of a launch for the int32 epilogue (bit 0: the
// product requant shifts left, bit 1: the second requant -- GELU output or
// align-add -- shifts left).
static int epilogue_dirs(const GemmArgs &g, int epi) {
  int d = g.shift_a <= 0 ? 1 : 0;
  if (epi == EPI_GELU && g.shift_b <= 0) d |= 2;
  if ((epi == EPI_RES || epi == EPI_PATCH) && g.os <= 0) d |= 2;
  return d;
}

// Launches kernel template K with FAST = false, or FAST = true and the
// launch's requant directions (bit 2: the GELU post-op from its step table,
// staged in dynamic LDS, direct kernel only).
template <int EPI, template <bool, int> class K>
static int launch_epi(const GemmArgs &g, long long grid, int n_blocks, hipStream_t s) {
  const dim3 gd((unsigned)grid), bd(256);
  if (!fast_epilogue(g, EPI)) {
    hv_launch(K<false, 0>::fn(), gd, bd, 0, s, g, n_blocks);
  } else {
    const int dirs = epilogue_dirs(g, EPI);
    if constexpr (EPI == EPI_GELU && K<true, 4>::kTable) {
      if (g.lut_words > 0) {
        // persistent: each workgroup stages the table once
        const dim3 gp((unsigned)(grid < kLutGridCap ? grid : kLutGridCap));
        const size_t lds = (size_t)g.lut_words * 4;
        if (dirs & 1) hv_launch(K<true, 5>::fn(), gp, bd, lds, s, g, n_blocks);
        else hv_launch(K<true, 4>::fn(), gp, bd, lds, s, g, n_blocks);
        return check_hip(hipGetLastError(), "k_gemm launch");
      }
    }
    switch (dirs) {
      case 0: hv_launch(K<true, 0>::fn(), gd, bd, 0, s, g, n_blocks); break;
      case 1: hv_launch(K<true, 1>::fn(), gd, bd, 0, s, g, n_blocks); break;
      case 2: hv_launch(K<true, 2>::fn(), gd, bd, 0, s, g, n_blocks); break;
      default: hv_launch(K<true, 3>::fn(), gd, bd, 0, s, g, n_blocks); break;
    }
  }
  return check_hip(hipGetLastError(), "k_gemm launch");
}

template <int MT, int NT, int WM, int EPI, int AMODE, int KTC>
struct DirectK {
  template <bool FAST, int DIRS>
  struct K {
    static constexpr bool kTable = true;
    static auto fn() { return &k_gemm<MT, NT, WM, EPI, AMODE, KTC, FAST, FAST ? DIRS : 0>; }
  };
};

template <int MT, int NT, int WM, int EPI, int AMODE, int KTC>
struct LdsK {
  template <bool FAST, int DIRS>
  struct K {
    static constexpr bool kTable = false;
    static auto fn() { return &k_gemm_lds<MT, NT, WM, EPI, AMODE, KTC, FAST, FAST ? DIRS & 3 : 0>; }
  };
};

template <int MT, int NT, int WM, int EPI, int AMODE, int KTC>
static int run(const GemmArgs &g, hipStream_t s) {
  constexpr int BM = 32 * MT * WM, BN = 32 * NT * (4 / WM);
  const int n_blocks = (g.n + BN - 1) / BN;
  const long long tiles = (long long)((g.m + BM - 1) / BM) * n_blocks;
  if (tiles <= 0) return HV_OK;
  long long grid = (tiles + 7) / 8 * 8;
  if (grid > kGridCap) grid = kGridCap;
  return launch_epi<EPI, DirectK<MT, NT, WM, EPI, AMODE, KTC>::template K>(g, grid, n_blocks, s);
}

template <int MT, int NT, int WM, int EPI, int AMODE, int KTC>
static int run_lds(const GemmArgs &g, hipStream_t s) {
  constexpr int BM = 32 * MT * WM, BN = 32 * NT * (4 / WM);
  const int n_blocks = (g.n + BN - 1) / BN;
  const long long tiles = (long long)((g.m + BM - 1) / BM) * n_blocks;
  if (tiles <= 0) return HV_OK;
  long long grid = (tiles + 7) / 8 * 8;
  if (grid > kLdsGridCap) grid = kLdsGridCap;
  return launch_epi<EPI, LdsK<MT, NT, WM, EPI, AMODE, KTC>::template K>(g, grid, n_blocks, s);
}

// Shapes (measured on the pruned batch-256 forward): the GELU GEMM (K = 192)
// uses the direct kernel with 64x64 tiles (its epilogue holds more
// registers); the other K = 192 and the K = 768 GEMMs (QKV, proj, FFN2,
// patch embedding) the LDS-staged kernel with 128x64 tiles and two
// persistent workgroups per CU (three per CU, one workgroup per tile,
// 128x128 tiles and 64x128 tiles were slower); the gathered head rows with
// K = 192 the direct kernel with every K step loaded up front; other K the
// runtime-K direct kernel.
template <int EPI>
static int dispatch(const GemmArgs &g, int a_mode, hipStream_t s) {
  if constexpr (EPI == EPI_PATCH) {
    // A from the NHWC images (gathered patches) or from patch rows [B*196][768]
    if (g.k != 768 || (a_mode != A_PATCH && (a_mode != A_ROWS || g.lda != 768)))
      return fail(HV_EVALUE, HV_ERR_DIMENSION, "gemm: bad patch GEMM");
    if (a_mode == A_ROWS) return run_lds<2, 1, 2, EPI_PATCH, A_ROWS, 24>(g, s);
    return run_lds<2, 1, 2, EPI_PATCH, A_PATCH, 24>(g, s);
  } else {
    if (a_mode == (A_ROWS | A_UNSIGNED)) return run<1, 1, 2, EPI, A_ROWS | A_UNSIGNED, 0>(g, s);
    if (a_mode == A_GATHER) {
      // the classifier head (K = 192 on the CLS rows): every fragment in
      // flight at once, one memory round trip instead of six
      if constexpr (EPI == EPI_I32)
        if (g.k == 192) return run<1, 1, 2, EPI, A_GATHER, 6>(g, s);
      return run<1, 1, 2, EPI, A_GATHER, 0>(g, s);
    }
    if (a_mode != A_ROWS) return fail(HV_EVALUE, HV_ERR_OPCODE, "gemm: bad A mode %d", a_mode);
    if constexpr (EPI == EPI_GELU) {
      if (g.k == 192) return run<1, 1, 2, EPI, A_ROWS, 6>(g, s);
    } else if constexpr (EPI != EPI_I32) {
      if (g.k == 192) return run_lds<2, 1, 2, EPI, A_ROWS, 6>(g, s);
      if (g.k == 768) return run_lds<2, 1, 2, EPI, A_ROWS, 24>(g, s);
    }
    return run<1, 1, 2, EPI, A_ROWS, 0>(g, s);
  }
}

int launch_gemm(const GemmArgs &g_in, int a_mode, int epi, hipStream_t s) {
  GemmArgs g = g_in;
  g.a_unsigned = (a_mode & A_UNSIGNED) != 0;
  if (g.a_unsigned && (a_mode != (A_ROWS | A_UNSIGNED) || epi == EPI_PATCH))
    return fail(HV_EVALUE, HV_ERR_OPCODE, "gemm: unsigned A needs HV_A_ROWS and a plain epilogue");
  epilogue_limits_pub(g, epi);
  if (g.k <= 0 || g.k % 32)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "gemm: K=%d must be a positive multiple of 32", g.k);
  if (g.a_unsigned && g.k > 65536)
    return fail(HV_EOVERFLOW, HV_ERR_DIMENSION, "gemm: unsigned A with K=%d may overflow int32",
                g.k);
  if (g.n <= 0) return fail(HV_EVALUE, HV_ERR_DIMENSION, "gemm: N=%d must be positive", g.n);
  if (g.m < 0) return fail(HV_EVALUE, HV_ERR_DIMENSION, "gemm: M=%d must be non-negative", g.m);
  if (a_mode != A_PATCH && (g.lda % 16 || ((uintptr_t)g.a & 15)))
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "gemm: A must be 16-byte aligned with lda %% 16 == 0");
  if (a_mode == A_PATCH && ((uintptr_t)g.a & 15))
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "gemm: images must be 16-byte aligned");
  if (g.bias && ((uintptr_t)g.bias & 15))
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "gemm: bias must be 16-byte aligned");
  if (g.k > 131071)
    return fail(HV_EOVERFLOW, HV_ERR_DIMENSION, "gemm: K=%d may overflow int32", g.k);
  g.lut_words = 0;
  if (epi == EPI_GELU && g.shift_b >= kGeluLutSoMin && g.shift_b <= kGeluLutSoMax) {
    const GeluLutInfo &t = kGeluLutInfo[g.shift_b - kGeluLutSoMin];
    g.lut_off = t.off;
    g.lut_words = t.words;
    g.lut_n1e = t.n1e;
    g.lut_qlo = t.qlo; g.lut_cb = -4 * (t.qlo >> kGeluCoarseShift);
    g.lut_qhi = t.qhi;
  }
  const int esz = epi == EPI_I32 ? 4 : 1;
  g.vec_out = ((uintptr_t)g.c & 15) == 0 && (g.ldc * esz) % 16 == 0 &&
              (!g.aux || ((uintptr_t)g.aux & 15) == 0);
  if (epi == EPI_RES) g.vec_res = ((uintptr_t)g.res & 15) == 0 && g.ldr % 16 == 0;
  if (epi == EPI_PATCH) g.vec_res = ((uintptr_t)g.pos & 15) == 0;
  switch (epi) {
    case EPI_I8: return dispatch<EPI_I8>(g, a_mode, s);
    case EPI_I32: return dispatch<EPI_I32>(g, a_mode, s);
    case EPI_GELU: return dispatch<EPI_GELU>(g, a_mode, s);
    case EPI_RES: return dispatch<EPI_RES>(g, a_mode, s);
    case EPI_PATCH: return dispatch<EPI_PATCH>(g, a_mode, s);
    default: return fail(HV_EVALUE, HV_ERR_OPCODE, "gemm: bad epilogue %d", epi);
  }
}

// ---------------------------------------------------------------------------
// Fused FFN (transformer.ffn, transformer.py:328-384) for the int32
// epilogues with a GELU step table: z = align_add(y, requant(GELU(ln2 W1 +
// b1) W2 + b2)).  A workgroup owns one block of 64 rows (the grid has one
// per row block):
//   phase A  the FFN1 tiles (2 row x 24 column tiles of 32; wavefront w
//            takes columns w, w+4, ...), the GELU post-op from the step
//            table, the hidden row block written to LDS ([64][768] at a
//            784-byte row stride, conflict-free 16-byte reads);
//   phase B  the FFN2 tiles (2 row x 6 column tiles, three per wavefront)
//            with K = 768 read from LDS and the residual epilogue.
// Optionally LayerNorm 2 of y runs in front of phase A (the normalised rows
// pass through LDS, y is read once more as the residual) and the next
// block's LayerNorm 1 of the output rows behind phase B (ln_rows, below);
// with LayerNorm 2 inside, the attention projection that produces y can run
// first as well (phase P: 2 x 6 tiles, K = 192; y stays on the CU).
// The hidden activations never leave the CU.  Each workgroup stages the
// GELU table, its loads in flight while the first rows load.
// ---------------------------------------------------------------------------
static constexpr int kFfnRows = 64, kFfnHRow = 784, kLnPrologueRow = 208;
static_assert(kFfnRows * kFfnHRow + 4 * kGeluLutMaxWords <= 160 * 1024 / 2,
              "the fused FFN's LDS must allow two workgroups per CU");
static_assert(kLnPrologueRow <= kFfnHRow, "LayerNorm rows fit the hidden block");
static_assert(kFfnRows * kLnPrologueRow <= 4 * kGeluLutMaxWords, "output rows fit the table");

// LayerNorm (nonlinear.py:136-186, the int32 form of k_layernorm32) of a
// block of 64 rows by 256 threads: 32 eight-lane groups, group j taking rows
// j and j + 32, each lane 24 channels.  Lane sub works out the constants of
// row sub % 2 and the group reads them from lanes 0 and 1, so the
// 64/128-bit set-up runs four times per row instead of eight.  Row i is
// read from src + min(i, clamp) * SS and written to dst + i * DS when
// i < store_rows; rows with i < report_rows (row r0 + i of the batch)
// report a negative variance to lw (the int32 form cannot produce one:
// with x_scale >= -16 the sum of squares is exact and the rounding of the
// mean moves mean^2 by less than the smallest nonzero variance).
// When `two` is false the block holds 32 rows (rows 32..63 are neither
// normalised nor stored, and their constants raise no exact pass).
// ln_rows' output half: rows grp and grp + 32 with the constants of lanes
// base + 0 and base + 1 of the 8-lane group.
template <bool EXACT, int DS>
__device__ __forceinline__ void ln_rows_out(const LnRow &mine, const int (&w)[2][6],
                                            const int (&gw)[6], const int (&bw)[6], const Ln32 &ln,
                                            int8_t *dst, int store_rows, int grp, int sub,
                                            bool two) {
  const int rnd = 1 << (ln.os - 1);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (r == 1 && !two) break;  // uniform
    const LnRow c = ln_row_shfl<EXACT>(mine, (threadIdx.x & 63 & ~7) + r);
    int ov[24], out[6];
#pragma unroll
    for (int j = 0; j < 24; ++j) {
      const int sh = 8 * (j & 3);
      const int xv = __builtin_amdgcn_sbfe(w[r][j >> 2], sh, 8);
      const int g = __builtin_amdgcn_sbfe(gw[j >> 2], sh, 8);
      const int bb = __builtin_amdgcn_sbfe(bw[j >> 2], sh, 8) * (1 << ln.bs);
      const int a = __mul24(ln_norm<EXACT>(xv, c), g) + bb;  // both within 24 bits
      const int o = (a + rnd + (a >> 31)) >> ln.os;
      ov[j] = min(max(o, -128), 127);
    }
#pragma unroll
    for (int q = 0; q < 6; ++q)
      out[q] = (int)pack_lo4(ov[4 * q], ov[4 * q + 1], ov[4 * q + 2], ov[4 * q + 3]);
    if (grp + 32 * r < store_rows) {
      int2 *yr = reinterpret_cast<int2 *>(dst + (grp + 32 * r) * DS + sub * 24);
#pragma unroll
      for (int q = 0; q < 3; ++q) yr[q] = int2{out[2 * q], out[2 * q + 1]};
    }
  }
}

template <int SS, int DS>
__device__ __forceinline__ void ln_rows(const int8_t *src, int clamp, int8_t *dst, int store_rows,
                                        const Ln32 &ln, const LnWarn &lw, int r0,
                                        int report_rows, bool two = true) {
  const int tid = threadIdx.x, sub = tid & 7, grp = tid >> 3;
  int w[2][6];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int2 *xr =
        reinterpret_cast<const int2 *>(src + min(grp + 32 * r, clamp) * SS + sub * 24);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int2 v = xr[q];
      w[r][2 * q] = v.x;
      w[r][2 * q + 1] = v.y;
    }
  }
  int gw[6], bw[6];
  {
    const int2 *gp = reinterpret_cast<const int2 *>(ln.gamma + sub * 24);
    const int2 *bp = reinterpret_cast<const int2 *>(ln.beta + sub * 24);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int2 a = gp[q], c = bp[q];
      gw[2 * q] = a.x; gw[2 * q + 1] = a.y;
      bw[2 * q] = c.x; bw[2 * q + 1] = c.y;
    }
  }
  int sx[2], sxx[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
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
    for (int r = 0; r < 2; ++r) {
      sx[r] += __shfl_xor(sx[r], off);
      sxx[r] += __shfl_xor(sxx[r], off);
    }
  const int mr = sub & 1;
  LnRow mine = ln_row_consts_e<LnEstHw>(mr ? sx[1] : sx[0], mr ? sxx[1] : sxx[0], ln.s, ln.t);
  if (!two && mr) mine.tie = false;
  if (sub < 2 && mine.neg_var && lw.img_warn && grp + 32 * sub < report_rows)
    ln_warn_row(lw.offsets, lw.batch, lw.img_warn, r0 + grp + 32 * sub);
  if (__any(mine.tie))
    ln_rows_out<true, DS>(mine, w, gw, bw, ln, dst, store_rows, grp, sub, two);
  else
    ln_rows_out<false, DS>(mine, w, gw, bw, ln, dst, store_rows, grp, sub, two);
}

// Epilogue of one attention-projection tile in the fused FFN: lane l's 16
// bytes of y = align_add(x, requant(ctx Wp + bp)) (transformer.py:267-272,
// 413-421), in the int32 form when every lane's biases allow it, else exact;
// acc started at the bias bs (the MFMA's C operand).
template <bool LA, bool LB>
__device__ __forceinline__ v4i proj_epi(const GemmArgs &gp, const v16i &acc, const v16i &bs,
                                        v4i x4, const Rq &rpa, const Rq &rpb, bool all_narrow) {
  bool fast = all_narrow;
  if (!all_narrow) {
    int bmax = bs[0], bmin = bmax;
#pragma unroll
    for (int j = 1; j < 16; ++j) {
      bmax = max(bmax, bs[j]);
      bmin = min(bmin, bs[j]);
    }
    fast = __all(bmax <= gp.acc_lim && bmin >= -gp.acc_lim);
  }
  int o[16];
  if (fast) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int t8 = rq_dir_nowrap<LA>(acc[j], rpa);
      const int r8 = (int)(int8_t)(x4[j >> 2] >> (8 * (j & 3)));
      o[j] = rq_dir<LB>(r8 * (1 << gp.da) + t8 * (1 << gp.db), rpb);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r8 = (int)(int8_t)(x4[j >> 2] >> (8 * (j & 3)));
      o[j] = epi_exact(EPI_RES, acc[j] - bs[j], bs[j], r8, gp.shift_a, gp.shift_b, gp.da,
                       gp.db, gp.os)[0];
    }
  }
  return v4i{pack4(o[0], o[1], o[2], o[3]), pack4(o[4], o[5], o[6], o[7]),
             pack4(o[8], o[9], o[10], o[11]), pack4(o[12], o[13], o[14], o[15])};
}

// LN: LayerNorm 2 in front (fl); LNE: the next block's LayerNorm 1 of the
// output rows behind (fe, output fe.ln.out): phase B also writes its rows to
// LDS where the GELU table was (phase A is done with it), and the rows are
// normalised once they are complete.  PJ (with LN): the attention
// projection and its residual (gp, requant directions dirsp) run first and
// produce y, which never leaves the CU: each wavefront computes the y tiles
// of its phase-B tiles and keeps their bytes as phase B's residual, and the
// y rows pass through LDS to LayerNorm 2.
// Workgroups 0 .. nfull - 1 take 64-row blocks; the ones after them blocks
// of 32 rows (one row tile: the steps of the second are skipped), so that a
// launch whose last 64-row blocks would double up on a few CUs spreads that
// work over twice as many.
template <int DIRS1, int DIRS2, bool LN, bool LNE, bool PJ>
__global__ __launch_bounds__(256) void k_ffn(GemmArgs g1, GemmArgs g2, LnPrologue fl,
                                             LnPrologue fe, GemmArgs gp, int dirsp, int nfull) {
  static_assert(!PJ || LN, "the projection feeds the LayerNorm in front");
  __shared__ __attribute__((aligned(16))) int8_t hid[kFfnRows * kFfnHRow];
  // static, so its LDS address is a constant the table reads can fold
  __shared__ __attribute__((aligned(16))) unsigned lut[kGeluLutMaxWords];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  // The step table loads in one round (at most eight 16-byte vectors per
  // thread), issued before the live row count it does not depend on, and
  // lands while the row block's LayerNorm or A fragments load; its LDS writes
  // precede the barrier in front of phase A.  Threads past the end reload the
  // last vector (no predicated loads or writes).
  static_assert(kGeluLutMaxWords / 4 <= 8 * 256, "one staging round");
  const int n4 = g1.lut_words >> 2;
  v4i tv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    tv[i] = reinterpret_cast<const v4i *>(kGeluLut + g1.lut_off)[min(tid + 256 * i, n4 - 1)];
  const int M = g1.m_dev ? min(*g1.m_dev, g1.m) : g1.m;
  const int bid = blockIdx.x;
  const int nrt = bid < nfull ? 2 : 1;  // row tiles of this block
  const int r0 = bid < nfull ? bid * kFfnRows : nfull * kFfnRows + (bid - nfull) * 32;
  if (r0 >= M) return;  // uniform: before any barrier
  const bool two = nrt == 2;
  const int live = min(M - r0, 32 * nrt);  // rows of this block
  auto write_lut = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) reinterpret_cast<v4i *>(lut)[min(tid + 256 * i, n4 - 1)] = tv[i];
  };
  const Rq r1a = rq_setup(g1.shift_a, -(1 << 23), (1 << 23) - 1);
  const Rq r2a = rq_setup(g2.shift_a, -128, 127), r2b = rq_setup(g2.os, -128, 127);
  constexpr bool LA1 = DIRS1 & 1;
  const bool all1 = tensor_narrow(g1.bias_max, g1.acc_lim);
  int qhi = g1.lut_qhi;
  asm("" : "+v"(qhi));  // the table clamp as one med3 (both bounds in VGPRs)

  {
    // Weight fragments single-buffered: the next column tile's load is
    // issued after the current tile's MFMAs and lands during its GELU
    // epilogues; the biases are double-buffered.
    v4i bf[6];
    v16i bs[2];
    auto load_w1 = [&](int ci, v16i &bi) {
      const int ct = wave + 4 * ci;
#pragma unroll
      for (int kt = 0; kt < 6; ++kt)
        bf[kt] = *reinterpret_cast<const v4i *>(g1.b + (size_t)(ct * 6 + kt) * 1024 + lane * 16);
      bi = *reinterpret_cast<const v16i *>(g1.bias + ct * 32 + 16 * h);
    };
    // Phase P (PJ): y tiles wave, wave + 4, wave + 8 of the 2 x 6 (phase B's
    // tiles), K = 192 from the ctx rows; their bytes stay in yres and go to
    // LDS (208-byte rows) for LayerNorm 2.
    v4i yres[PJ ? 3 : 1] = {};
    if constexpr (PJ) {
      const Rq rpa = rq_setup(gp.shift_a, -128, 127), rpb = rq_setup(gp.os, -128, 127);
      const bool allp = tensor_narrow(gp.bias_max, gp.acc_lim);
#pragma unroll
      for (int ti = 0; ti < 3; ++ti) {
        const int t = wave + 4 * ti, rt = t / 6, ct = t - rt * 6;
        if (rt >= nrt) break;  // uniform in the wavefront
        const int8_t *ap = gp.a + (size_t)min(r0 + 32 * rt + l32, M - 1) * 192 + 16 * h;
        const int8_t *bp = gp.b + (size_t)ct * 6 * 1024 + lane * 16;
        v4i pa[6], pw[6];
#pragma unroll
        for (int kt = 0; kt < 6; ++kt) {
          pa[kt] = *reinterpret_cast<const v4i *>(ap + kt * 32);
          pw[kt] = *reinterpret_cast<const v4i *>(bp + kt * 1024);
        }
        const v16i pbs = *reinterpret_cast<const v16i *>(gp.bias + ct * 32 + 16 * h);
        const v4i x4 = *reinterpret_cast<const v4i *>(
            gp.res + (size_t)min(r0 + 32 * rt + l32, M - 1) * 192 + ct * 32 + 16 * h);
        v16i acc = pbs;  // the accumulator starts at the bias
#pragma unroll
        for (int kt = 0; kt < 6; ++kt)
          acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(pw[kt], pa[kt], acc, 0, 0, 0);
        v4i yv;
        switch (dirsp) {
          case 0: yv = proj_epi<false, false>(gp, acc, pbs, x4, rpa, rpb, allp); break;
          case 1: yv = proj_epi<true, false>(gp, acc, pbs, x4, rpa, rpb, allp); break;
          case 2: yv = proj_epi<false, true>(gp, acc, pbs, x4, rpa, rpb, allp); break;
          default: yv = proj_epi<true, true>(gp, acc, pbs, x4, rpa, rpb, allp); break;
        }
        yres[ti] = yv;
        *reinterpret_cast<v4i *>(&hid[(32 * rt + l32) * kLnPrologueRow + ct * 32 + 16 * h]) = yv;
      }
    }
    // Phase A.  A fragments of both row tiles, all six K-steps; the weight
    // fragments and biases of column tile ci + 1 load while tile ci runs.
    v4i af[2][6];
    if constexpr (PJ) {
      // y complete in LDS; LayerNorm 2 in place (each group rewrites the
      // rows it read)
      write_lut();
      __syncthreads();
      load_w1(0, bs[0]);
      ln_rows<kLnPrologueRow, kLnPrologueRow>(hid, kFfnRows - 1, hid, kFfnRows, fl.ln, fl.lw, r0,
                                              live, two);
      __syncthreads();
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kt = 0; kt < 6; ++kt)
          af[rt][kt] = *reinterpret_cast<const v4i *>(&hid[(32 * rt + l32) * kLnPrologueRow +
                                                           kt * 32 + 16 * h]);
      __syncthreads();
    } else if constexpr (LN) {
      // the first weight tile loads while the LayerNorm runs; its rows
      // pass through hid (free until phase A writes it)
      load_w1(0, bs[0]);
      ln_rows<192, kLnPrologueRow>(fl.x + (size_t)r0 * 192, M - 1 - r0, hid, kFfnRows, fl.ln,
                                   fl.lw, r0, live, two);
      write_lut();
      __syncthreads();
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kt = 0; kt < 6; ++kt)
          af[rt][kt] = *reinterpret_cast<const v4i *>(&hid[(32 * rt + l32) * kLnPrologueRow +
                                                           kt * 32 + 16 * h]);
      __syncthreads();
    } else {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int8_t *ap = g1.a + (size_t)min(r0 + 32 * rt + l32, M - 1) * g1.lda + 16 * h;
#pragma unroll
        for (int kt = 0; kt < 6; ++kt) af[rt][kt] = *reinterpret_cast<const v4i *>(ap + kt * 32);
      }
      load_w1(0, bs[0]);
      write_lut();
      __syncthreads();
    }
#pragma unroll 2
    for (int ci = 0; ci < 6; ++ci) {
      const int cur = ci & 1;
      const int c0 = (wave + 4 * ci) * 32 + 16 * h;
      // the accumulators start at the bias (the first MFMA's C operand)
      v16i acc[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        acc[rt] = bs[cur];
#pragma unroll
        for (int kt = 0; kt < 6; ++kt)
          acc[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[kt], af[rt][kt], acc[rt], 0, 0, 0);
      }
      if (ci + 1 < 6) load_w1(ci + 1, bs[cur ^ 1]);
      bool fast = all1;
      if (!all1) {
        int bmax = bs[cur][0], bmin = bmax;
#pragma unroll
        for (int j = 1; j < 16; ++j) {
          bmax = max(bmax, bs[cur][j]);
          bmin = min(bmin, bs[cur][j]);
        }
        fast = __all(bmax <= g1.acc_lim && bmin >= -g1.acc_lim);
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        // a 32-row block multiplies its second tile's (unused) rows too,
        // keeping the two accumulator chains interleaved, but skips their
        // epilogue
        if (rt >= nrt) break;
        v4i ow;
        if (fast) {
          int qv[16];
          unsigned ov[4];
#pragma unroll
          for (int j = 0; j < 16; ++j) qv[j] = shift_nowrap<LA1>(acc[rt][j], r1a);
          gelu_table_pack_n<16>(qv, ov, lut, g1.lut_cb, g1.lut_qlo, qhi);
          ow = v4i{(int)ov[0], (int)ov[1], (int)ov[2], (int)ov[3]};
        } else {
          int o[16];
#pragma unroll
          for (int j = 0; j < 16; ++j)
            o[j] = epi_exact(EPI_GELU, acc[rt][j] - bs[cur][j], bs[cur][j], 0, g1.shift_a,
                             g1.shift_b, 0, 0, 0)[0];
          ow = v4i{pack4(o[0], o[1], o[2], o[3]), pack4(o[4], o[5], o[6], o[7]),
                   pack4(o[8], o[9], o[10], o[11]), pack4(o[12], o[13], o[14], o[15])};
        }
        *reinterpret_cast<v4i *>(&hid[(32 * rt + l32) * kFfnHRow + c0]) = ow;
      }
    }
    // The first phase-B tile's operands and first weight chunk load before
    // the barrier.
    auto tile_of = [&](int ti, int &rt, int &ct) {
      const int t = wave + 4 * ti;
      rt = t / 6;
      ct = t - rt * 6;
    };
    v4i wb[3][4], bias4[1][4], res4[1][1];
    v16i bsb;  // the tile's biases, the accumulator's start
    int rt, ct;
    tile_of(0, rt, ct);
    // tiles of this wavefront: 3, or with one row tile those of row tile 0
    const int nt = two ? 3 : (wave < 2 ? 2 : 1);
    // the tile's biases and residual bytes (PJ: the residual from yres)
    auto operands = [&]() {
      const int arow[1] = {min(r0 + 32 * rt + l32, M - 1)};
      if constexpr (PJ) {
        epi_operands<1, 1, EPI_I8>(g2, arow, ct, h, bias4, res4);
        res4[0][0] = yres[0];
      } else {
        epi_operands<1, 1, EPI_RES>(g2, arow, ct, h, bias4, res4);
      }
      bsb = *reinterpret_cast<const v16i *>(g2.bias + ct * 32 + 16 * h);
#pragma unroll
      for (int j = 0; j < 16; ++j) bias4[0][j >> 2][j & 3] = bsb[j];
    };
    operands();
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wb[c][j] = *reinterpret_cast<const v4i *>(g2.b + ((size_t)ct * 24 + c * 4 + j) * 1024 +
                                                  lane * 16);
    __syncthreads();
    // Phase B: tiles wave, wave + 4, wave + 8 of the 2 x 6; 24 K-steps in
    // chunks of 4 through a ring of three chunk buffers: the chunk two
    // ahead (within the tile or the next tile's first two) is in flight.
#pragma unroll 1
    for (int ti = 0; ti < nt; ++ti) {
      const int8_t *hp = &hid[(32 * rt + l32) * kFfnHRow + 16 * h];
      const int8_t *bp = g2.b + (size_t)ct * 24 * 1024 + lane * 16;
      int nxrt = rt, nct = ct;
      if (ti + 1 < nt) tile_of(ti + 1, nxrt, nct);
      v16i acc[1][1] = {{bsb}};
#pragma unroll
      for (int c = 0; c < 6; ++c) {
        const int cur = c % 3, nxt = (c + 2) % 3;
        if (c + 2 < 6) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            wb[nxt][j] = *reinterpret_cast<const v4i *>(bp + ((c + 2) * 4 + j) * 1024);
        } else if (ti + 1 < nt) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            wb[nxt][j] = *reinterpret_cast<const v4i *>(
                g2.b + ((size_t)nct * 24 + (c - 4) * 4 + j) * 1024 + lane * 16);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
              wb[cur][j], *reinterpret_cast<const v4i *>(hp + (c * 4 + j) * 32), acc[0][0], 0, 0,
              0);
        __builtin_amdgcn_sched_barrier(0);  // one chunk of LDS reads in flight at a time
      }
      epi_tile<1, 1, EPI_RES, true, DIRS2, true>(
          g2, acc, bias4, res4, r0 + 32 * rt, ct, M, h, l32, r2a, r2b, nullptr,
          LNE ? reinterpret_cast<int8_t *>(lut) + 32 * rt * kLnPrologueRow : nullptr,
          kLnPrologueRow);
      if (ti + 1 < nt) {
        rt = nxrt;
        ct = nct;
        if constexpr (PJ) {
          yres[0] = yres[1];
          yres[1] = yres[2];
        }
        operands();
      }
    }
    if constexpr (LNE) {
      __syncthreads();  // every output row is in zs
      const int8_t *zs = reinterpret_cast<const int8_t *>(lut);
      ln_rows<kLnPrologueRow, 192>(zs, kFfnRows - 1, fe.ln.out + (size_t)r0 * 192, live, fe.ln,
                                   fe.lw, r0, live, two);
    }
  }
}

// ---------------------------------------------------------------------------
// The fused FFN over blocks of 32 rows by eight wavefronts (k_ffn32): the
// same phases and epilogues as k_ffn, with a quarter of k_ffn's work per
// wavefront, for batches whose 64-row blocks would leave CUs idle (the
// pruned stages of one forward at a time).  One row tile of 32:
//   phase P  wavefront w < 6: projection column tile w (K = 192);
//   LN       16 lanes per row (ln_rows16);
//   phase A  wavefront w: FFN1 column tiles w, w + 8, w + 16, GELU from the
//            step table into the hidden block [32][768] (784-byte rows);
//   phase B  wavefront w < 6: FFN2 column tile w over K = 768, residual;
//   LNE      the next block's LayerNorm 1 of the output rows.
// ---------------------------------------------------------------------------
static constexpr int kFfn32Rows = 32;

// LayerNorm (nonlinear.py:136-186, int32 form) of a block of 32 rows by 512
// threads: 16 lanes per row, 12 channels each, every lane working out its
// row's constants (no broadcast).  Row i is read from src + min(i, clamp) *
// SS and written to dst + i * DS when i < store_rows; rows i < report_rows
// (row r0 + i of the batch) report a negative variance to lw.
template <int SS, int DS>
__device__ __forceinline__ void ln_rows16(const int8_t *src, int clamp, int8_t *dst,
                                          int store_rows, const Ln32 &ln, const LnWarn &lw,
                                          int r0, int report_rows) {
  const int tid = threadIdx.x, sub = tid & 15, row = tid >> 4;
  int w[3], gm[3], bt[3], out[3];
  const int *xr = reinterpret_cast<const int *>(src + min(row, clamp) * SS + sub * 12);
  const int *gp = reinterpret_cast<const int *>(ln.gamma + sub * 12);
  const int *bp = reinterpret_cast<const int *>(ln.beta + sub * 12);
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    w[q] = xr[q];
    gm[q] = gp[q];
    bt[q] = bp[q];
  }
  const bool neg = ln32_row<16>(w, gm, bt, ln, out);
  if (sub == 0 && neg && lw.img_warn && row < report_rows)
    ln_warn_row(lw.offsets, lw.batch, lw.img_warn, r0 + row);
  if (row < store_rows) {
    int *yr = reinterpret_cast<int *>(dst + row * DS + sub * 12);
#pragma unroll
    for (int q = 0; q < 3; ++q) yr[q] = out[q];
  }
}

template <int DIRS1, int DIRS2, bool LN, bool LNE, bool PJ>
__global__ __launch_bounds__(512, 4) void k_ffn32(GemmArgs g1, GemmArgs g2, LnPrologue fl,
                                               LnPrologue fe, GemmArgs gp, int dirsp) {
  static_assert(!PJ || LN, "the projection feeds the LayerNorm in front");
  static_assert(kFfn32Rows * kLnPrologueRow <= 4 * kGeluLutMaxWords, "output rows fit the table");
  __shared__ __attribute__((aligned(16))) int8_t hid[kFfn32Rows * kFfnHRow];
  __shared__ __attribute__((aligned(16))) unsigned lut[kGeluLutMaxWords];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  // Loads that need no row index go out before the live row count, whose
  // latency they share: the step table in one round of at most four 16-byte
  // vectors per thread (written to LDS before the barrier in front of phase
  // A) and, with PJ, wavefront w < 6's projection weights and biases.
  static_assert(kGeluLutMaxWords / 4 <= 4 * 512, "one staging round");
  const int n4 = g1.lut_words >> 2;
  v4i tv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    tv[i] = reinterpret_cast<const v4i *>(kGeluLut + g1.lut_off)[min(tid + 512 * i, n4 - 1)];
  v4i pw[6];
  v16i pbs;
  if constexpr (PJ) {
    if (wave < 6) {
      const int8_t *bp = gp.b + (size_t)wave * 6 * 1024 + lane * 16;
#pragma unroll
      for (int kt = 0; kt < 6; ++kt) pw[kt] = *reinterpret_cast<const v4i *>(bp + kt * 1024);
      pbs = *reinterpret_cast<const v16i *>(gp.bias + wave * 32 + 16 * h);
    }
  }
  const int M = g1.m_dev ? min(*g1.m_dev, g1.m) : g1.m;
  if ((int)blockIdx.x >= (M + kFfn32Rows - 1) / kFfn32Rows) return;  // uniform
  const int r0 = blockIdx.x * kFfn32Rows;
  const int arow = min(r0 + l32, M - 1);
  auto write_lut = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<v4i *>(lut)[min(tid + 512 * i, n4 - 1)] = tv[i];
  };
  const Rq r1a = rq_setup(g1.shift_a, -(1 << 23), (1 << 23) - 1);
  const Rq r2a = rq_setup(g2.shift_a, -128, 127), r2b = rq_setup(g2.os, -128, 127);
  constexpr bool LA1 = DIRS1 & 1;
  const bool all1 = tensor_narrow(g1.bias_max, g1.acc_lim);
  int qhi = g1.lut_qhi;
  asm("" : "+v"(qhi));  // the table clamp as one med3 (both bounds in VGPRs)

  // Phase P (PJ): wavefront w < 6 computes y tile w and keeps its bytes as
  // phase B's residual; the y rows go to LDS (208-byte rows) for LayerNorm 2.
  v4i yres = v4i{0};
  if constexpr (PJ) {
    if (wave < 6) {
      const int ct = wave;
      const Rq rpa = rq_setup(gp.shift_a, -128, 127), rpb = rq_setup(gp.os, -128, 127);
      const bool allp = tensor_narrow(gp.bias_max, gp.acc_lim);
      const int8_t *ap = gp.a + (size_t)arow * 192 + 16 * h;
      v4i pa[6];
#pragma unroll
      for (int kt = 0; kt < 6; ++kt) pa[kt] = *reinterpret_cast<const v4i *>(ap + kt * 32);
      const v4i x4 =
          *reinterpret_cast<const v4i *>(gp.res + (size_t)arow * 192 + ct * 32 + 16 * h);
      v16i acc = pbs;  // the accumulator starts at the bias
#pragma unroll
      for (int kt = 0; kt < 6; ++kt)
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(pw[kt], pa[kt], acc, 0, 0, 0);
      switch (dirsp) {
        case 0: yres = proj_epi<false, false>(gp, acc, pbs, x4, rpa, rpb, allp); break;
        case 1: yres = proj_epi<true, false>(gp, acc, pbs, x4, rpa, rpb, allp); break;
        case 2: yres = proj_epi<false, true>(gp, acc, pbs, x4, rpa, rpb, allp); break;
        default: yres = proj_epi<true, true>(gp, acc, pbs, x4, rpa, rpb, allp); break;
      }
      *reinterpret_cast<v4i *>(&hid[l32 * kLnPrologueRow + ct * 32 + 16 * h]) = yres;
    }
  }
  // Phase A's first weight tile loads during LayerNorm 2; the row tile's A
  // fragments come through hid (LayerNorm 2 rows) or from the caller's rows.
  v4i bf[6];
  auto load_w1 = [&](int ci) {
    const int ct = wave + 8 * ci;
#pragma unroll
    for (int kt = 0; kt < 6; ++kt)
      bf[kt] = *reinterpret_cast<const v4i *>(g1.b + (size_t)(ct * 6 + kt) * 1024 + lane * 16);
  };
  load_w1(0);
  v4i af[6];
  if constexpr (PJ) {
    write_lut();
    __syncthreads();  // y complete in LDS; LayerNorm 2 in place
    ln_rows16<kLnPrologueRow, kLnPrologueRow>(hid, kFfn32Rows - 1, hid, kFfn32Rows, fl.ln, fl.lw,
                                              r0, M - r0);
    __syncthreads();
  } else if constexpr (LN) {
    ln_rows16<192, kLnPrologueRow>(fl.x + (size_t)r0 * 192, M - 1 - r0, hid, kFfn32Rows, fl.ln,
                                   fl.lw, r0, M - r0);
    write_lut();
    __syncthreads();
  }
  if constexpr (LN) {
#pragma unroll
    for (int kt = 0; kt < 6; ++kt)
      af[kt] = *reinterpret_cast<const v4i *>(&hid[l32 * kLnPrologueRow + kt * 32 + 16 * h]);
    __syncthreads();  // phase A rewrites hid
  } else {
    const int8_t *ap = g1.a + (size_t)arow * g1.lda + 16 * h;
#pragma unroll
    for (int kt = 0; kt < 6; ++kt) af[kt] = *reinterpret_cast<const v4i *>(ap + kt * 32);
    write_lut();
    __syncthreads();
  }
  // Phase A: column tiles wave + 8 ci; the next tile's weight fragments load
  // during the current tile's GELU epilogue, its biases during its MFMAs.
  {
#pragma unroll
    for (int ci = 0; ci < 3; ++ci) {
      const int c0 = (wave + 8 * ci) * 32 + 16 * h;
      // the accumulator starts at the bias (the first MFMA's C operand)
      const v16i bs = *reinterpret_cast<const v16i *>(g1.bias + c0);
      v16i acc = bs;
#pragma unroll
      for (int kt = 0; kt < 6; ++kt)
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[kt], af[kt], acc, 0, 0, 0);
      if (ci + 1 < 3) load_w1(ci + 1);
      bool fast = all1;
      if (!all1) {
        int bmax = bs[0], bmin = bmax;
#pragma unroll
        for (int j = 1; j < 16; ++j) {
          bmax = max(bmax, bs[j]);
          bmin = min(bmin, bs[j]);
        }
        fast = __all(bmax <= g1.acc_lim && bmin >= -g1.acc_lim);
      }
      v4i ow;
      if (fast) {
        // the lookups in two stages of eight (registers)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          int qv[8];
          unsigned ov[2];
#pragma unroll
          for (int j = 0; j < 8; ++j) qv[j] = shift_nowrap<LA1>(acc[8 * hf + j], r1a);
          gelu_table_pack_n<8>(qv, ov, lut, g1.lut_cb, g1.lut_qlo, qhi);
          ow[2 * hf] = (int)ov[0];
          ow[2 * hf + 1] = (int)ov[1];
        }
      } else {
        int o[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
          o[j] = epi_exact(EPI_GELU, acc[j] - bs[j], bs[j], 0, g1.shift_a, g1.shift_b, 0, 0,
                           0)[0];
        ow = v4i{pack4(o[0], o[1], o[2], o[3]), pack4(o[4], o[5], o[6], o[7]),
                 pack4(o[8], o[9], o[10], o[11]), pack4(o[12], o[13], o[14], o[15])};
      }
      *reinterpret_cast<v4i *>(&hid[l32 * kFfnHRow + c0]) = ow;
    }
  }
  // Phase B: wavefront w < 6 takes FFN2 column tile w over K = 768 in chunks
  // of 4 K-steps through a ring of three chunk buffers, two chunks ahead;
  // its operands and first two weight chunks load before the barrier.
  const int ct = wave;
  v4i wb[3][4], bias4[1][4], res4[1][1];
  v16i bsb;  // the tile's biases, the accumulator's start
  if (wave < 6) {
    const int arows[1] = {arow};
    if constexpr (PJ) {
      epi_operands<1, 1, EPI_I8>(g2, arows, ct, h, bias4, res4);
      res4[0][0] = yres;
    } else {
      epi_operands<1, 1, EPI_RES>(g2, arows, ct, h, bias4, res4);
    }
    bsb = *reinterpret_cast<const v16i *>(g2.bias + ct * 32 + 16 * h);
#pragma unroll
    for (int j = 0; j < 16; ++j) bias4[0][j >> 2][j & 3] = bsb[j];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      wb[j >> 2][j & 3] =
          *reinterpret_cast<const v4i *>(g2.b + ((size_t)ct * 24 + j) * 1024 + lane * 16);
  }
  __syncthreads();
  if (wave < 6) {
    const int8_t *hp = &hid[l32 * kFfnHRow + 16 * h];
    const int8_t *bp = g2.b + (size_t)ct * 24 * 1024 + lane * 16;
    v16i acc[1][1] = {{bsb}};
#pragma unroll
    for (int c = 0; c < 6; ++c) {
      const int cur = c % 3, nxt = (c + 2) % 3;
      if (c + 2 < 6) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          wb[nxt][j] = *reinterpret_cast<const v4i *>(bp + ((c + 2) * 4 + j) * 1024);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
            wb[cur][j], *reinterpret_cast<const v4i *>(hp + (c * 4 + j) * 32), acc[0][0], 0, 0,
            0);
      __builtin_amdgcn_sched_barrier(0);  // one chunk of LDS reads in flight at a time
    }
    epi_tile<1, 1, EPI_RES, true, DIRS2, true>(g2, acc, bias4, res4, r0, ct, M, h, l32, r2a, r2b,
                                         nullptr,
                                         LNE ? reinterpret_cast<int8_t *>(lut) : nullptr,
                                         kLnPrologueRow);
  }
  if constexpr (LNE) {
    __syncthreads();  // every output row is in the table's LDS
    ln_rows16<kLnPrologueRow, 192>(reinterpret_cast<const int8_t *>(lut), kFfn32Rows - 1,
                                   fe.ln.out + (size_t)r0 * 192, M - r0, fe.ln, fe.lw, r0, M - r0);
  }
}

template <int DIRS1, bool LN, bool LNE, bool PJ>
static void launch_ffn32_d(const GemmArgs &g1, const GemmArgs &g2, const LnPrologue &fl,
                           const LnPrologue &fe, const GemmArgs &gp, int dirsp, int dirs2,
                           dim3 grid, hipStream_t s) {
  const dim3 b(512);
  switch (dirs2) {
    case 0: hv_launch(k_ffn32<DIRS1, 0, LN, LNE, PJ>, grid, b, 0, s, g1, g2, fl, fe, gp, dirsp); break;
    case 1: hv_launch(k_ffn32<DIRS1, 1, LN, LNE, PJ>, grid, b, 0, s, g1, g2, fl, fe, gp, dirsp); break;
    case 2: hv_launch(k_ffn32<DIRS1, 2, LN, LNE, PJ>, grid, b, 0, s, g1, g2, fl, fe, gp, dirsp); break;
    default: hv_launch(k_ffn32<DIRS1, 3, LN, LNE, PJ>, grid, b, 0, s, g1, g2, fl, fe, gp, dirsp); break;
  }
}

template <int DIRS1, bool LN, bool LNE, bool PJ>
static void launch_ffn_d(const GemmArgs &g1, const GemmArgs &g2, const LnPrologue &fl,
                         const LnPrologue &fe, const GemmArgs &gp, int dirsp, int dirs2, dim3 grid,
                         int nfull, size_t lds, hipStream_t s) {
  const dim3 b(256);
  const int nf = nfull;
  switch (dirs2) {
    case 0: hv_launch(k_ffn<DIRS1, 0, LN, LNE, PJ>, grid, b, lds, s, g1, g2, fl, fe, gp, dirsp, nf); break;
    case 1: hv_launch(k_ffn<DIRS1, 1, LN, LNE, PJ>, grid, b, lds, s, g1, g2, fl, fe, gp, dirsp, nf); break;
    case 2: hv_launch(k_ffn<DIRS1, 2, LN, LNE, PJ>, grid, b, lds, s, g1, g2, fl, fe, gp, dirsp, nf); break;
    default: hv_launch(k_ffn<DIRS1, 3, LN, LNE, PJ>, grid, b, lds, s, g1, g2, fl, fe, gp, dirsp, nf); break;
  }
}

// CUs of the current device (cached per device; host threads may race to
// fill an entry, all with the same value).  It only places the split of
// ffn_full_blocks: any split gives the same outputs.
static int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (!n) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// The 64-row blocks of a k_ffn launch over m rows, the first nfull of them
// whole and the rest split in two: with q whole rounds of one block per CU
// and r blocks over them (1 <= r <= CUs / 2), the CUs that would run a block
// more than the others (two at once, or one after their last pair) instead
// share its rows with another CU, in 32-row blocks that run beside the
// other CUs' last 64-row block.
static int ffn_full_blocks(int m, bool balanced) {
  const int nrb = (m + kFfnRows - 1) / kFfnRows;
  if (!balanced) return nrb;
  const int cus = device_cus(), q = nrb / cus, r = nrb % cus;
  return q >= 1 && r >= 1 && 2 * r <= cus ? nrb - r : nrb;
}

// Returns HV_OK when the fused kernel was launched, 1 when the shapes or
// exponents need the two GEMM launches instead.
int launch_ffn(const GemmArgs &g1_in, const GemmArgs &g2_in, hipStream_t s,
               const LnPrologue *ln, const LnPrologue *ln_next, const GemmArgs *proj,
               int rows) {
  const bool rows32 = rows == FFN_ROWS32;
  GemmArgs g1 = g1_in, g2 = g2_in;
  GemmArgs gp = proj ? *proj : GemmArgs{};
  if (proj) {
    if (!ln || gp.k != 192 || gp.n != 192 || gp.lda != 192 || gp.ldr != 192 || !gp.a || !gp.b ||
        !gp.bias || !gp.res || gp.aux || gp.a_rows ||
        (((uintptr_t)gp.a | (uintptr_t)gp.bias | (uintptr_t)gp.res) & 15))
      return 1;
    epilogue_limits_pub(gp, EPI_RES);
    if (!fast_epilogue(gp, EPI_RES)) return 1;
  }
  if (g1.k != 192 || g1.n != 768 || g2.k != 768 || g2.n != 192 || g1.lda != 192 ||
      g2.ldc != 192 || g2.ldr != 192 || !g1.bias || !g2.bias || !g2.res || g1.m <= 0)
    return 1;
  if (((uintptr_t)(ln ? nullptr : g1.a) | (uintptr_t)g1.bias | (uintptr_t)g2.bias |
       (uintptr_t)g2.c | (uintptr_t)g2.res | (uintptr_t)g2.aux) & 15)
    return 1;
  if (ln && ((!proj && (!ln->x || ((uintptr_t)ln->x & 7))) || ((uintptr_t)ln->ln.gamma & 7) ||
             ((uintptr_t)ln->ln.beta & 7)))
    return 1;
  if (ln_next && (!ln_next->ln.out || ((uintptr_t)ln_next->ln.out & 7) ||
                  ((uintptr_t)ln_next->ln.gamma & 7) || ((uintptr_t)ln_next->ln.beta & 7)))
    return 1;
  if (g1.shift_b < kGeluLutSoMin || g1.shift_b > kGeluLutSoMax) return 1;
  epilogue_limits_pub(g1, EPI_GELU);
  epilogue_limits_pub(g2, EPI_RES);
  if (!fast_epilogue(g1, EPI_GELU) || !fast_epilogue(g2, EPI_RES)) return 1;
  const GeluLutInfo &t = kGeluLutInfo[g1.shift_b - kGeluLutSoMin];
  g1.lut_off = t.off;
  g1.lut_words = t.words;
  g1.lut_n1e = t.n1e;
  g1.lut_qlo = t.qlo; g1.lut_cb = -4 * (t.qlo >> kGeluCoarseShift);
  g1.lut_qhi = t.qhi;
  g2.vec_out = 1;
  g2.vec_res = 1;
  const size_t lds = 0;  // the table's LDS is static in k_ffn
  // One workgroup per row block (the dispatcher balances them; a persistent
  // grid left half the workgroups with one block more than the others).
  const int nfull = ffn_full_blocks(g1.m, proj && rows == FFN_ROWS64_BALANCED);
  const int rest = g1.m - nfull * kFfnRows;  // rows of the 32-row blocks
  const dim3 grid(nfull + (rest > 0 ? (rest + 31) / 32 : 0));
  const int d1 = epilogue_dirs(g1, EPI_GELU) & 1, d2 = epilogue_dirs(g2, EPI_RES);
  const LnPrologue fl = ln ? *ln : LnPrologue{}, fe = ln_next ? *ln_next : LnPrologue{};
  const int dp = proj ? epilogue_dirs(gp, EPI_RES) : 0;
  const int mode = (ln ? 1 : 0) | (ln_next ? 2 : 0) | (d1 ? 4 : 0);
  if (proj && rows32) {
    const dim3 grid32((g1.m + kFfn32Rows - 1) / kFfn32Rows);
    switch (mode) {
      case 1: launch_ffn32_d<4, true, false, true>(g1, g2, fl, fe, gp, dp, d2, grid32, s); break;
      case 3: launch_ffn32_d<4, true, true, true>(g1, g2, fl, fe, gp, dp, d2, grid32, s); break;
      case 5: launch_ffn32_d<5, true, false, true>(g1, g2, fl, fe, gp, dp, d2, grid32, s); break;
      default: launch_ffn32_d<5, true, true, true>(g1, g2, fl, fe, gp, dp, d2, grid32, s); break;
    }
    return check_hip(hipGetLastError(), "k_ffn32 launch");
  }
  if (proj) {
    switch (mode) {
      case 1: launch_ffn_d<4, true, false, true>(g1, g2, fl, fe, gp, dp, d2, grid, nfull, lds, s); break;
      case 3: launch_ffn_d<4, true, true, true>(g1, g2, fl, fe, gp, dp, d2, grid, nfull, lds, s); break;
      case 5: launch_ffn_d<5, true, false, true>(g1, g2, fl, fe, gp, dp, d2, grid, nfull, lds, s); break;
      default: launch_ffn_d<5, true, true, true>(g1, g2, fl, fe, gp, dp, d2, grid, nfull, lds, s); break;
    }
    return check_hip(hipGetLastError(), "k_ffn launch");
  }
  switch (mode) {
    case 0: launch_ffn_d<4, false, false, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
    case 1: launch_ffn_d<4, true, false, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
    case 2: launch_ffn_d<4, false, true, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
    case 3: launch_ffn_d<4, true, true, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
    case 4: launch_ffn_d<5, false, false, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
    case 5: launch_ffn_d<5, true, false, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
    case 6: launch_ffn_d<5, false, true, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
    default: launch_ffn_d<5, true, true, false>(g1, g2, fl, fe, gp, 0, d2, grid, nfull, lds, s); break;
  }
  return check_hip(hipGetLastError(), "k_ffn launch");
}

// The GELU post-op of the FFN epilogue over int64 Q8.16 values (saturated
// to 24 bits): evaluated as the int32 epilogue does, or from the step table.
__global__ __launch_bounds__(256) void k_gelu_post(int table, const int64_t *in, int64_t *out,
                                                   int64_t n, int so, GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) unsigned lut[];
  if (table) stage_lut(g, lut);
  const Rq rb = rq_setup(so, -128, 127);
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t v = in[i];
    const int q = (int)(v < -(1 << 23) ? -(1 << 23) : (v > (1 << 23) - 1 ? (1 << 23) - 1 : v));
    out[i] = !table ? rq(gelu_q16(q), rb)
                    : (int)(int8_t)gelu_lut(q, lut, g.lut_qhi, g);
  }
}

int launch_gelu_post(bool table, const int64_t *in, int64_t *out, int64_t n, int so,
                     hipStream_t s) {
  if (so < -30 || so > 30)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "GELU post-op shift %d outside [-30, 30]", so);
  GemmArgs g{};
  if (table) {
    if (so < kGeluLutSoMin || so > kGeluLutSoMax)
      return fail(HV_EVALUE, HV_ERR_DIMENSION, "no GELU step table for shift %d (tables: [%d, %d])",
                  so, kGeluLutSoMin, kGeluLutSoMax);
    const GeluLutInfo &t = kGeluLutInfo[so - kGeluLutSoMin];
    g.lut_off = t.off;
    g.lut_words = t.words;
    g.lut_n1e = t.n1e;
    g.lut_qlo = t.qlo; g.lut_cb = -4 * (t.qlo >> kGeluCoarseShift);
    g.lut_qhi = t.qhi;
  }
  if (n <= 0) return HV_OK;
  const int64_t blocks = (n + 255) / 256;
  hv_launch(k_gelu_post, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256),
            (size_t)g.lut_words * 4, s, table ? 1 : 0, in, out, n, so, g);
  return check_hip(hipGetLastError(), "k_gelu_post launch");
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
                       hipStream_t s, bool patch_rows, bool cls_rows) {
  if (batch <= 0) return HV_OK;
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
  g.lda = patch_rows ? 768 : 0;
  int rc = launch_gemm(g, patch_rows ? A_ROWS : A_PATCH, EPI_PATCH, s);
  if (rc || !cls_rows) return rc;
  hv_launch(k_cls_rows, dim3(batch), dim3(192), 0, s, p.cls, p.pos, x, p.cls_exp,
                     p.pos_exp, p.tokens_exp);
  return check_hip(hipGetLastError(), "k_cls_rows launch");
}

}  // namespace hv
