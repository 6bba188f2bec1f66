// hv_internal.h -- launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/heatvit_hip.h"
#include "hv_device.h"

namespace hv {

// Error reporting: a thread-local message and HV_ERR_* class (hv_capi.hip).
int fail(int status, int cls, const char *fmt, ...);
void clear_error();  // entry points start with a clean record
int check_hip(hipError_t e, const char *what);

// Kernel launch.  While kernel-class profiling is on and a class is active
// (hv_capi.hip), prof_events hands out a start/stop event pair that the
// dispatch itself records, so the measured time is the kernel's own.
void prof_events(hipEvent_t *start, hipEvent_t *stop);
template <typename F, typename... Args>
inline void hv_launch(F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t s, Args... args) {
  hipEvent_t a = nullptr, b = nullptr;
  prof_events(&a, &b);
  hipExtLaunchKernelGGL(kernel, grid, block, shm, s, a, b, 0, args...);
}

// Per-image warning sink of the LayerNorm kernels: a row with a negative
// variance ORs HV_WARN_LN_NEGATIVE_VARIANCE into img_warn[b] of the image b
// whose rows offsets[b] .. offsets[b+1] hold it.  img_warn NULL: off.
struct LnWarn {
  const int32_t *offsets;
  int batch;
  int32_t *img_warn;
};

// A-operand sources of the GEMM.
// A_UNSIGNED is a flag bit of the A mode (A_ROWS only).
enum { A_ROWS = HV_A_ROWS, A_GATHER = HV_A_GATHER, A_PATCH = 2, A_UNSIGNED = HV_A_UNSIGNED };

struct GemmArgs {
  const int8_t *a;
  const int32_t *a_rows;
  const int8_t *b;  // mfma32-packed weights
  const int32_t *bias;
  void *c;
  const int8_t *res;
  int8_t *aux;
  const int32_t *m_dev;
  const int8_t *pos;  // patch mode: [197][192] position table
  int m, n, k, lda, ldc, ldr;
  int shift_a;  // epilogue shifts, see k_gemm
  int shift_b;
  int res_exp, mid_exp, out_exp;
  // Filled by launch_gemm: A bytes unsigned (A_UNSIGNED in the A mode).
  int a_unsigned;
  // Filled by launch_gemm: int32 epilogue preconditions.
  int acc_lim;     // a column takes the int32 path when |bias| <= acc_lim
  int narrow_ok;   // acc_lim > 0
  // Optional device word: the largest |bias| of the whole bias tensor (as
  // unsigned).  When it is at most acc_lim every column takes the int32
  // path and the kernels skip their per-tile bias vote.
  const unsigned *bias_max;
  int da, db, os;  // residual / patch align-add shifts
  int vec_out;     // c (and aux) allow 16-byte row stores
  int vec_res;     // res (or pos) allow 16-byte row loads
  // GELU post-op step table (gen_gelu_lut.py), staged in LDS when
  // lut_words > 0: words [lut_off, lut_off + lut_words) of kGeluLut;
  // lut_cb = -4 * (lut_qlo >> kGeluCoarseShift).
  int lut_off, lut_words, lut_n1e, lut_qlo, lut_qhi, lut_cb;
};

// epilogue: HV_EPI_* or 4 (patch: A_PATCH gather, position-row residual).
int launch_gemm(const GemmArgs &g, int a_mode, int epilogue, hipStream_t s);
// FFN1 + GELU + FFN2 + residual in one kernel (hidden rows in LDS): g1 as
// for the GELU GEMM (c unused), g2 as for the residual GEMM (a unused).
// Returns HV_OK when launched, 1 when the shapes or exponents need the two
// GEMM launches (no GELU step table, wide shifts, unaligned pointers).
// ln (optional): the LayerNorm in front of FFN1 runs in the same kernel
// over the rows of ln->x (row stride 192, 8-byte aligned; int32 form of
// ln32_setup, whose output pointer is unused), g1.a unused.  ln_next
// (optional): a LayerNorm of the output rows (the next block's LayerNorm 1)
// runs at the kernel's end and writes ln_next->ln.out (row stride 192;
// ln_next->x unused).  Negative variances reach the lw of each.  proj
// (optional, with ln): the residual GEMM in front of the LayerNorm
// (attention projection: a = ctx rows, res = x, K = N = 192) runs in the
// same kernel and its output rows y feed the LayerNorm and g2's residual
// on the CU: ln->x and g2.res unused, proj->c not written, proj->aux must
// be NULL.
struct LnPrologue {
  const int8_t *x;
  Ln32 ln;
  LnWarn lw;
};
// Row blocking of the fused FFN with proj (the same outputs in each):
//   FFN_ROWS64           blocks of 64 rows by four wavefronts (k_ffn);
//   FFN_ROWS32           blocks of 32 rows by eight wavefronts (k_ffn32), for
//                        batches whose 64-row blocks leave CUs idle;
//   FFN_ROWS64_BALANCED  k_ffn, with the last 64-row blocks split into
//                        32-row ones when the blocks exceed a whole number
//                        of blocks per CU by at most half the CUs.
enum FfnRows { FFN_ROWS64 = 0, FFN_ROWS32 = 1, FFN_ROWS64_BALANCED = 2 };
int launch_ffn(const GemmArgs &g1, const GemmArgs &g2, hipStream_t s,
               const LnPrologue *ln = nullptr, const LnPrologue *ln_next = nullptr,
               const GemmArgs *proj = nullptr, int rows = FFN_ROWS64);
// Fills acc_lim / narrow_ok / da / db / os of the int32 epilogue paths.
void epilogue_limits_pub(GemmArgs &g, int epilogue);

// HV_PRIM_GELU_POST / HV_PRIM_GELU_TABLE (table = true) over n int64 Q8.16
// values with output shift so.
int launch_gelu_post(bool table, const int64_t *in, int64_t *out, int64_t n, int so,
                     hipStream_t s);

// Patch embedding (transformer.patch_embedding): A rows are gathered
// patches of NHWC 224x224x3 images (or, with patch_rows, the patch matrix
// [B*196][768] itself), epilogue adds the position rows, and the CLS rows
// are written by a second small kernel.
// cls_rows false: the CLS rows are written elsewhere (launch_init_offsets).
int launch_patch_embed(const hv_patch_dev &p, const int8_t *images, int batch, int8_t *x,
                       hipStream_t s, bool patch_rows = false, bool cls_rows = true);

// Image front end: float CHW [B][3][224][224] -> int8 at input_exp, as flat
// NHWC images or (patch_rows) as the patch matrix [B*196][768].
int launch_image_front(const float *chw, int batch, int input_exp, int8_t *out, bool patch_rows,
                       hipStream_t s);

// Fills *ln for the int32 LayerNorm path (hv_device.h) when the exponents
// and pointer alignment allow it.
bool ln32_setup(const int8_t *g, const int8_t *b, int8_t *y, int x_exp, int g_exp, int b_exp,
                int out_exp, Ln32 *ln);

// Image of `row` (the last b with offsets[b] <= row, in [0, batch)) gets
// the negative-variance warning bit.  Rare: only rows that clamp reach it.
static __device__ __noinline__ void ln_warn_row(const int32_t *offsets, int batch,
                                                int32_t *img_warn, int row) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] <= row) lo = mid;
    else hi = mid - 1;
  }
  atomicOr(img_warn + lo, HV_WARN_LN_NEGATIVE_VARIANCE);
}

int launch_layernorm(const int8_t *x, const int8_t *g, const int8_t *b, int8_t *y, int rows,
                     const int32_t *rows_dev, int x_exp, int g_exp, int b_exp, int out_exp,
                     uint8_t *neg_var, const LnWarn &lw, hipStream_t s);

struct AttnArgs {
  const int8_t *qkv;  // [T][576]
  const int32_t *offsets;
  int8_t *ctx;        // [T][192]
  int32_t *score;     // optional [B][3][197][197]
  uint8_t *prob;      // optional
  int batch;
  int score_shift;    // score_exp - 2*qkv_out_exp (requant to int32)
  int q16_shift;      // -(score_exp + 13)
  int ctx_shift;      // context_out_exp - (prob_exp + qkv_out_exp)
  int q16_mode, q16_s, q16_rnd;  // int32 fast path for the score -> Q8.16 conversion
  int ctx_fast, ctx_rnd;         // int32 context requant (shift in [1, 30])
  int rows_cap;                  // rows of qkv / ctx; images outside are skipped
  // Fused QKV (ln1 non-NULL): each head's Q, K and V come from the kernel's
  // own GEMM over the LayerNorm 1 rows (row stride 192, the same row
  // offsets), qkv unused.  wqkv mfma32-packed [192][576]; the int8 requant
  // by qkv_shift in [-30, 30] (left: qkv_shift <= 0) takes the int32 form
  // for columns with |bias| <= qkv_acc_lim, the exact one otherwise.
  const int8_t *ln1;
  const int8_t *wqkv;
  const int32_t *bqkv;
  int qkv_shift, qkv_acc_lim;
  const unsigned *bqkv_max;  // optional: largest |bias| of bqkv (GemmArgs::bias_max)
};

// Whether a tensor-wide bias bound (GemmArgs::bias_max) puts every column on
// the int32 path: a uniform scalar load and compare.
__device__ __forceinline__ bool tensor_narrow(const unsigned *bias_max, int acc_lim) {
  return bias_max && acc_lim > 0 && *bias_max <= (unsigned)acc_lim;
}
int launch_attention(const AttnArgs &a, hipStream_t s);

int launch_softmax_rows(const int32_t *x, const int32_t *offsets, int rows, uint8_t *att,
                        int32_t *sel, hipStream_t s);
int launch_primitive(int op, const int64_t *in, int64_t *out, int64_t n, int a, int b, int c,
                     hipStream_t s);

struct SelectorArgs {
  const hv_selector_dev *p;  // host copy passed by value; NULL: fused is an input
  const int8_t *tokens;
  const int32_t *offsets;
  const uint8_t *pkg_in;
  int batch;
  int8_t *out_tokens;
  int32_t *out_offsets;
  uint8_t *pkg_out;
  int32_t *fused;       // [B][196]
  int32_t *kept_index;  // [B][196]
  int32_t *state;       // [B][5]
  int8_t *pkg_rows;     // workspace [B][192]: package rows (selector forward)
  int32_t *token_counts;  // optional [B][4] column `stage`
  int stage;
  int32_t *img_warn;      // optional [B]: the state's warning bits are ORed in
  hv_selector_ckpt ck;    // optional intermediate outputs (null pointers skip)
};
int launch_selector(const SelectorArgs &a, hipStream_t s);

// Small utility kernels.
// cls, x (optional): also writes the CLS row (row 0 of each image's
// HV_MAX_TOKENS rows) of the patch embedding into x.  blocks, bias_max
// (optional): also writes the largest |bias| of each block's bqkv, bproj,
// b1 and b2 to bias_max[4 * block + t] (GemmArgs::bias_max).
int launch_init_offsets(int32_t *offsets, uint8_t *pkg, int32_t *token_counts,
                        int32_t *warnings, int batch, int rows_per_image, hipStream_t s,
                        const hv_patch_dev *cls = nullptr, int8_t *x = nullptr,
                        const hv_block_dev *blocks = nullptr, unsigned *bias_max = nullptr);
// Per-image token-count check of a caller's offsets: status[b] =
// HV_ERR_TOKEN_COUNT unless 1 <= count <= 197 and the rows lie in
// [0, capacity), else 0; warnings[b] = 0.  Either pointer may be NULL.
int launch_image_check(const int32_t *offsets, int batch, int capacity, int32_t *status,
                       int32_t *warnings, hipStream_t s);
int launch_copy_ckpt(const int8_t *x, const int32_t *offsets, int batch, int8_t *ckpt,
                     int32_t *ckpt_rows, int slot, hipStream_t s);
int launch_cls_rows(const int32_t *offsets, int batch, int32_t *rows_out, hipStream_t s);

}  // namespace hv
