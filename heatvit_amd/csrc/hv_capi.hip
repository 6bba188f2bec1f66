// hv_capi.hip -- extern "C" entry points of libheatvit_hip.so and the host
// orchestration of the block, selector and full-model forwards.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "hv_device.h"
#include "hv_internal.h"

namespace hv {

static thread_local char g_err[512];
static thread_local int g_err_class = HV_ERR_NONE;

int fail(int status, int cls, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  g_err_class = cls;
  return status;
}

int check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess) return HV_OK;
  return fail(HV_EHIP, HV_ERR_MEMORY_PROTOCOL, "%s: %s", what, hipGetErrorString(e));
}

void clear_error() {
  g_err[0] = 0;
  g_err_class = HV_ERR_NONE;
}

// ---------------------------------------------------------------- profiling
// With profiling on, every kernel launched inside a class scope carries a
// start/stop event pair that its dispatch records (hipExtLaunchKernelGGL),
// so each interval is the kernel's own execution; hv_profile_read() sums
// them per kernel class.  Host-side state: one profiling client at a time.

struct ProfEvent {
  int cls;
  hipEvent_t a, b;
};
static bool g_prof_on = false;
static std::vector<ProfEvent> g_prof;

// Active kernel class of the calling thread (-1: none).
static thread_local int g_prof_cls = -1;

struct ProfScope {
  int prev;
  ProfScope(int c, hipStream_t) : prev(g_prof_cls) { g_prof_cls = c; }
  ~ProfScope() { g_prof_cls = prev; }
};

void prof_events(hipEvent_t *start, hipEvent_t *stop) {
  *start = *stop = nullptr;
  if (!g_prof_on || g_prof_cls < 0) return;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return;
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    return;
  }
  g_prof.push_back({g_prof_cls, a, b});
  *start = a;
  *stop = b;
}

static void prof_clear() {
  for (auto &e : g_prof) {
    (void)hipEventDestroy(e.a);
    (void)hipEventDestroy(e.b);
  }
  g_prof.clear();
}

// ---------------------------------------------------------------- utilities

// cls (optional): row 0 of each image's 197 rows in x is the CLS row,
// align_add(cls, pos[0]) (transformer.py:130-145), written here rather than
// by a launch of its own after the patch embedding.
// The model's GEMM bias tensors whose largest |bias| the first kernel of a
// forward writes (GemmArgs::bias_max): entry 4 * block + t for t = 0 bqkv,
// 1 bproj, 2 b1, 3 b2.
struct BiasJobs {
  const int32_t *p[48];
  unsigned *out;
};
__device__ constexpr int kBiasCount[4] = {576, 192, 768, 192};

__global__ void k_init_offsets(int32_t *offsets, uint8_t *pkg, int32_t *token_counts,
                               int32_t *warnings, int batch, int rows, hv_patch_dev cls,
                               int8_t *x, BiasJobs bj, int init_blocks) {
  if ((int)blockIdx.x >= init_blocks) {  // uniform: one bias tensor per workgroup
    __shared__ unsigned red[4];
    const int j = blockIdx.x - init_blocks, n = kBiasCount[j & 3];
    unsigned m = 0;
    for (int k = threadIdx.x; k < n; k += blockDim.x) {
      const int b = bj.p[j][k];
      m = max(m, b < 0 ? 0u - (unsigned)b : (unsigned)b);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) bj.out[j] = max(max(red[0], red[1]), max(red[2], red[3]));
    return;
  }
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= batch) offsets[i] = i * rows;
  if (i < batch) {
    pkg[i] = 0;
    if (token_counts)
      for (int s = 0; s < 4; ++s) token_counts[(size_t)i * 4 + s] = rows;
    if (warnings) warnings[i] = 0;
  }
  if (x)
    for (int j = i; j < batch * 192; j += gridDim.x * blockDim.x) {
      const int b = j / 192, c = j - b * 192;
      x[(size_t)b * HV_MAX_TOKENS * 192 + c] =
          (int8_t)align_add_i8(cls.cls[c], cls.cls_exp, cls.pos[c], cls.pos_exp, cls.tokens_exp);
    }
}

int launch_init_offsets(int32_t *offsets, uint8_t *pkg, int32_t *token_counts,
                        int32_t *warnings, int batch, int rows, hipStream_t s,
                        const hv_patch_dev *cls, int8_t *x, const hv_block_dev *blocks,
                        unsigned *bias_max) {
  // batch + 1 offsets; with the CLS rows, batch * 192 bytes (a superset);
  // with blocks, 48 more workgroups for the bias bounds
  const int items = cls && x ? batch * 192 : batch + 1;
  const int init_blocks = (items + 255) / 256;
  BiasJobs bj{};
  const bool bias = blocks && bias_max;
  if (bias) {
    for (int i = 0; i < 12; ++i) {
      bj.p[4 * i] = blocks[i].bqkv;
      bj.p[4 * i + 1] = blocks[i].bproj;
      bj.p[4 * i + 2] = blocks[i].b1;
      bj.p[4 * i + 3] = blocks[i].b2;
    }
    bj.out = bias_max;
  }
  hv_launch(k_init_offsets, dim3(init_blocks + (bias ? 48 : 0)), dim3(256), 0, s, offsets, pkg,
            token_counts, warnings, batch, rows, cls ? *cls : hv_patch_dev{}, cls ? x : nullptr,
            bj, init_blocks);
  return check_hip(hipGetLastError(), "k_init_offsets launch");
}

// The attention's skip condition (k_attention), reported per image.
__global__ void k_image_check(const int32_t *offsets, int batch, int capacity, int32_t *status,
                              int32_t *warnings) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int row0 = offsets[b], n = offsets[b + 1] - row0;
  const bool ok = n >= 1 && n <= HV_MAX_TOKENS && row0 >= 0 && row0 <= capacity - n;
  if (status) status[b] = ok ? HV_ERR_NONE : HV_ERR_TOKEN_COUNT;
  if (warnings) warnings[b] = 0;
}

int launch_image_check(const int32_t *offsets, int batch, int capacity, int32_t *status,
                       int32_t *warnings, hipStream_t s) {
  if (!status && !warnings) return HV_OK;
  hv_launch(k_image_check, dim3((batch + 255) / 256), dim3(256), 0, s, offsets, batch, capacity,
            status, warnings);
  return check_hip(hipGetLastError(), "k_image_check launch");
}

__global__ void k_copy_ckpt(const int8_t *x, const int32_t *offsets, int8_t *ckpt,
                            int32_t *ckpt_rows, int slot) {
  const int b = blockIdx.x;
  const int r0 = offsets[b], n = offsets[b + 1] - r0;
  int8_t *dst = ckpt + ((size_t)b * 17 + slot) * 197 * 192;
  for (int i = threadIdx.x; i < n * 12; i += blockDim.x)
    reinterpret_cast<v4i *>(dst)[i] = reinterpret_cast<const v4i *>(x + (size_t)r0 * 192)[i];
  if (threadIdx.x == 0 && ckpt_rows) ckpt_rows[(size_t)b * 17 + slot] = n;
}

int launch_copy_ckpt(const int8_t *x, const int32_t *offsets, int batch, int8_t *ckpt,
                     int32_t *ckpt_rows, int slot, hipStream_t s) {
  hv_launch(k_copy_ckpt, dim3(batch), dim3(256), 0, s, x, offsets, ckpt, ckpt_rows,
                     slot);
  return check_hip(hipGetLastError(), "k_copy_ckpt launch");
}

// Bump allocator over the caller's workspace (256-byte aligned slices).
struct Carve {
  uint8_t *base;
  size_t cap, used = 0;
  bool ok = true;
  template <class T>
  T *take(size_t count) {
    size_t off = (used + 255) & ~(size_t)255;
    size_t bytes = count * sizeof(T);
    if (base && off + bytes > cap) ok = false;
    used = off + bytes;
    return base && ok ? reinterpret_cast<T *>(base + off) : nullptr;
  }
};

struct BlockWs {
  int8_t *ln, *qkv, *ctx, *y, *hidden;
};

static BlockWs carve_block(Carve &cv, size_t rows) {
  BlockWs w;
  w.ln = cv.take<int8_t>(rows * 192);
  w.qkv = cv.take<int8_t>(rows * 576);
  w.ctx = cv.take<int8_t>(rows * 192);
  w.y = cv.take<int8_t>(rows * 192);
  w.hidden = cv.take<int8_t>(rows * 768);
  return w;
}

// Chaining of LayerNorm 1 between consecutive blocks of the model: ln1_in
// (optional) holds this block's LayerNorm 1 of x, written by the previous
// block's FFN kernel; next (optional) is the following block, whose
// LayerNorm 1 of z this block's FFN kernel then writes to next_ln1 when it
// can (*next_done tells).
struct LnChain {
  const int8_t *ln1_in;
  const hv_block_dev *next;
  int8_t *next_ln1;
  bool *next_done;
};

// Whether the fused FFN's 64-row blocks of `rows` rows fill less than one
// round of the GPU's 256 CUs at two workgroups each (then blocks of 32 rows
// finish sooner, one forward at a time).
static bool small_rows(long long rows) { return rows < 2 * 256 * 64; }

// Images per batch from which the attention kernel runs the QKV GEMM.
static constexpr int kFusedQkvMinBatch = 32;

// transformer_block (transformer.py:401-431) on rows [0, offsets[batch]):
// LN1, QKV, attention, proj + residual, LN2, FFN1 + GELU, FFN2 + residual.
// warnings (optional, [B]) receive the LayerNorms' negative-variance bit.
// bias_max (optional, device): the largest |bias| of bqkv, bproj, b1 and b2.
// ffn_rows: the fused FFN's row blocking (FfnRows, launch_ffn).
static int block_forward(const hv_block_dev &p, const int8_t *x, const int32_t *offsets,
                         int batch, int max_rows, int8_t *z, const hv_block_ckpt *ck,
                         int32_t *warnings, const BlockWs &w, hipStream_t s,
                         const LnChain &chain = LnChain{}, const unsigned *bias_max = nullptr,
                         int ffn_rows = FFN_ROWS64) {
  const int32_t *rows_dev = offsets + batch;
  const LnWarn lw{offsets, batch, warnings};
  int8_t *qkv = ck && ck->fused_qkv ? ck->fused_qkv : w.qkv;
  int8_t *ctx = ck && ck->concat ? ck->concat : w.ctx;
  int8_t *y = ck && ck->y ? ck->y : w.y;
  int8_t *hidden = ck && ck->hidden ? ck->hidden : w.hidden;
  int rc;

  int8_t *ln1_out = ck && ck->ln1 ? ck->ln1 : w.ln;
  int8_t *ln2 = ck && ck->ln2 ? ck->ln2 : w.ln;
  if (chain.next_done) *chain.next_done = false;
  // QKV reads LayerNorm 1 from the previous block's FFN kernel when it wrote
  // it, else from this block's own LayerNorm launch.
  const bool chained_in = chain.ln1_in && !ck;
  const int8_t *ln1 = chained_in ? chain.ln1_in : ln1_out;
  if (!chained_in) {
    ProfScope ps(HV_PROF_LAYERNORM, s);
    rc = launch_layernorm(x, p.ln1_gamma, p.ln1_beta, ln1_out, max_rows, rows_dev, p.x_exp,
                          p.gamma1_exp, p.beta1_exp, p.ln1_out_exp, nullptr, lw, s);
    if (rc) return rc;
  }
  GemmArgs g{};
  g.a = ln1; g.b = p.wqkv_p; g.bias = p.bqkv; g.c = qkv; g.m_dev = rows_dev;
  g.bias_max = bias_max;
  g.m = max_rows; g.n = 576; g.k = 192; g.lda = 192; g.ldc = 576;
  g.shift_a = p.qkv_out_exp - (p.ln1_out_exp + p.wqkv_exp);
  // Without checkpoints the attention kernel computes each head's Q, K and
  // V itself when their requant takes the int32 form: qkv never reaches
  // memory.  Small batches keep the separate GEMM: with a few workgroups
  // per head the in-kernel GEMM would run on a few CUs in series with the
  // attention (one image: 0.63 ms → 0.67 ms per forward).
  epilogue_limits_pub(g, HV_EPI_I8);
  const bool fuse_qkv = !ck && batch >= kFusedQkvMinBatch && g.narrow_ok && g.shift_a >= -30 &&
                        g.shift_a <= 30 &&
                        !(((uintptr_t)ln1 | (uintptr_t)p.wqkv_p | (uintptr_t)p.bqkv) & 15);
  if (!fuse_qkv) {
    ProfScope ps(HV_PROF_GEMM_QKV, s);
    rc = launch_gemm(g, A_ROWS, HV_EPI_I8, s);
    if (rc) return rc;
  }

  AttnArgs a{};
  if (fuse_qkv) {
    a.ln1 = ln1; a.wqkv = p.wqkv_p; a.bqkv = p.bqkv;
    a.qkv_shift = g.shift_a; a.qkv_acc_lim = g.acc_lim; a.bqkv_max = bias_max;
  }
  a.qkv = qkv; a.offsets = offsets; a.ctx = ctx; a.batch = batch; a.rows_cap = max_rows;
  a.score = ck ? ck->score : nullptr;
  a.prob = ck ? ck->prob : nullptr;
  a.score_shift = p.score_exp - 2 * p.qkv_out_exp;
  a.q16_shift = -(p.score_exp + 13);
  a.ctx_shift = p.context_out_exp - (p.prob_exp + p.qkv_out_exp);
  {
    ProfScope ps(HV_PROF_ATTENTION, s);
    rc = launch_attention(a, s);
  }
  if (rc) return rc;

  g = GemmArgs{};
  g.a = ctx; g.b = p.wproj_p; g.bias = p.bproj; g.c = y; g.res = x; g.aux = ck ? ck->msa : nullptr;
  g.bias_max = bias_max ? bias_max + 1 : nullptr;
  g.m_dev = rows_dev; g.m = max_rows; g.n = 192; g.k = 192; g.lda = 192; g.ldc = 192; g.ldr = 192;
  g.shift_a = p.msa_out_exp - (p.context_out_exp + p.wproj_exp);
  g.mid_exp = p.msa_out_exp; g.res_exp = p.x_exp; g.out_exp = p.ffn_x_exp;

  GemmArgs g1{};
  g1.a = ln2; g1.b = p.w1_p; g1.bias = p.b1; g1.c = hidden; g1.m_dev = rows_dev;
  g1.bias_max = bias_max ? bias_max + 2 : nullptr;
  g1.m = max_rows; g1.n = 768; g1.k = 192; g1.lda = 192; g1.ldc = 768;
  g1.shift_a = -16 - (p.ln2_out_exp + p.w1_exp);
  g1.shift_b = p.hidden_out_exp + 16;
  GemmArgs g2{};
  g2.a = hidden; g2.b = p.w2_p; g2.bias = p.b2; g2.c = z; g2.res = y;
  g2.bias_max = bias_max ? bias_max + 3 : nullptr;
  g2.aux = ck ? ck->ffn_out : nullptr;
  g2.m_dev = rows_dev; g2.m = max_rows; g2.n = 192; g2.k = 768; g2.lda = 768; g2.ldc = 192;
  g2.ldr = 192;
  g2.shift_a = p.ffn_out_exp - (p.hidden_out_exp + p.w2_exp);
  g2.mid_exp = p.ffn_out_exp; g2.res_exp = p.ffn_x_exp; g2.out_exp = p.out_exp;
  // LayerNorm 2 inside the fused FFN kernel (its rows pass through LDS)
  // when neither its output nor the hidden rows are wanted and its
  // exponents take the int32 form; the next block's LayerNorm 1 of z at the
  // kernel's end when its exponents take the int32 form.
  Ln32 ln, ln_n;
  const bool ln2_in = !(ck && (ck->hidden || ck->ln2)) &&
                      ln32_setup(p.ln2_gamma, p.ln2_beta, ln2, p.ffn_x_exp, p.gamma2_exp,
                                 p.beta2_exp, p.ln2_out_exp, &ln);
  const hv_block_dev *nx = ck ? nullptr : chain.next;
  const bool chained = ln2_in && nx && chain.next_ln1 &&
                       ln32_setup(nx->ln1_gamma, nx->ln1_beta, chain.next_ln1, nx->x_exp,
                                  nx->gamma1_exp, nx->beta1_exp, nx->ln1_out_exp, &ln_n);
  const LnPrologue fe{nullptr, ln_n, lw};
  // Without checkpoints the projection runs in the fused FFN kernel too, y
  // staying on the CU.
  if (ln2_in && !ck) {
    const LnPrologue fl{nullptr, ln, lw};
    ProfScope ps(HV_PROF_FFN, s);
    rc = launch_ffn(g1, g2, s, &fl, chained ? &fe : nullptr, &g, ffn_rows);
    if (rc != 1) {
      if (rc == HV_OK && chained && chain.next_done) *chain.next_done = true;
      return rc;
    }
  }
  {
    ProfScope ps(HV_PROF_GEMM_PROJ, s);
    rc = launch_gemm(g, A_ROWS, HV_EPI_RESIDUAL, s);
  }
  if (rc) return rc;
  if (ln2_in) {
    const LnPrologue fl{y, ln, lw};
    ProfScope ps(HV_PROF_FFN, s);
    rc = launch_ffn(g1, g2, s, &fl, chained ? &fe : nullptr);
    if (rc != 1) {
      if (rc == HV_OK && chained && chain.next_done) *chain.next_done = true;
      return rc;
    }
  }
  {
    ProfScope ps(HV_PROF_LAYERNORM, s);
    rc = launch_layernorm(y, p.ln2_gamma, p.ln2_beta, ln2, max_rows, rows_dev, p.ffn_x_exp,
                          p.gamma2_exp, p.beta2_exp, p.ln2_out_exp, nullptr, lw, s);
  }
  if (rc) return rc;
  // One fused kernel (hidden rows in LDS) unless the hidden checkpoint is
  // wanted or the exponents need the general epilogues.
  if (!(ck && ck->hidden)) {
    ProfScope ps(HV_PROF_FFN, s);
    rc = launch_ffn(g1, g2, s);
    if (rc != 1) return rc;
  }
  {
    ProfScope ps(HV_PROF_GEMM_FFN1, s);
    rc = launch_gemm(g1, A_ROWS, HV_EPI_GELU, s);
  }
  if (rc) return rc;
  ProfScope ps(HV_PROF_GEMM_FFN2, s);
  return launch_gemm(g2, A_ROWS, HV_EPI_RESIDUAL, s);
}

static bool exp_ok(int e) { return e >= -32 && e <= 31; }

static int check_block(const hv_block_dev &p) {
  const int e[] = {p.x_exp, p.gamma1_exp, p.beta1_exp, p.ln1_out_exp, p.wqkv_exp,
                   p.qkv_out_exp, p.score_exp, p.prob_exp, p.context_out_exp, p.wproj_exp,
                   p.msa_out_exp, p.ffn_x_exp, p.gamma2_exp, p.beta2_exp, p.ln2_out_exp,
                   p.w1_exp, p.hidden_out_exp, p.w2_exp, p.ffn_out_exp, p.out_exp};
  for (int v : e)
    if (!exp_ok(v))
      return fail(HV_EVALUE, HV_ERR_DIMENSION, "block scale exponent %d outside [-32, 31]", v);
  if (p.x_exp > 0 || p.ffn_x_exp > 0)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "layernorm input scale must be in [-32, 0]");
  return HV_OK;
}

}  // namespace hv

using namespace hv;

extern "C" {

const char *hv_last_error(void) { return g_err; }

int hv_last_error_class(void) { return g_err_class; }

int hv_abi_version(void) { return 5; }

int hv_eval_primitive(int op, const int64_t *in, int64_t *out, int64_t n, int a, int b, int c,
                      hv_stream_t stream) {
  clear_error();
  return launch_primitive(op, in, out, n, a, b, c, (hipStream_t)stream);
}

int hv_softmax_rows(const int32_t *x, const int32_t *offsets, int rows, uint8_t *attention,
                    int32_t *selector, hv_stream_t stream) {
  clear_error();
  return launch_softmax_rows(x, offsets, rows, attention, selector, (hipStream_t)stream);
}

int hv_layernorm_i8(const int8_t *x, const int8_t *gamma, const int8_t *beta, int8_t *y,
                    int rows, const int32_t *rows_dev, int x_exp, int gamma_exp, int beta_exp,
                    int out_exp, uint8_t *neg_var, hv_stream_t stream) {
  clear_error();
  return launch_layernorm(x, gamma, beta, y, rows, rows_dev, x_exp, gamma_exp, beta_exp,
                          out_exp, neg_var, LnWarn{}, (hipStream_t)stream);
}

int hv_attention_i8(const int8_t *qkv, const int32_t *offsets, int batch, int rows, int8_t *ctx,
                    int32_t *score, uint8_t *prob, int qkv_exp, int score_exp, int prob_exp,
                    int context_exp, int32_t *status, hv_stream_t stream) {
  clear_error();
  if (!qkv || !offsets || !ctx) return fail(HV_EVALUE, HV_ERR_ADDRESS, "attention: null argument");
  if (batch <= 0 || rows <= 0)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "attention: empty batch");
  for (int v : {qkv_exp, score_exp, prob_exp, context_exp})
    if (!exp_ok(v))
      return fail(HV_EVALUE, HV_ERR_DIMENSION, "attention scale exponent %d outside [-32, 31]",
                  v);
  if (((uintptr_t)qkv & 15) || ((uintptr_t)ctx & 3))
    return fail(HV_EVALUE, HV_ERR_ADDRESS,
                "attention: qkv must be 16-byte and ctx 4-byte aligned");
  const hipStream_t s = (hipStream_t)stream;
  int rc = launch_image_check(offsets, batch, rows, status, nullptr, s);
  if (rc) return rc;
  AttnArgs a{};
  a.qkv = qkv; a.offsets = offsets; a.ctx = ctx; a.batch = batch; a.rows_cap = rows;
  a.score = score; a.prob = prob;
  a.score_shift = score_exp - 2 * qkv_exp;
  a.q16_shift = -(score_exp + 13);
  a.ctx_shift = context_exp - (prob_exp + qkv_exp);
  return launch_attention(a, s);
}

int hv_gemm_i8(const hv_gemm_desc *d, hv_stream_t stream) {
  clear_error();
  if (!d) return fail(HV_EVALUE, HV_ERR_ADDRESS, "gemm: null descriptor");
  GemmArgs g{};
  g.a = d->a; g.a_rows = d->a_rows; g.b = d->b_packed; g.bias = d->bias; g.c = d->c;
  g.res = d->residual; g.aux = d->aux; g.m_dev = d->m_dev;
  g.m = d->m; g.n = d->n; g.k = d->k; g.lda = d->lda; g.ldc = d->ldc; g.ldr = d->ldr;
  switch (d->epilogue) {
    case HV_EPI_I8:
    case HV_EPI_I32: g.shift_a = d->dst_exp - d->src_exp; break;
    case HV_EPI_GELU:
      g.shift_a = -16 - d->src_exp;
      g.shift_b = d->dst_exp + 16;
      break;
    case HV_EPI_RESIDUAL:
      if (!d->residual)
        return fail(HV_EVALUE, HV_ERR_ADDRESS, "gemm: residual epilogue needs a residual");
      g.shift_a = d->mid_exp - d->src_exp;
      g.mid_exp = d->mid_exp; g.res_exp = d->res_exp; g.out_exp = d->dst_exp;
      break;
    default: return fail(HV_EVALUE, HV_ERR_OPCODE, "gemm: bad epilogue %d", d->epilogue);
  }
  if (d->a_mode == HV_A_GATHER && !d->a_rows)
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "gemm: gather without rows");
  return launch_gemm(g, d->a_mode, d->epilogue, (hipStream_t)stream);
}

size_t hv_block_workspace_bytes(int batch, int max_rows) {
  (void)batch;
  Carve cv{nullptr, 0};
  carve_block(cv, (size_t)max_rows);
  return cv.used + 256;
}

int hv_block_forward(const hv_block_dev *p, const int8_t *x, const int32_t *offsets, int batch,
                     int max_rows, int8_t *z, const hv_block_ckpt *ck, int32_t *status,
                     int32_t *warnings, void *workspace, size_t workspace_bytes,
                     hv_stream_t stream) {
  clear_error();
  if (!p || !x || !offsets || !z) return fail(HV_EVALUE, HV_ERR_ADDRESS, "block: null argument");
  if (batch <= 0 || max_rows <= 0) return fail(HV_EVALUE, HV_ERR_DIMENSION, "block: empty batch");
  int rc = check_block(*p);
  if (rc) return rc;
  Carve cv{(uint8_t *)workspace, workspace_bytes};
  BlockWs w = carve_block(cv, (size_t)max_rows);
  if (!cv.ok || !workspace) return fail(HV_EVALUE, HV_ERR_ADDRESS, "block: workspace too small");
  if ((rc = launch_image_check(offsets, batch, max_rows, status, warnings, (hipStream_t)stream)))
    return rc;
  return block_forward(*p, x, offsets, batch, max_rows, z, ck, warnings, w, (hipStream_t)stream,
                       LnChain{}, nullptr,
                       small_rows(max_rows) ? FFN_ROWS32 : FFN_ROWS64_BALANCED);
}

struct SelectorWs {
  int8_t *pkg_rows;
};

static SelectorWs carve_selector(Carve &cv, int batch) {
  SelectorWs w;
  w.pkg_rows = cv.take<int8_t>((size_t)batch * 192);
  return w;
}

size_t hv_selector_workspace_bytes(int batch) {
  if (batch <= 0) return 0;
  Carve cv{nullptr, 0};
  carve_selector(cv, batch);
  return cv.used;
}

int hv_selector_forward(const hv_selector_dev *p, const int8_t *tokens, const int32_t *offsets,
                        const uint8_t *pkg_in, int batch, int8_t *out_tokens,
                        int32_t *out_offsets, uint8_t *pkg_out, int32_t *fused,
                        int32_t *kept_index, int32_t *state, const hv_selector_ckpt *ck,
                        void *workspace, size_t workspace_bytes, hv_stream_t stream) {
  clear_error();
  if (!p || !tokens || !offsets || !out_tokens || !out_offsets || !pkg_out || !fused ||
      !kept_index || !state)
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "selector: null argument");
  if (batch <= 0) return HV_OK;
  Carve cv{(uint8_t *)workspace, workspace_bytes};
  const SelectorWs w = carve_selector(cv, batch);
  if (!cv.ok || !workspace) return fail(HV_EVALUE, HV_ERR_ADDRESS, "selector: workspace too small");
  SelectorArgs a{};
  a.pkg_rows = w.pkg_rows;
  a.p = p; a.tokens = tokens; a.offsets = offsets; a.pkg_in = pkg_in; a.batch = batch;
  a.out_tokens = out_tokens; a.out_offsets = out_offsets; a.pkg_out = pkg_out; a.fused = fused;
  a.kept_index = kept_index; a.state = state;
  if (ck) a.ck = *ck;
  return launch_selector(a, (hipStream_t)stream);
}

}  // extern "C"

namespace hv {
// Scratch of hv_selector_forward_noalloc: the selector workspace carved for
// HV_SELECTOR_NOALLOC_MAX_BATCH images.  Host code never uses the array's
// name as an address: each device's copy is found once with
// hipGetSymbolAddress (with that device current) and kept per device.
static constexpr size_t kNoAllocScratchBytes = 256 * 1024;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int noalloc_scratch(void **out) {
  int dev = -1;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "selector noalloc: device %d beyond %d", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress");
    if (rc) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return HV_OK;
}
}  // namespace hv

extern "C" {

int hv_selector_forward_noalloc(const hv_selector_dev *p, const int8_t *tokens,
                                const int32_t *offsets, const uint8_t *pkg_in, int batch,
                                int8_t *out_tokens, int32_t *out_offsets, uint8_t *pkg_out,
                                int32_t *fused, int32_t *kept_index, int32_t *state,
                                const hv_selector_ckpt *ck, hv_stream_t stream) {
  clear_error();
  if (batch > HV_SELECTOR_NOALLOC_MAX_BATCH)
    return fail(HV_EVALUE, HV_ERR_DIMENSION,
                "selector noalloc: batch %d exceeds the fixed scratch's %d images", batch,
                HV_SELECTOR_NOALLOC_MAX_BATCH);
  static_assert(kNoAllocScratchBytes >= (size_t)HV_SELECTOR_NOALLOC_MAX_BATCH * 192 + 256,
                "scratch holds the selector workspace of the largest batch");
  if (batch <= 0) return hv_selector_forward(p, tokens, offsets, pkg_in, batch, out_tokens,
                                             out_offsets, pkg_out, fused, kept_index, state, ck,
                                             nullptr, 0, stream);
  void *ws = nullptr;
  int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  const size_t need = hv_selector_workspace_bytes(batch);
  if (need > kNoAllocScratchBytes)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "selector noalloc: workspace %zu > scratch %zu",
                need, kNoAllocScratchBytes);
  return hv_selector_forward(p, tokens, offsets, pkg_in, batch, out_tokens, out_offsets, pkg_out,
                             fused, kept_index, state, ck, ws, kNoAllocScratchBytes, stream);
}

int hv_selector_finalize(const int8_t *tokens, const int32_t *offsets, const uint8_t *pkg_in,
                         const int32_t *fused, int batch, int8_t *out_tokens,
                         int32_t *out_offsets, uint8_t *pkg_out, int32_t *kept_index,
                         int32_t *state, hv_stream_t stream) {
  clear_error();
  if (!tokens || !offsets || !fused || !out_tokens || !out_offsets || !pkg_out || !kept_index ||
      !state)
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "finalize: null argument");
  SelectorArgs a{};
  a.p = nullptr; a.tokens = tokens; a.offsets = offsets; a.pkg_in = pkg_in; a.batch = batch;
  a.out_tokens = out_tokens; a.out_offsets = out_offsets; a.pkg_out = pkg_out;
  a.fused = const_cast<int32_t *>(fused); a.kept_index = kept_index; a.state = state;
  return launch_selector(a, (hipStream_t)stream);
}

int hv_patch_embedding(const hv_patch_dev *p, const int8_t *images, int batch, int8_t *x,
                       hv_stream_t stream) {
  clear_error();
  if (!p || !images || !x) return fail(HV_EVALUE, HV_ERR_ADDRESS, "patch: null argument");
  const int e[] = {p->image_exp, p->weight_exp, p->activation_exp, p->tokens_exp, p->cls_exp,
                   p->pos_exp};
  for (int v : e)
    if (!exp_ok(v))
      return fail(HV_EVALUE, HV_ERR_DIMENSION, "patch scale exponent %d outside [-32, 31]", v);
  return launch_patch_embed(*p, images, batch, x, (hipStream_t)stream);
}

struct ModelWs {
  int8_t *xa, *xb;
  BlockWs blk;
  int32_t *off_a, *off_b, *fused, *kept, *state;
  uint8_t *pkg_a, *pkg_b;
  unsigned *bias_max;  // [12][4], k_init_offsets
  SelectorWs sel;
};

static ModelWs carve_model(Carve &cv, int batch) {
  const size_t rows = (size_t)batch * HV_MAX_TOKENS;
  ModelWs w;
  w.xa = cv.take<int8_t>(rows * 192);
  w.xb = cv.take<int8_t>(rows * 192);
  w.blk = carve_block(cv, rows);
  w.off_a = cv.take<int32_t>(batch + 1);
  w.off_b = cv.take<int32_t>(batch + 1);
  w.fused = cv.take<int32_t>((size_t)batch * 196);
  w.kept = cv.take<int32_t>((size_t)batch * 196);
  w.state = cv.take<int32_t>((size_t)batch * 3 * 5);
  w.pkg_a = cv.take<uint8_t>(batch);
  w.pkg_b = cv.take<uint8_t>(batch);
  w.bias_max = cv.take<unsigned>(48);
  w.sel = carve_selector(cv, batch);
  return w;
}

size_t hv_model_workspace_bytes(int batch) {
  Carve cv{nullptr, 0};
  carve_model(cv, batch);
  return cv.used + 256;
}

// HeatViTModel.infer over a batch; images are int8 NHWC or, with
// float_images, float CHW quantised at the patch's image exponent on the way
// into the patch matrix.
static int model_forward(const hv_model_dev *p, const void *images, bool float_images, int batch,
                         int32_t *logits, int32_t *token_counts, int32_t *state,
                         int32_t *warnings, int8_t *ckpt, int32_t *ckpt_rows, void *workspace,
                         size_t workspace_bytes, int options, hipStream_t s) {
  if (!p || !images || !logits) return fail(HV_EVALUE, HV_ERR_ADDRESS, "model: null argument");
  if (batch <= 0) return fail(HV_EVALUE, HV_ERR_DIMENSION, "model: empty batch");
  if ((long long)batch * HV_MAX_TOKENS * 768 > 0x7fffffffLL)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "model: batch %d too large", batch);
  if (p->n_selectors < 0 || p->n_selectors > 3)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "model: bad selector count");
  for (int i = 0; i < 12; ++i) {
    int rc = check_block(p->blocks[i]);
    if (rc) return rc;
  }
  if (p->blocks[11].out_exp > 0)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "layernorm input scale must be in [-32, 0]");
  Carve cv{(uint8_t *)workspace, workspace_bytes};
  ModelWs w = carve_model(cv, batch);
  if (!cv.ok || !workspace) return fail(HV_EVALUE, HV_ERR_ADDRESS, "model: workspace too small");
  const int max_rows = batch * HV_MAX_TOKENS;
  int32_t *st = state ? state : w.state;
  int rc;

  {
    ProfScope ps(HV_PROF_OTHER, s);
    rc = launch_init_offsets(w.off_a, w.pkg_a, token_counts, warnings, batch, HV_MAX_TOKENS,
                             s, &p->patch, w.xa, p->blocks, w.bias_max);
  }
  if (rc) return rc;
  {
    ProfScope ps(HV_PROF_PATCH, s);
    if (float_images) {
      // the FFN hidden buffer ([B*197][768]) is free until block 1's FFN
      rc = launch_image_front(static_cast<const float *>(images), batch, p->patch.image_exp,
                              w.blk.hidden, true, s);
      if (rc == HV_OK)
        rc = launch_patch_embed(p->patch, w.blk.hidden, batch, w.xa, s, true, false);
    } else {
      rc = launch_patch_embed(p->patch, static_cast<const int8_t *>(images), batch, w.xa, s,
                              false, false);
    }
  }
  if (rc) return rc;
  if (ckpt && (rc = launch_copy_ckpt(w.xa, w.off_a, batch, ckpt, ckpt_rows, 0, s))) return rc;

  int sel = 0;
  const int8_t *ln1_ready = nullptr;  // this block's LayerNorm 1, from the previous FFN
  // The final LayerNorm (model.py:102-106) as the "next LayerNorm" of block
  // 12's FFN kernel: the same fields in the layout the chain reads.
  hv_block_dev fin{};
  fin.ln1_gamma = p->final_gamma;
  fin.ln1_beta = p->final_beta;
  fin.x_exp = p->blocks[11].out_exp;
  fin.gamma1_exp = p->final_gamma_exp;
  fin.beta1_exp = p->final_beta_exp;
  fin.ln1_out_exp = p->final_ln_out_exp;
  bool final_done = false;
  for (int blk = 1; blk <= 12; ++blk) {
    if (sel < p->n_selectors && p->selector_blocks[sel] == blk) {
      SelectorArgs a{};
      a.p = &p->selectors[sel];
      a.tokens = w.xa; a.offsets = w.off_a; a.pkg_in = w.pkg_a; a.batch = batch;
      a.out_tokens = w.xb; a.out_offsets = w.off_b; a.pkg_out = w.pkg_b;
      a.fused = w.fused; a.kept_index = w.kept; a.state = st + (size_t)sel * batch * 5;
      a.pkg_rows = w.sel.pkg_rows;
      a.token_counts = token_counts; a.stage = sel + 1; a.img_warn = warnings;
      {
        ProfScope ps(HV_PROF_SELECTOR, s);
        rc = launch_selector(a, s);
      }
      if (rc) return rc;
      std::swap(w.xa, w.xb);
      std::swap(w.off_a, w.off_b);
      std::swap(w.pkg_a, w.pkg_b);
      ++sel;
      if (ckpt && (rc = launch_copy_ckpt(w.xa, w.off_a, batch, ckpt, ckpt_rows, sel, s))) return rc;
    }
    // The next block's LayerNorm 1 (after block 12 the final LayerNorm)
    // inside this block's FFN kernel, unless a selector changes the rows in
    // between.
    const bool chain_next =
        blk == 12 || !(sel < p->n_selectors && p->selector_blocks[sel] == blk + 1);
    bool next_done = false;
    const LnChain chain{ln1_ready, chain_next ? (blk < 12 ? &p->blocks[blk] : &fin) : nullptr,
                        w.blk.ln, &next_done};
    // One forward at a time, 32-row FFN blocks once a selector has cut the
    // rows (or for small batches), else 64-row blocks with the launch's last
    // ones split where that evens out the CUs' work; pipelined callers,
    // whose other batches fill the CUs a launch leaves idle, keep 64.
    const int ffn_rows = (options & HV_FWD_PIPELINED)               ? FFN_ROWS64
                         : (sel > 0 || small_rows((long long)max_rows)) ? FFN_ROWS32
                                                                        : FFN_ROWS64_BALANCED;
    if ((rc = block_forward(p->blocks[blk - 1], w.xa, w.off_a, batch, max_rows, w.xb, nullptr,
                            warnings, w.blk, s, chain, w.bias_max + 4 * (blk - 1), ffn_rows)))
      return rc;
    ln1_ready = next_done ? w.blk.ln : nullptr;
    if (blk == 12) final_done = next_done;
    std::swap(w.xa, w.xb);
    if (ckpt && (rc = launch_copy_ckpt(w.xa, w.off_a, batch, ckpt, ckpt_rows, 3 + blk, s))) return rc;
  }
  // Final LayerNorm over every row (model.py:102-106) unless block 12's FFN
  // kernel wrote it, head on CLS rows.
  if (!final_done) {
    ProfScope ps(HV_PROF_LAYERNORM, s);
    rc = launch_layernorm(w.xa, p->final_gamma, p->final_beta, w.blk.ln, max_rows,
                          w.off_a + batch, p->blocks[11].out_exp, p->final_gamma_exp,
                          p->final_beta_exp, p->final_ln_out_exp, nullptr,
                          LnWarn{w.off_a, batch, warnings}, s);
    if (rc) return rc;
  }
  if (ckpt && (rc = launch_copy_ckpt(w.blk.ln, w.off_a, batch, ckpt, ckpt_rows, 16, s))) return rc;
  GemmArgs g{};
  g.a = w.blk.ln; g.a_rows = w.off_a; g.b = p->head_w_p; g.bias = p->head_b; g.c = logits;
  g.m = batch; g.n = 1000; g.k = 192; g.lda = 192; g.ldc = 1000;
  g.shift_a = -14 - (p->final_ln_out_exp + p->head_w_exp);
  ProfScope ps(HV_PROF_HEAD, s);
  return launch_gemm(g, A_GATHER, HV_EPI_I32, s);
}

int hv_model_forward(const hv_model_dev *p, const int8_t *images, int batch, int32_t *logits,
                     int32_t *token_counts, int32_t *state, int32_t *warnings, int8_t *ckpt,
                     int32_t *ckpt_rows, void *workspace, size_t workspace_bytes,
                     hv_stream_t stream) {
  clear_error();
  return model_forward(p, images, false, batch, logits, token_counts, state, warnings, ckpt,
                       ckpt_rows, workspace, workspace_bytes, 0, (hipStream_t)stream);
}

int hv_model_forward_ex(const hv_model_dev *p, const int8_t *images, int batch, int32_t *logits,
                        int32_t *token_counts, int32_t *state, int32_t *warnings, int8_t *ckpt,
                        int32_t *ckpt_rows, void *workspace, size_t workspace_bytes, int options,
                        hv_stream_t stream) {
  clear_error();
  if (options & ~HV_FWD_PIPELINED)
    return fail(HV_EVALUE, HV_ERR_OPCODE, "model: unknown options 0x%x", options);
  return model_forward(p, images, false, batch, logits, token_counts, state, warnings, ckpt,
                       ckpt_rows, workspace, workspace_bytes, options, (hipStream_t)stream);
}

int hv_model_forward_f32(const hv_model_dev *p, const float *images, int batch, int32_t *logits,
                         int32_t *token_counts, int32_t *state, int32_t *warnings, int8_t *ckpt,
                         int32_t *ckpt_rows, void *workspace, size_t workspace_bytes,
                         hv_stream_t stream) {
  clear_error();
  return model_forward(p, images, true, batch, logits, token_counts, state, warnings, ckpt,
                       ckpt_rows, workspace, workspace_bytes, 0, (hipStream_t)stream);
}

int hv_model_forward_f32_ex(const hv_model_dev *p, const float *images, int batch,
                            int32_t *logits, int32_t *token_counts, int32_t *state,
                            int32_t *warnings, int8_t *ckpt, int32_t *ckpt_rows, void *workspace,
                            size_t workspace_bytes, int options, hv_stream_t stream) {
  clear_error();
  if (options & ~HV_FWD_PIPELINED)
    return fail(HV_EVALUE, HV_ERR_OPCODE, "model: unknown options 0x%x", options);
  return model_forward(p, images, true, batch, logits, token_counts, state, warnings, ckpt,
                       ckpt_rows, workspace, workspace_bytes, options, (hipStream_t)stream);
}

int hv_quantize_images(const float *images, int batch, int input_exp, int layout, int8_t *out,
                       hv_stream_t stream) {
  clear_error();
  if (!images || !out) return fail(HV_EVALUE, HV_ERR_ADDRESS, "images: null argument");
  if (layout != HV_IMAGE_NHWC && layout != HV_IMAGE_PATCHES)
    return fail(HV_EVALUE, HV_ERR_OPCODE, "images: unknown layout %d", layout);
  return launch_image_front(images, batch, input_exp, out, layout == HV_IMAGE_PATCHES,
                            (hipStream_t)stream);
}

int hv_profile_enable(int on) {
  prof_clear();
  g_prof_on = on != 0;
  return HV_OK;
}

int hv_profile_read(float *ms, int32_t *launches, int n) {
  clear_error();
  for (int i = 0; i < n; ++i) {
    if (ms) ms[i] = 0.f;
    if (launches) launches[i] = 0;
  }
  int rc = HV_OK;
  for (auto &e : g_prof) {
    float t = 0.f;
    if (rc == HV_OK) rc = check_hip(hipEventSynchronize(e.b), "profile sync");
    if (rc == HV_OK) rc = check_hip(hipEventElapsedTime(&t, e.a, e.b), "profile elapsed");
    if (rc == HV_OK && e.cls >= 0 && e.cls < n) {
      if (ms) ms[e.cls] += t;
      if (launches) launches[e.cls] += 1;
    }
  }
  prof_clear();
  return rc;
}

}  // extern "C"
