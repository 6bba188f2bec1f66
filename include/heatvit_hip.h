/*
 * heatvit_hip.h -- C ABI of libheatvit_hip.so, the gfx950 (MI355X) HIP
 * implementation of HeatViT-T's integer inference path.
 *
 * The reference (YOUXINYANG/HeatViT) has no FFI: its golden model is plain
 * Python that callers import (verification/heatvit_ref).  Each entry point
 * below replaces one golden-model function; the Python package heatvit_amd
 * binds them with ctypes and keeps the reference's Python signatures.
 *
 * Conventions
 *  - All tensor pointers are device pointers (hipMalloc'd or torch-owned);
 *    the library never allocates or frees caller memory.  Scratch space is
 *    passed in as `workspace` (size from the matching *_workspace_bytes).
 *  - All work is enqueued on the caller's stream; nothing synchronises the
 *    device.  Ragged row counts stay on the device (offset arrays).
 *  - Weights are passed in the packed layouts documented per struct; the
 *    host package produces them (heatvit_amd/device.py).
 *  - Return value: HV_OK or a negative status; hv_last_error() describes it.
 *    Status classes mirror the golden model's exceptions: HV_EVALUE is
 *    ValueError, HV_EOVERFLOW is OverflowError.
 *
 * Packed GEMM weight layout ("mfma32"): a logical int8 matrix W[K][N]
 * (row-major, the reference's layout) with K % 32 == 0 is padded to
 * N32 = ceil(N/32)*32 columns and stored as [N32/32][K/32][64][16] bytes:
 * element (k, n) lives at tile (n/32, k/32), lane r(n%32) + 32*((k%32)/16),
 * byte k%16, where r(c) = 8*((c%16)/4) + 4*(c/16) + c%4.  Each 1 KiB tile is
 * the first operand of one 32x32x32 int8 MFMA; the row order r puts output
 * channels 16*(l/32) .. +15 of a token row in result lane l.
 */
#ifndef HEATVIT_HIP_H
#define HEATVIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HV_OK 0
#define HV_EVALUE (-2)    /* invalid shape / range / exponent (ValueError) */
#define HV_EOVERFLOW (-3) /* accumulator outside int32 (OverflowError)    */
#define HV_EHIP (-4)      /* HIP runtime error                           */

/* Error codes of the reference engine (heatvit_pkg.sv:109-118; meanings
 * docs/heatvit.md:751-763), recorded by every failing call and, for
 * token counts found on the device, per image (hv_block_forward status;
 * hv_selector_forward state token_count -1). */
#define HV_ERR_NONE 0
#define HV_ERR_OPCODE 1           /* unknown primitive, epilogue or A mode      */
#define HV_ERR_DIMENSION 2        /* shape, batch, count or scale exponent      */
#define HV_ERR_ADDRESS 3          /* null or misaligned pointer, short workspace */
#define HV_ERR_TOKEN_COUNT 4      /* per-image token count outside its range     */
#define HV_ERR_MEMORY_PROTOCOL 5  /* HIP runtime failure on a launch or copy     */
#define HV_ERR_SOFTMAX_ZERO_SUM 6 /* never raised: a row maximum adds exp(0) = 2^16 */
#define HV_ERR_BUSY_START 7       /* never raised: calls queue on their stream   */

/* Warning bits of the reference engine (heatvit_pkg.sv:120-122). */
#define HV_WARN_HEAD_DEN_ZERO 1        /* fuse: zero head-weight sum, equal weights */
#define HV_WARN_PACKAGE_DEN_ZERO 2     /* finalize: zero package weight, plain mean */
#define HV_WARN_LN_NEGATIVE_VARIANCE 4 /* LayerNorm variance clamped to zero        */

#define HV_MAX_TOKENS 197 /* rows per image; attention tiles assume <= 208 */

/* hipStream_t without pulling in the HIP headers. */
typedef void *hv_stream_t;

/* Last error message of the calling thread ("" when none). */
const char *hv_last_error(void);
/* HV_ERR_* code of the calling thread's last failure (HV_ERR_NONE after a
 * successful call). */
int hv_last_error_class(void);
/* ABI version, bumped on any incompatible change. */
int hv_abi_version(void);

/* ------------------------------------------------------------------ */
/* Primitive evaluators (device implementations of fixed.py and         */
/* nonlinear.py, exposed so they can be checked element by element).    */
/* ------------------------------------------------------------------ */

#define HV_PRIM_REQUANT 0 /* out = requant(in, a, b, c)          fixed.py:37  */
#define HV_PRIM_GELU 1    /* out = gelu(in)                      nonlinear.py:60 */
#define HV_PRIM_PLAN 2    /* out = plan_sigmoid(in)              nonlinear.py:83 */
#define HV_PRIM_RSA 3     /* out = round_shift_away(in, a)       fixed.py:15  */
/* GEMM+GELU post-op on Q8.16 inputs (saturated to 24 bits first):
 * out = requant(gelu(in), -16, a - 16, 8), transformer.py:349-358.  _POST
 * computes it, _TABLE looks it up in the step tables the FFN GEMM uses for
 * a in [3, 12] (HV_EVALUE outside). */
#define HV_PRIM_GELU_POST 4
#define HV_PRIM_GELU_TABLE 5

/* Element-wise: out[i] = op(in[i]; a, b, c) over n int64 values. */
int hv_eval_primitive(int op, const int64_t *in, int64_t *out, int64_t n, int a, int b,
                      int c, hv_stream_t stream);

/* Softmax over ragged rows (nonlinear.py:109-133): row r is
 * x[offsets[r] .. offsets[r+1]); writes the attention UQ0.8 bytes and the
 * selector Q0.16 values (either output may be NULL).  Row length <= 256. */
int hv_softmax_rows(const int32_t *x, const int32_t *offsets, int rows, uint8_t *attention,
                    int32_t *selector, hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* LayerNorm (nonlinear.layernorm, nonlinear.py:136-186)                */
/* ------------------------------------------------------------------ */

/* y[r] = layernorm(x[r]) for r < rows (rows_dev, when non-NULL, holds the
 * live row count on the device and `rows` is the capacity).  neg_var, when
 * non-NULL, receives one byte per row (negative-variance flag). */
int hv_layernorm_i8(const int8_t *x, const int8_t *gamma, const int8_t *beta, int8_t *y,
                    int rows, const int32_t *rows_dev, int x_exp, int gamma_exp,
                    int beta_exp, int out_exp, uint8_t *neg_var, hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* Attention core of mhsa (transformer.py:228-266)                      */
/* ------------------------------------------------------------------ */

/* Image b owns rows offsets[b] .. offsets[b+1] of qkv [rows][576] (the
 * fused QKV projection: Q, K, V column blocks, heads of 64 lanes,
 * layout.qkv_unpack, layout.py:92-129).  Per head h:
 *   score = requant(Q_h K_h^T, 2*qkv_exp, score_exp, 32)
 *   prob  = softmax_attention(sat24(rsa(score, -(score_exp + 13))))   UQ0.8
 *   ctx   = requant(prob V_h, prob_exp + qkv_exp, context_exp, 8)
 * with the heads concatenated lane-wise (layout.head_concat,
 * layout.py:132-155) into ctx [rows][192].  score / prob, when non-NULL,
 * receive the [B][3][197][197] checkpoints (row and column stride 197).
 * status (optional, [B]) gets HV_ERR_TOKEN_COUNT for an image whose token
 * count is outside [1, 197] or whose rows fall outside `rows`; such images
 * are skipped.  qkv must be 16-byte aligned, ctx 4-byte aligned. */
int hv_attention_i8(const int8_t *qkv, const int32_t *offsets, int batch, int rows, int8_t *ctx,
                    int32_t *score, uint8_t *prob, int qkv_exp, int score_exp, int prob_exp,
                    int context_exp, int32_t *status, hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* int8 GEMM with fused epilogues (gemm.gemm_numpy + gemm_writeback,    */
/* gemm.py:93-139; transformer.py:349-358 GELU; transformer.py:96-101   */
/* residual align-add)                                                  */
/* ------------------------------------------------------------------ */

#define HV_EPI_I8 0       /* c = requant(acc + bias, src, dst, 8)                    */
#define HV_EPI_I32 1      /* c = requant(acc + bias, src, dst, 32) (int32 output)    */
#define HV_EPI_GELU 2     /* c = requant(gelu(requant(acc+bias, src, -16, 24)), -16, dst, 8) */
#define HV_EPI_RESIDUAL 3 /* t = requant(acc+bias, src, mid, 8); c = align_add(res@res_exp, t@mid -> dst) */

#define HV_A_ROWS 0   /* A row r at a + r*lda                                         */
#define HV_A_GATHER 1 /* A row r at a + a_rows[r]*lda                                 */
/* ORed onto HV_A_ROWS: A bytes are unsigned 0..255 (gemm_numpy a_unsigned,
 * gemm.py:93-114); K <= 65536 so the int32 accumulator cannot overflow. */
#define HV_A_UNSIGNED 4

typedef struct {
  const int8_t *a;         /* [M][lda] int8                                  */
  const int32_t *a_rows;   /* HV_A_GATHER row indices [M]                     */
  const int8_t *b_packed;  /* "mfma32" packed weights for W[K][N]             */
  const int32_t *bias;     /* [N] or NULL                                    */
  void *c;                 /* [M][ldc] int8, or int32 for HV_EPI_I32          */
  const int8_t *residual;  /* [M][ldr] for HV_EPI_RESIDUAL                    */
  int8_t *aux;             /* optional [M][ldc]: t of HV_EPI_RESIDUAL        */
  const int32_t *m_dev;    /* optional device-side live M (<= m)             */
  int32_t m, n, k, lda, ldc, ldr;
  int32_t a_mode, epilogue;
  int32_t src_exp, dst_exp, mid_exp, res_exp;
} hv_gemm_desc;

int hv_gemm_i8(const hv_gemm_desc *d, hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* Parameter views (device pointers) for the fused stages                */
/* ------------------------------------------------------------------ */

/* PatchParams (transformer.py:51-93); weight packed mfma32 from [768][192]. */
typedef struct {
  const int8_t *weight_p;
  const int32_t *bias;
  const int8_t *cls, *pos; /* [192], [197][192] */
  int32_t image_exp, weight_exp, activation_exp, tokens_exp, cls_exp, pos_exp;
} hv_patch_dev;

/* BlockParams = MhsaParams + FfnParams (transformer.py:148-198, 287-325);
 * wqkv_p/wproj_p/w1_p/w2_p packed mfma32 from the [K][N] matrices. */
typedef struct {
  const int8_t *ln1_gamma, *ln1_beta, *wqkv_p, *wproj_p;
  const int8_t *ln2_gamma, *ln2_beta, *w1_p, *w2_p;
  const int32_t *bqkv, *bproj, *b1, *b2;
  int32_t x_exp, gamma1_exp, beta1_exp, ln1_out_exp, wqkv_exp, qkv_out_exp, score_exp,
      prob_exp, context_out_exp, wproj_exp, msa_out_exp;
  int32_t ffn_x_exp, gamma2_exp, beta2_exp, ln2_out_exp, w1_exp, hidden_out_exp, w2_exp,
      ffn_out_exp, out_exp;
} hv_block_dev;

/* SelectorParams (selector.py:111-222).  Weight matrices are stored
 * output-major ("transposed"): local_wt [3][32][64], w1t [3][32][64],
 * w2t [3][16][32], w3t [3][2][16], hw_w1t [3][3], hw_w2t [3][3], i.e.
 * wt[h][j][k] = w[h][k][j]. */
typedef struct {
  const int8_t *local_wt, *w1t, *w2t, *w3t, *hw_w1t, *hw_w2t;
  const int32_t *local_b, *b1, *b2, *b3, *hw_b1, *hw_b2;
  int32_t in_exp, local_w_exp, local_out_exp, concat_out_exp, score_w1_exp, score_w2_exp,
      score_w3_exp, h1_out_exp, h2_out_exp, logits_out_exp, stats_out_exp, hw_w1_exp,
      hw_hidden_out_exp, hw_w2_exp;
} hv_selector_dev;

/* HeatViTParams (model.py:24-47); head_w packed mfma32 from [192][1000]. */
typedef struct {
  hv_patch_dev patch;
  hv_block_dev blocks[12];
  hv_selector_dev selectors[3];
  int32_t n_selectors;
  int32_t selector_blocks[3];
  const int8_t *final_gamma, *final_beta, *head_w_p;
  const int32_t *head_b;
  int32_t final_gamma_exp, final_beta_exp, final_ln_out_exp, head_w_exp;
} hv_model_dev;

/* ------------------------------------------------------------------ */
/* Descriptor front end.  The reference engine executes a ROM of 320-bit */
/* descriptors (rtl/generated/heatvit_descriptors.mem; fields            */
/* descriptor.py:131-161, sequence generate_descriptors.py:222-480) over */
/* a four-region memory image.  hv_schedule_compile validates the ROM    */
/* as the engine does (HV_ERR_OPCODE / _DIMENSION / _ADDRESS), checks     */
/* that it is the HeatViT-T sequence (patch, 12 blocks, up to three       */
/* selectors, final LayerNorm, classifier) with chained scale exponents,  */
/* and returns every tensor's weight-region offset and the exponents;    */
/* hv_schedule_bind repacks a device copy of the weight region into      */
/* `packed` and fills an hv_model_dev for hv_model_forward.  Images are  */
/* the input region (NHWC int8), logits the output region (int32).       */
/* ------------------------------------------------------------------ */

#define HV_DESC_WORD_BYTES 40 /* one descriptor, little-endian: bit i in byte i/8 */

typedef struct {
  uint32_t gamma1, beta1, wqkv, bqkv, wproj, bproj, gamma2, beta2, w1, b1, w2, b2;
} hv_schedule_block;
typedef struct {
  uint32_t local_w, local_b, score_w1, score_b1, score_w2, score_b2, score_w3, score_b3, hw_w1,
      hw_b1, hw_w2, hw_b2;
} hv_schedule_selector;
typedef struct {
  uint32_t patch_w, patch_b, cls, pos; /* weight-region byte offsets */
  hv_schedule_block blocks[12];
  hv_schedule_selector selectors[3];
  uint32_t final_gamma, final_beta, head_w, head_b;
  uint64_t weight_bytes; /* end of the last tensor the schedule reads */
  hv_model_dev model;    /* exponents, selector count and placement; NULL pointers */
} hv_schedule;

int hv_schedule_compile(const uint8_t *words, int n_desc, hv_schedule *out);
size_t hv_schedule_packed_bytes(const hv_schedule *s);
int hv_schedule_bind(const hv_schedule *s, const uint8_t *weights, size_t weight_bytes,
                     void *packed, size_t packed_bytes, hv_model_dev *model, hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* transformer.transformer_block (transformer.py:401-431) over a ragged  */
/* batch: image b owns rows offsets[b] .. offsets[b+1] of x.             */
/* ------------------------------------------------------------------ */

typedef struct {
  int8_t *ln1, *fused_qkv, *concat, *msa, *y, *ln2, *hidden, *ffn_out; /* [T][..] */
  int32_t *score; /* [B][3][197][197] (row/col stride 197) */
  uint8_t *prob;  /* [B][3][197][197] */
} hv_block_ckpt;

/* status (optional, [B]): HV_ERR_TOKEN_COUNT for an image whose row count
 * is outside [1, 197] or whose rows leave [0, max_rows) -- such an image
 * is skipped by the attention and its z rows are unspecified -- else 0.
 * warnings (optional, [B]): HV_WARN_LN_NEGATIVE_VARIANCE when a row of the
 * image had a negative variance in LN1 or LN2, else 0. */
size_t hv_block_workspace_bytes(int batch, int max_rows);
int hv_block_forward(const hv_block_dev *p, const int8_t *x, const int32_t *offsets, int batch,
                     int max_rows, int8_t *z, const hv_block_ckpt *ck, int32_t *status,
                     int32_t *warnings, void *workspace, size_t workspace_bytes,
                     hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* selector.token_selector (selector.py:503-563) over a ragged batch.    */
/* Image b: rows offsets[b]..offsets[b+1] of tokens, package flag        */
/* pkg_in[b].  Outputs: out_tokens (compacted), out_offsets [B+1],       */
/* pkg_out [B], fused [B][196] (Q0.16 per candidate), kept_index         */
/* [B][196] (candidate index of each kept normal, -1 padded),            */
/* state [B][5] = {token_count, package_present, kept, pruned, warnings}; */
/* token_count -1 marks an image the selector rejects (HV_ERR_TOKEN_COUNT: */
/* fewer than two tokens, more than 197, or a package with no normal).    */
/* ------------------------------------------------------------------ */

/* Optional selector checkpoints (SelectorResult fields, selector.py:235-250);
 * candidate axes are padded to 196. */
typedef struct {
  int8_t *local;         /* [B][3][196][32] */
  int8_t *global;        /* [B][3][32]      */
  int32_t *head_scores;  /* [B][3][196]     */
  int8_t *head_stats;    /* [B][196][3]     */
  int32_t *head_weights; /* [B][196][3]     */
  int8_t *h2;            /* [B][3][196][16]: score MLP layer 2 (selector.py:307-335), 16-byte aligned */
} hv_selector_ckpt;

size_t hv_selector_workspace_bytes(int batch);
int hv_selector_forward(const hv_selector_dev *p, const int8_t *tokens, const int32_t *offsets,
                        const uint8_t *pkg_in, int batch, int8_t *out_tokens,
                        int32_t *out_offsets, uint8_t *pkg_out, int32_t *fused,
                        int32_t *kept_index, int32_t *state, const hv_selector_ckpt *ck,
                        void *workspace, size_t workspace_bytes, hv_stream_t stream);

/* hv_selector_forward with no workspace argument and no allocation: the
 * package rows (192 bytes per image) and the offset scratch live in a fixed
 * 256 KiB device array of the library (per GPU, held until the process
 * ends), so callers that cannot
 * call hipMalloc (code under HIP graph capture, serving loops, harnesses
 * that forbid allocation) can run the selector.  No counterpart in the
 * reference.  batch <= HV_SELECTOR_NOALLOC_MAX_BATCH (HV_EVALUE /
 * HV_ERR_DIMENSION beyond).  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams or threads) race.
 * Nothing in the array needs clearing between calls. */
#define HV_SELECTOR_NOALLOC_MAX_BATCH 1024
int hv_selector_forward_noalloc(const hv_selector_dev *p, const int8_t *tokens,
                                const int32_t *offsets, const uint8_t *pkg_in, int batch,
                                int8_t *out_tokens, int32_t *out_offsets, uint8_t *pkg_out,
                                int32_t *fused, int32_t *kept_index, int32_t *state,
                                const hv_selector_ckpt *ck, hv_stream_t stream);

/* selector.finalize_tokens (selector.py:421-500) from given fused scores
 * fused [B][196] (Q0.16, candidate c of image b at b*196 + c; the last
 * candidate is the incoming package when pkg_in[b]); outputs as in
 * hv_selector_forward.  An image with a score outside [0, 65536] is
 * rejected (state token count -1), as selector._q016 raises ValueError. */
int hv_selector_finalize(const int8_t *tokens, const int32_t *offsets, const uint8_t *pkg_in,
                         const int32_t *fused, int batch, int8_t *out_tokens,
                         int32_t *out_offsets, uint8_t *pkg_out, int32_t *kept_index,
                         int32_t *state, hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* transformer.patch_embedding (transformer.py:104-145) over a batch of  */
/* NHWC 224x224x3 int8 images: x [B][197][192] int8 at tokens_exp.       */
/* ------------------------------------------------------------------ */

int hv_patch_embedding(const hv_patch_dev *p, const int8_t *images, int batch, int8_t *x,
                       hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* model.HeatViTModel.infer (model.py:73-123) over a batch of images.    */
/* images [B][224*224*3] NHWC int8; logits [B][1000] int32 at exp -14;   */
/* token_counts [B][4]: rows entering block 1, and after each selector;  */
/* state [3][B][5] per-selector state as in hv_selector_forward.         */
/* warnings (optional, [B]): the engine's warning bits of each image's   */
/* forward: HV_WARN_* of its three selectors and of its 25 LayerNorms.   */
/* ckpt (optional): [B][17][197][192] int8 in the slot order patch,      */
/* selector_01..03, block_01..12, final_ln, rows per slot in ckpt_rows   */
/* [B][17].                                                              */
/* ------------------------------------------------------------------ */

size_t hv_model_workspace_bytes(int batch);
int hv_model_forward(const hv_model_dev *p, const int8_t *images, int batch, int32_t *logits,
                     int32_t *token_counts, int32_t *state, int32_t *warnings, int8_t *ckpt,
                     int32_t *ckpt_rows, void *workspace, size_t workspace_bytes,
                     hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* Image front end: preprocessed float images, CHW [B][3][224][224]     */
/* (16-byte aligned), quantised to int8 q = clamp(round_half_even(x /   */
/* 2^input_exp), -128, 127) as in p2_export_weights.real_image_list     */
/* (tools/p2/p2_export_weights.py:246-251) and p2_sim.forward_image     */
/* (tools/p2/p2_sim.py:536-543); NaN gives 0.                           */
/* ------------------------------------------------------------------ */

#define HV_IMAGE_NHWC 0    /* out [B][224*224*3]: the golden model's image      */
#define HV_IMAGE_PATCHES 1 /* out [B*196][768]: layout.patchify rows (layout.py:31-72) */

int hv_quantize_images(const float *images, int batch, int input_exp, int layout, int8_t *out,
                       hv_stream_t stream);

/* hv_model_forward from float CHW images, quantised at the patch's
 * image_exp straight into the patch matrix (no NHWC copy); same outputs
 * and workspace. */
int hv_model_forward_f32(const hv_model_dev *p, const float *images, int batch, int32_t *logits,
                         int32_t *token_counts, int32_t *state, int32_t *warnings, int8_t *ckpt,
                         int32_t *ckpt_rows, void *workspace, size_t workspace_bytes,
                         hv_stream_t stream);

/* hv_model_forward and hv_model_forward_f32 with options (no counterpart   */
/* in the reference: launch shapes only, the outputs are the same bytes).   */
/* Without options a forward is taken to run alone on the GPU: the fused    */
/* FFN then uses blocks of 32 rows wherever blocks of 64 would leave CUs    */
/* idle (after the first selector, or for batches under 166 images).        */
/* HV_FWD_PIPELINED: the caller keeps other forwards in flight on the same  */
/* GPU (heatvit_amd.model.Pipeline), which fills the CUs the small stages   */
/* leave idle; the fused FFN keeps its 64-row blocks throughout.           */
#define HV_FWD_PIPELINED 1
int hv_model_forward_ex(const hv_model_dev *p, const int8_t *images, int batch, int32_t *logits,
                        int32_t *token_counts, int32_t *state, int32_t *warnings, int8_t *ckpt,
                        int32_t *ckpt_rows, void *workspace, size_t workspace_bytes, int options,
                        hv_stream_t stream);
int hv_model_forward_f32_ex(const hv_model_dev *p, const float *images, int batch,
                            int32_t *logits, int32_t *token_counts, int32_t *state,
                            int32_t *warnings, int8_t *ckpt, int32_t *ckpt_rows, void *workspace,
                            size_t workspace_bytes, int options, hv_stream_t stream);

/* ------------------------------------------------------------------ */
/* Kernel-class timing with HIP events (for benchmarks).  While enabled, */
/* every kernel the forwards launch carries a start/stop event pair      */
/* recorded by its own dispatch; hv_profile_read() waits for them and    */
/* returns the summed milliseconds and launch counts per class (arrays   */
/* of n entries), then clears the record.  Not thread-safe: one          */
/* profiling client at a time.                                           */
/* ------------------------------------------------------------------ */

#define HV_PROF_PATCH 0
#define HV_PROF_LAYERNORM 1
#define HV_PROF_GEMM_QKV 2
#define HV_PROF_ATTENTION 3
#define HV_PROF_GEMM_PROJ 4
#define HV_PROF_GEMM_FFN1 5
#define HV_PROF_GEMM_FFN2 6
#define HV_PROF_SELECTOR 7
#define HV_PROF_HEAD 8
#define HV_PROF_OTHER 9
#define HV_PROF_FFN 10 /* FFN1 + GELU + FFN2 + residual in one kernel */
#define HV_PROF_CLASSES 11

int hv_profile_enable(int on);
int hv_profile_read(float *ms, int32_t *launches, int n);

#ifdef __cplusplus
}
#endif
#endif
