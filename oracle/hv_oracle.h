/*
 * hv_oracle.h -- CPU restatement of the HeatViT-T integer golden model.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  Nothing in heatvit_amd/ links, imports or calls it.
 *
 * Every function restates one function of the reference's golden model
 * (verification/heatvit_ref, one .py per stage); the citation is on the
 * definition in
 * hv_oracle.c.  Python's unbounded integers are reproduced with int64 where
 * the reachable range provably fits and with __int128 elsewhere.
 *
 * Status codes: 0 ok, HVO_EVALUE (ValueError), HVO_EOVERFLOW (OverflowError).
 */
#ifndef HV_ORACLE_H
#define HV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HVO_OK 0
#define HVO_EVALUE (-2)
#define HVO_EOVERFLOW (-3)

/* Warning bits of the reference engine (heatvit_pkg.sv:120-122). */
#define HVO_WARN_HEAD_DEN_ZERO 1
#define HVO_WARN_PACKAGE_DEN_ZERO 2
#define HVO_WARN_LN_NEGATIVE_VARIANCE 4

#define HVO_D 192
#define HVO_HEADS 3
#define HVO_HEAD_DIM 64
#define HVO_FFN 768
#define HVO_CLASSES 1000
#define HVO_TOKENS 197

/* ---- primitives (fixed.py, nonlinear.py) ---- */
int64_t hvo_round_shift_away(int64_t value, int shift);
int64_t hvo_sat_signed(int64_t value, int bits);
int64_t hvo_requant(int64_t value, int src_exp, int dst_exp, int bits);
void hvo_requant_array(const int64_t *v, int64_t *out, int64_t n, int src_exp, int dst_exp,
                       int bits);
int hvo_round_div(int64_t num, int64_t den, int64_t *out);
int hvo_udiv(uint64_t num, uint64_t den, uint64_t *quot, uint64_t *rem);
uint64_t hvo_isqrt(uint64_t radicand, uint64_t *rem);
int32_t hvo_gelu(int32_t x);
int32_t hvo_plan_sigmoid(int32_t x);
void hvo_gelu_array(const int32_t *x, int32_t *out, int64_t n);
/* nonlinear._softmax_exp (nonlinear.py:98-106) of one x_tilde <= 0. */
int64_t hvo_softmax_exp(int64_t xt);
int hvo_softmax_scaled(const int32_t *x, int n, int32_t delta2, int32_t *out);
int hvo_softmax_attention(const int32_t *x, int n, uint8_t *out);
int hvo_softmax_selector(const int32_t *x, int n, int32_t *out);
int hvo_layernorm(const int8_t *x, const int8_t *gamma, const int8_t *beta,
                  int x_exp, int gamma_exp, int beta_exp, int out_exp,
                  int8_t *out, int *negative_variance);

/* ---- GEMM (gemm.py) ----
 * acc[M][N] = A[M][K] * B (B is [K][N], or [N][K] when transpose_b) + bias.
 * a_unsigned reads A as bytes 0..255.  Returns HVO_EOVERFLOW if a pre-bias
 * accumulator leaves int32, as gemm_numpy does. */
int hvo_gemm(const void *a, const int8_t *b, const int32_t *bias, int m, int n,
             int k, int transpose_b, int a_unsigned, int64_t *acc);
int hvo_gemm_writeback(const int64_t *acc, int count, int src_exp, int dst_exp,
                       int bits, void *out);

/* ---- parameter views (transformer.py, selector.py, model.py) ---- */
typedef struct {
  const int8_t *weight;  /* [patch*patch*3][192] */
  const int32_t *bias;   /* [192] */
  const int8_t *cls;     /* [192] */
  const int8_t *pos;     /* [197][192] */
  int32_t width, height, patch;
  int32_t image_exp, weight_exp, activation_exp, tokens_exp, cls_exp, pos_exp;
} hvo_patch;

typedef struct {
  const int8_t *ln1_gamma, *ln1_beta; /* [192] */
  const int8_t *wqkv;                 /* [192][576] */
  const int32_t *bqkv;                /* [576] */
  const int8_t *wproj;                /* [192][192] */
  const int32_t *bproj;               /* [192] */
  const int8_t *ln2_gamma, *ln2_beta; /* [192] */
  const int8_t *w1;                   /* [192][768] */
  const int32_t *b1;                  /* [768] */
  const int8_t *w2;                   /* [768][192] */
  const int32_t *b2;                  /* [192] */
  /* MhsaParams exponents */
  int32_t x_exp, gamma1_exp, beta1_exp, ln1_out_exp, wqkv_exp, qkv_out_exp,
      score_exp, prob_exp, context_out_exp, wproj_exp, msa_out_exp;
  /* FfnParams exponents */
  int32_t ffn_x_exp, gamma2_exp, beta2_exp, ln2_out_exp, w1_exp,
      hidden_out_exp, w2_exp, ffn_out_exp, out_exp;
} hvo_block;

typedef struct {
  const int8_t *local_w;  /* [3][64][32] */
  const int32_t *local_b; /* [3][32] */
  const int8_t *w1;       /* [3][64][32] */
  const int32_t *b1;      /* [3][32] */
  const int8_t *w2;       /* [3][32][16] */
  const int32_t *b2;      /* [3][16] */
  const int8_t *w3;       /* [3][16][2] */
  const int32_t *b3;      /* [3][2] */
  const int8_t *hw_w1;    /* [3][3] */
  const int32_t *hw_b1;   /* [3] */
  const int8_t *hw_w2;    /* [3][3] */
  const int32_t *hw_b2;   /* [3] */
  int32_t in_exp, local_w_exp, local_out_exp, concat_out_exp, score_w1_exp,
      score_w2_exp, score_w3_exp, h1_out_exp, h2_out_exp, logits_out_exp,
      stats_out_exp, hw_w1_exp, hw_hidden_out_exp, hw_w2_exp;
} hvo_selector;

typedef struct {
  hvo_patch patch;
  hvo_block blocks[12];
  hvo_selector selectors[3];
  int32_t n_selectors;
  int32_t selector_blocks[3];
  const int8_t *final_gamma, *final_beta; /* [192] */
  const int8_t *head_w;                   /* [192][1000] */
  const int32_t *head_b;                  /* [1000] */
  int32_t final_gamma_exp, final_beta_exp, final_ln_out_exp, head_w_exp;
} hvo_model;

/* Optional per-block checkpoints (any pointer may be NULL). */
typedef struct {
  int8_t *ln1;       /* [N][192] */
  int8_t *fused_qkv; /* [N][576] */
  int32_t *score;    /* [3][N][N] */
  uint8_t *prob;     /* [3][N][N] */
  int8_t *context;   /* [3][N][64] */
  int8_t *concat;    /* [N][192] */
  int8_t *msa;       /* [N][192] */
  int8_t *y;         /* [N][192] */
  int8_t *ln2;       /* [N][192] */
  int8_t *hidden;    /* [N][768] */
  int8_t *ffn_out;   /* [N][192] */
  int32_t *warnings; /* [1]: HVO_WARN_LN_NEGATIVE_VARIANCE ORed in by LN1/LN2 */
} hvo_block_ckpt;

/* Optional selector checkpoints (any pointer may be NULL); C = N - 1. */
typedef struct {
  int8_t *local;         /* [3][C][32] */
  int8_t *global;        /* [3][32] */
  int32_t *head_scores;  /* [3][C] */
  int8_t *head_stats;    /* [C][3] */
  int32_t *head_weights; /* [C][3] */
  int32_t *fused;        /* [C] */
  int8_t *h2;            /* [3][C][16]: score MLP layer 2 (score_mlp_layers h2) */
} hvo_selector_ckpt;

typedef struct {
  int32_t token_count, package_present, kept_normal_count, pruned_normal_count,
      warnings;
} hvo_selector_state;

int hvo_patchify(const int8_t *image, int width, int height, int patch, int8_t *patches);
int hvo_quantize_image(const float *chw, int width, int height, int input_exp, int8_t *nhwc);
int hvo_patch_embedding(const int8_t *image, const hvo_patch *p, int8_t *out);
int hvo_transformer_block(const int8_t *x, int n, const hvo_block *p,
                          int8_t *z, hvo_block_ckpt *ck);
void hvo_fuse_head_scores(const int32_t *scores, const int32_t *weights, int C,
                          int32_t *fused, int *warn);
int hvo_finalize_tokens(const int8_t *cls, const int8_t *normal, int n_normal,
                        const int8_t *incoming_package, const int32_t *scores,
                        int n_scores, int width, int8_t *out_tokens,
                        int32_t *kept_index, hvo_selector_state *st);
int hvo_token_selector(const int8_t *tokens, int n, int package_present,
                       const hvo_selector *p, int8_t *out_tokens,
                       int32_t *kept_index, hvo_selector_state *st,
                       hvo_selector_ckpt *ck);

/* Model checkpoint slots: 0 patch, 1..3 selector_01..03, 4..15 block_01..12,
 * 16 final_ln; each slot holds up to 197 rows of 192 bytes. */
#define HVO_CKPT_SLOTS 17
/* *warnings (optional): the engine's warning bits of the whole forward
 * (heatvit_top.sv:5-6 OR-latch): the selectors' bits 0/1 and bit 2 when any
 * LayerNorm row had a negative variance. */
int hvo_model_infer(const int8_t *image, const hvo_model *m, int32_t *logits,
                    int8_t *ckpt /* [17][197][192] or NULL */,
                    int32_t *ckpt_rows /* [17] or NULL */,
                    hvo_selector_state *summary /* [3] or NULL */,
                    int32_t *warnings /* [1] or NULL */);
/* Runs hvo_model_infer over `count` images (image stride 150528 B for the
 * default 224x224x3) with `threads` OpenMP threads; logits [count][1000],
 * token_counts [count][4] (input rows of the final LN per stage). */
int hvo_model_infer_batch(const int8_t *images, int count, const hvo_model *m,
                          int threads, int32_t *logits, int32_t *token_counts,
                          int32_t *status, int32_t *warnings /* [count] or NULL */);

#ifdef __cplusplus
}
#endif
#endif
