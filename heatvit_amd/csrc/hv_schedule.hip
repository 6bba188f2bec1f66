// hv_schedule.hip -- descriptor front end.
//
// The reference engine runs a compiled ROM of 320-bit descriptors
// (rtl/generated/heatvit_descriptors.mem; fields descriptor.py:131-161,
// sequence generate_descriptors.py:222-480, docs/heatvit.md:271-291) over a
// four-region memory image (input, weight, scratch, output).  On the GPU the
// forward is a handful of fused kernels, not one engine pass per
// descriptor, so the ROM is compiled instead of interpreted:
// hv_schedule_compile validates every descriptor as the engine would,
// recognises the HeatViT-T operator sequence (patch stage, 12 blocks, up to
// three selectors, final LayerNorm, classifier), checks that the scale
// exponents chain the way the fused kernels assume, and returns the weight-
// region offset of every tensor with the exponents in hv_model_dev form.
// hv_schedule_bind then repacks the weight region on the device into the
// kernels' layouts.
#include <string.h>

#include "hv_internal.h"

namespace hv {
namespace {

enum Op {
  OP_NOP = 0, OP_PATCHIFY, OP_COPY_ADD_POS, OP_GEMM, OP_LAYERNORM, OP_RESIDUAL, OP_QKV_UNPACK,
  OP_HEAD_CONCAT, OP_ATTN_SOFTMAX, OP_SELECTOR_SOFTMAX, OP_REDUCE_MEAN, OP_CONCAT_LOCAL_GLOBAL,
  OP_HEAD_FUSE, OP_SELECTOR_FINALIZE, OP_FINISH
};
enum Flag {
  F_RHS_TRANSPOSE = 0, F_BIAS = 1, F_AUX = 2, F_DYN_M = 3, F_SWAP = 4, F_HEAD_MODE = 5,
  F_OUT_I32 = 7, F_SRC0_INPUT = 11, F_SRC1_SCRATCH = 12, F_BIAS_SCRATCH = 13, F_AUX_WEIGHT = 14,
  F_DST_OUTPUT = 15, F_SRC0_UNSIGNED = 18
};
enum Post { POST_NONE = 0, POST_GELU = 2, POST_PLAN = 5 };
constexpr int kUq08 = -8, kQ016 = -16, kLogit = -14;

struct Desc {
  int op, flags, m, n, k, heads, s0, s1, saux, sdst, next, param0, param1, reserved;
  uint32_t src0, src1, bias, aux, dst;
  bool has(int f) const { return (flags >> f) & 1; }
  int post() const { return (flags >> 8) & 7; }
};

// Bits [lsb, lsb + width) of a little-endian 320-bit word.
uint32_t bits(const uint8_t *w, int lsb, int width) {
  uint32_t v = 0;
  for (int i = 0; i < width; ++i) v |= (uint32_t)((w[(lsb + i) >> 3] >> ((lsb + i) & 7)) & 1) << i;
  return v;
}
int signed6(uint32_t b) { return b >= 32 ? (int)b - 64 : (int)b; }

Desc decode(const uint8_t *w) {
  Desc d;
  d.reserved = bits(w, 0, 4);
  d.param1 = bits(w, 4, 16);
  d.param0 = bits(w, 20, 16);
  d.next = bits(w, 36, 16);
  d.sdst = signed6(bits(w, 52, 6));
  d.saux = signed6(bits(w, 58, 6));
  d.s1 = signed6(bits(w, 64, 6));
  d.s0 = signed6(bits(w, 70, 6));
  d.dst = bits(w, 76, 32);
  d.aux = bits(w, 108, 32);
  d.bias = bits(w, 140, 32);
  d.src1 = bits(w, 172, 32);
  d.src0 = bits(w, 204, 32);
  d.heads = bits(w, 236, 4);
  d.k = bits(w, 240, 16);
  d.n = bits(w, 256, 16);
  d.m = bits(w, 272, 16);
  d.flags = bits(w, 288, 24);
  d.op = bits(w, 312, 8);
  return d;
}

// Descriptor.validate (descriptor.py:167-219) and the engine's descriptor
// rules (docs/heatvit.md:271-291): error codes 1 (opcode), 2 (reserved
// bits, flags, post-op, heads, dimensions), 3 (alignment).
int validate(const Desc &d, int i) {
  if (d.op > OP_FINISH)
    return fail(HV_EVALUE, HV_ERR_OPCODE, "descriptor %d: unknown opcode %d", i, d.op);
  if (d.reserved || (d.flags >> 22))
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: reserved bits set", i);
  if (d.post() > 6)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: post-op %d", i, d.post());
  if (d.heads != 0 && d.heads != 3)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: %d heads", i, d.heads);
  if (d.has(F_SRC0_UNSIGNED) &&
      !(d.op == OP_GEMM && d.has(F_HEAD_MODE) && d.heads == 3 && d.post() == POST_NONE))
    return fail(HV_EVALUE, HV_ERR_DIMENSION,
                "descriptor %d: unsigned src0 only on the Attention*V GEMM", i);
  if (d.has(F_DYN_M)) {
    const bool dyn = d.op == OP_GEMM || (d.op >= OP_LAYERNORM && d.op <= OP_SELECTOR_FINALIZE);
    if (!dyn) return fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: dynamic M on op %d", i, d.op);
    if ((d.param0 & 3) >= 2)
      return fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: dynamic-M select %d", i,
                  d.param0 & 3);
  }
  if (d.op == OP_GEMM && (d.m == 0 || d.n == 0 || d.k == 0))
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: zero GEMM dimension", i);
  if (d.op == OP_LAYERNORM && d.n != 192)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: LayerNorm over %d channels", i, d.n);
  if ((d.src0 | d.src1 | d.bias | d.aux | d.dst) & 7)
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "descriptor %d: offset not 8-byte aligned", i);
  return HV_OK;
}

// Sequence matcher over the validated descriptors.
struct Reader {
  const Desc *d;
  int count, pos = 0, rc = HV_OK;
  uint64_t weight_end = 0;  // bytes of weight region the tensors reach

  bool ok() const { return rc == HV_OK; }
  const Desc *peek() const { return pos < count ? &d[pos] : nullptr; }
  // The next descriptor, which must have opcode `op` and the given shape
  // (negative: any).
  const Desc *take(int op, int n = -1, int k = -1, int heads = -1, int post = -1) {
    if (!ok()) return nullptr;
    if (pos >= count) {
      rc = fail(HV_EVALUE, HV_ERR_OPCODE, "schedule ends at descriptor %d", pos);
      return nullptr;
    }
    const Desc *x = &d[pos];
    if (x->op != op) {
      rc = fail(HV_EVALUE, HV_ERR_OPCODE, "descriptor %d: opcode %d where the HeatViT-T "
                "schedule has %d", pos, x->op, op);
      return nullptr;
    }
    if ((n >= 0 && x->n != n) || (k >= 0 && x->k != k) || (heads >= 0 && x->heads != heads) ||
        (post >= 0 && x->post() != post)) {
      rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d (opcode %d): shape n=%d k=%d "
                "heads=%d post=%d is not the HeatViT-T one", pos, op, x->n, x->k, x->heads,
                x->post());
      return nullptr;
    }
    ++pos;
    return x;
  }
  // Scale chain: the fused kernels take one exponent where the schedule
  // names it twice.
  void same(int a, int b, const char *what) {
    if (ok() && a != b)
      rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: %s exponents differ (%d vs %d)",
                pos - 1, what, a, b);
  }
  // A tensor of `bytes` read from the weight region.
  uint32_t weight(uint32_t off, uint32_t bytes, bool from_weight_region) {
    if (ok() && !from_weight_region)
      rc = fail(HV_EVALUE, HV_ERR_ADDRESS, "descriptor %d: parameter outside the weight region",
                pos - 1);
    if (off + (uint64_t)bytes > weight_end) weight_end = off + bytes;
    return off;
  }
  // GEMM weights: src1 and bias from the weight region, bias enabled, the
  // weights read as [K][N] against a signed activation with the operands in
  // place (RHS_TRANSPOSE, SWAP_ACTIVATION and SRC0_UNSIGNED clear), and an
  // int8 output unless out_i32 (the classifier).
  void gemm_weights(const Desc *g, uint32_t wbytes, uint32_t bbytes, uint32_t *w, uint32_t *b,
                    bool out_i32 = false) {
    if (ok() && !g->has(F_BIAS))
      rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: GEMM without bias", pos - 1);
    if (ok() && (g->has(F_RHS_TRANSPOSE) || g->has(F_SWAP) || g->has(F_SRC0_UNSIGNED) ||
                 g->has(F_OUT_I32) != out_i32))
      rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: weight GEMM flags 0x%x", pos - 1,
                g->flags);
    *w = weight(g->src1, wbytes, !g->has(F_SRC1_SCRATCH));
    *b = weight(g->bias, bbytes, !g->has(F_BIAS_SCRATCH));
  }
};

void parse_block(Reader &r, int x_exp, hv_block_dev &e, hv_schedule_block &o) {
  const Desc *ln1 = r.take(OP_LAYERNORM);
  const Desc *qkv = r.take(OP_GEMM, 576, 192, 0, POST_NONE);
  const Desc *unpack = r.take(OP_QKV_UNPACK, 576, -1, 3);
  const Desc *qk = r.take(OP_GEMM, -1, 64, 3, POST_NONE);
  const Desc *sm = r.take(OP_ATTN_SOFTMAX, -1, -1, 3);
  const Desc *av = r.take(OP_GEMM, 64, -1, 3, POST_NONE);
  const Desc *cat = r.take(OP_HEAD_CONCAT, 192, -1, 3);
  const Desc *proj = r.take(OP_GEMM, 192, 192, 0, POST_NONE);
  const Desc *res1 = r.take(OP_RESIDUAL, 192);
  const Desc *ln2 = r.take(OP_LAYERNORM);
  const Desc *ffn1 = r.take(OP_GEMM, 768, 192, 0, POST_GELU);
  const Desc *ffn2 = r.take(OP_GEMM, 192, 768, 0, POST_NONE);
  const Desc *res2 = r.take(OP_RESIDUAL, 192);
  if (!r.ok()) return;
  if (!qk->has(F_RHS_TRANSPOSE) || !qk->has(F_OUT_I32) || !av->has(F_SRC0_UNSIGNED))
    r.rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "block at descriptor %d: attention GEMM flags",
                r.pos - 13);
  e.x_exp = ln1->s0;
  r.same(x_exp, ln1->s0, "block input");
  e.gamma1_exp = ln1->s1;
  e.beta1_exp = ln1->saux;
  e.ln1_out_exp = ln1->sdst;
  o.gamma1 = r.weight(ln1->src1, 192, !ln1->has(F_SRC1_SCRATCH));
  o.beta1 = r.weight(ln1->aux, 192, ln1->has(F_AUX_WEIGHT));
  r.same(qkv->s0, e.ln1_out_exp, "LN1 -> QKV");
  e.wqkv_exp = qkv->s1;
  e.qkv_out_exp = qkv->sdst;
  r.gemm_weights(qkv, 192 * 576, 576 * 4, &o.wqkv, &o.bqkv);
  r.same(unpack->s0, e.qkv_out_exp, "QKV unpack");
  r.same(unpack->sdst, e.qkv_out_exp, "QKV unpack");
  r.same(qk->s0, e.qkv_out_exp, "Q");
  r.same(qk->s1, e.qkv_out_exp, "K");
  e.score_exp = qk->sdst;
  r.same(sm->s0, e.score_exp - 3, "score / sqrt(64)");
  r.same(sm->sdst, kUq08, "attention probability");
  e.prob_exp = sm->sdst;
  r.same(av->s0, e.prob_exp, "probability -> A*V");
  r.same(av->s1, e.qkv_out_exp, "V");
  e.context_out_exp = av->sdst;
  r.same(cat->s0, e.context_out_exp, "head concat");
  r.same(cat->sdst, e.context_out_exp, "head concat");
  r.same(proj->s0, e.context_out_exp, "context -> projection");
  e.wproj_exp = proj->s1;
  e.msa_out_exp = proj->sdst;
  r.gemm_weights(proj, 192 * 192, 192 * 4, &o.wproj, &o.bproj);
  r.same(res1->s0, e.x_exp, "residual 1 input");
  r.same(res1->saux, e.msa_out_exp, "residual 1 MSA");
  e.ffn_x_exp = res1->sdst;
  r.same(ln2->s0, e.ffn_x_exp, "residual 1 -> LN2");
  e.gamma2_exp = ln2->s1;
  e.beta2_exp = ln2->saux;
  e.ln2_out_exp = ln2->sdst;
  o.gamma2 = r.weight(ln2->src1, 192, !ln2->has(F_SRC1_SCRATCH));
  o.beta2 = r.weight(ln2->aux, 192, ln2->has(F_AUX_WEIGHT));
  r.same(ffn1->s0, e.ln2_out_exp, "LN2 -> FFN1");
  e.w1_exp = ffn1->s1;
  e.hidden_out_exp = ffn1->sdst;
  r.gemm_weights(ffn1, 192 * 768, 768 * 4, &o.w1, &o.b1);
  r.same(ffn2->s0, e.hidden_out_exp, "FFN1 -> FFN2");
  e.w2_exp = ffn2->s1;
  e.ffn_out_exp = ffn2->sdst;
  r.gemm_weights(ffn2, 768 * 192, 192 * 4, &o.w2, &o.b2);
  r.same(res2->s0, e.ffn_x_exp, "residual 2 input");
  r.same(res2->saux, e.ffn_out_exp, "residual 2 FFN");
  e.out_exp = res2->sdst;
}

void parse_selector(Reader &r, int in_exp, hv_selector_dev &e, hv_schedule_selector &o) {
  const Desc *local = r.take(OP_GEMM, 32, 64, 3, POST_GELU);
  const Desc *mean = r.take(OP_REDUCE_MEAN, 32, -1, 3);
  const Desc *cat = r.take(OP_CONCAT_LOCAL_GLOBAL, 64, -1, 3);
  const Desc *h1 = r.take(OP_GEMM, 32, 64, 3, POST_GELU);
  const Desc *h2 = r.take(OP_GEMM, 16, 32, 3, POST_GELU);
  const Desc *lg = r.take(OP_GEMM, 2, 16, 3, POST_NONE);
  const Desc *sm = r.take(OP_SELECTOR_SOFTMAX, 2, -1, 3);
  const Desc *stats = r.take(OP_REDUCE_MEAN, 64, -1, 3);
  const Desc *hw1 = r.take(OP_GEMM, 3, 3, 0, POST_GELU);
  const Desc *hw2 = r.take(OP_GEMM, 3, 3, 0, POST_PLAN);
  const Desc *fuse = r.take(OP_HEAD_FUSE, 3, -1, 3);
  const Desc *fin = r.take(OP_SELECTOR_FINALIZE, 192);
  if (!r.ok()) return;
  e.in_exp = local->s0;
  r.same(local->s0, in_exp, "selector input");
  e.local_w_exp = local->s1;
  e.local_out_exp = local->sdst;
  r.gemm_weights(local, 3 * 64 * 32, 3 * 32 * 4, &o.local_w, &o.local_b);
  if (r.ok() && (mean->param0 >> 2 & 3) != 0)
    r.rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: candidate mean axis", r.pos - 11);
  r.same(mean->s0, e.local_out_exp, "candidate mean");
  r.same(mean->sdst, e.local_out_exp, "candidate mean");
  r.same(cat->s0, e.local_out_exp, "local/global concat");
  e.concat_out_exp = cat->sdst;
  r.same(h1->s0, e.concat_out_exp, "concat -> score MLP");
  e.score_w1_exp = h1->s1;
  e.h1_out_exp = h1->sdst;
  r.gemm_weights(h1, 3 * 64 * 32, 3 * 32 * 4, &o.score_w1, &o.score_b1);
  r.same(h2->s0, e.h1_out_exp, "score MLP layer 2");
  e.score_w2_exp = h2->s1;
  e.h2_out_exp = h2->sdst;
  r.gemm_weights(h2, 3 * 32 * 16, 3 * 16 * 4, &o.score_w2, &o.score_b2);
  r.same(lg->s0, e.h2_out_exp, "score MLP layer 3");
  e.score_w3_exp = lg->s1;
  e.logits_out_exp = lg->sdst;
  r.gemm_weights(lg, 3 * 16 * 2, 3 * 2 * 4, &o.score_w3, &o.score_b3);
  r.same(sm->s0, e.logits_out_exp, "keep softmax");
  r.same(sm->sdst, kQ016, "keep score");
  if (r.ok() && (stats->param0 >> 2 & 3) != 1)
    r.rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: head statistics axis", r.pos - 5);
  r.same(stats->s0, e.in_exp, "head statistics input");
  e.stats_out_exp = stats->sdst;
  r.same(hw1->s0, e.stats_out_exp, "head-weight MLP");
  e.hw_w1_exp = hw1->s1;
  e.hw_hidden_out_exp = hw1->sdst;
  r.gemm_weights(hw1, 9, 12, &o.hw_w1, &o.hw_b1);
  r.same(hw2->s0, e.hw_hidden_out_exp, "head-weight MLP layer 2");
  e.hw_w2_exp = hw2->s1;
  r.same(hw2->sdst, kQ016, "head weight");
  r.gemm_weights(hw2, 9, 12, &o.hw_w2, &o.hw_b2);
  r.same(fuse->s0, kQ016, "head fuse");
  r.same(fuse->s1, kQ016, "head fuse");
  r.same(fuse->sdst, kQ016, "head fuse");
  r.same(fin->s0, e.in_exp, "finalize tokens");
  r.same(fin->sdst, e.in_exp, "finalize tokens");
  r.same(fin->s1, kQ016, "finalize scores");
}

// 256-byte aligned slices of the packed buffer.
struct Slots {
  size_t used = 0;
  size_t take(size_t bytes) {
    const size_t off = (used + 255) & ~(size_t)255;
    used = off + bytes;
    return off;
  }
};

size_t packed_mfma(int k, int n) { return (size_t)k * ((n + 31) / 32 * 32); }

// W[K][N] row-major int8 -> mfma32 (include/heatvit_hip.h): one thread per
// 16-byte lane fragment, zero columns beyond N.
__global__ void k_pack_mfma32(const int8_t *__restrict__ w, int K, int N, int8_t *__restrict__ out) {
  const int KT = K / 32, NT = (N + 31) / 32;
  const int frags = NT * KT * 64;
  for (int f = blockIdx.x * blockDim.x + threadIdx.x; f < frags; f += gridDim.x * blockDim.x) {
    const int tile = f >> 6, lane = f & 63;
    const int nt = tile / KT, kt = tile - nt * KT;
    const int r = lane & 31, h = lane >> 5;
    const int n = nt * 32 + 16 * ((r & 7) >> 2) + 4 * (r >> 3) + (r & 3);
    const int k0 = kt * 32 + 16 * h;
    int word[4] = {0, 0, 0, 0};
    if (n < N)
      for (int j = 0; j < 16; ++j)
        word[j >> 2] |= (w[(size_t)(k0 + j) * N + n] & 0xFF) << (8 * (j & 3));
    int4 *dst = reinterpret_cast<int4 *>(out + (size_t)f * 16);
    *dst = int4{word[0], word[1], word[2], word[3]};
  }
}

// [H][K][N] -> [H][N][K] (selector weights, output-major).
__global__ void k_transpose_heads(const int8_t *__restrict__ w, int H, int K, int N,
                                  int8_t *__restrict__ out) {
  const int total = H * K * N;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const int h = i / (N * K), rem = i - h * N * K, n = rem / K, k = rem - n * K;
    out[i] = w[((size_t)h * K + k) * N + n];
  }
}

struct Binder {
  const uint8_t *wr;
  uint8_t *packed;
  hipStream_t s;
  Slots slots;
  int rc = HV_OK;

  template <class T>
  const T *copy(uint32_t off, size_t bytes) {
    const size_t o = slots.take(bytes);
    if (rc == HV_OK && packed)
      rc = check_hip(hipMemcpyAsync(packed + o, wr + off, bytes, hipMemcpyDeviceToDevice, s),
                     "schedule weight copy");
    return reinterpret_cast<const T *>(packed + o);
  }
  const int8_t *mfma(uint32_t off, int k, int n) {
    const size_t o = slots.take(packed_mfma(k, n));
    if (rc == HV_OK && packed) {
      const int frags = (n + 31) / 32 * (k / 32) * 64;
      hv_launch(k_pack_mfma32, dim3((frags + 255) / 256), dim3(256), 0, s,
                reinterpret_cast<const int8_t *>(wr + off), k, n,
                reinterpret_cast<int8_t *>(packed + o));
      rc = check_hip(hipGetLastError(), "k_pack_mfma32 launch");
    }
    return reinterpret_cast<const int8_t *>(packed + o);
  }
  const int8_t *heads_t(uint32_t off, int h, int k, int n) {
    const size_t o = slots.take((size_t)h * k * n);
    if (rc == HV_OK && packed) {
      hv_launch(k_transpose_heads, dim3((h * k * n + 255) / 256), dim3(256), 0, s,
                reinterpret_cast<const int8_t *>(wr + off), h, k, n,
                reinterpret_cast<int8_t *>(packed + o));
      rc = check_hip(hipGetLastError(), "k_transpose_heads launch");
    }
    return reinterpret_cast<const int8_t *>(packed + o);
  }

  // Fills the pointers of m (exponents already there); with packed == NULL
  // only sizes the buffer.
  void bind(const hv_schedule &sc, hv_model_dev &m) {
    m.patch.weight_p = mfma(sc.patch_w, 768, 192);
    m.patch.bias = copy<int32_t>(sc.patch_b, 192 * 4);
    m.patch.cls = copy<int8_t>(sc.cls, 192);
    m.patch.pos = copy<int8_t>(sc.pos, 197 * 192);
    for (int b = 0; b < 12; ++b) {
      const hv_schedule_block &o = sc.blocks[b];
      hv_block_dev &e = m.blocks[b];
      e.wqkv_p = mfma(o.wqkv, 192, 576);
      e.wproj_p = mfma(o.wproj, 192, 192);
      e.w1_p = mfma(o.w1, 192, 768);
      e.w2_p = mfma(o.w2, 768, 192);
      e.bqkv = copy<int32_t>(o.bqkv, 576 * 4);
      e.bproj = copy<int32_t>(o.bproj, 192 * 4);
      e.b1 = copy<int32_t>(o.b1, 768 * 4);
      e.b2 = copy<int32_t>(o.b2, 192 * 4);
      e.ln1_gamma = copy<int8_t>(o.gamma1, 192);
      e.ln1_beta = copy<int8_t>(o.beta1, 192);
      e.ln2_gamma = copy<int8_t>(o.gamma2, 192);
      e.ln2_beta = copy<int8_t>(o.beta2, 192);
    }
    for (int s = 0; s < sc.model.n_selectors; ++s) {
      const hv_schedule_selector &o = sc.selectors[s];
      hv_selector_dev &e = m.selectors[s];
      e.local_wt = heads_t(o.local_w, 3, 64, 32);
      e.w1t = heads_t(o.score_w1, 3, 64, 32);
      e.w2t = heads_t(o.score_w2, 3, 32, 16);
      e.w3t = heads_t(o.score_w3, 3, 16, 2);
      e.hw_w1t = heads_t(o.hw_w1, 1, 3, 3);
      e.hw_w2t = heads_t(o.hw_w2, 1, 3, 3);
      e.local_b = copy<int32_t>(o.local_b, 96 * 4);
      e.b1 = copy<int32_t>(o.score_b1, 96 * 4);
      e.b2 = copy<int32_t>(o.score_b2, 48 * 4);
      e.b3 = copy<int32_t>(o.score_b3, 6 * 4);
      e.hw_b1 = copy<int32_t>(o.hw_b1, 12);
      e.hw_b2 = copy<int32_t>(o.hw_b2, 12);
    }
    m.final_gamma = copy<int8_t>(sc.final_gamma, 192);
    m.final_beta = copy<int8_t>(sc.final_beta, 192);
    m.head_w_p = mfma(sc.head_w, 192, 1000);
    m.head_b = copy<int32_t>(sc.head_b, 1000 * 4);
  }
};

}  // namespace
}  // namespace hv

using namespace hv;

extern "C" {

int hv_schedule_compile(const uint8_t *words, int n_desc, hv_schedule *out) {
  clear_error();
  if (!words || !out) return fail(HV_EVALUE, HV_ERR_ADDRESS, "schedule: null argument");
  if (n_desc <= 0 || n_desc > 65536)
    return fail(HV_EVALUE, HV_ERR_DIMENSION, "schedule: %d descriptors", n_desc);
  Desc *d = new Desc[n_desc];
  int rc = HV_OK;
  for (int i = 0; i < n_desc && rc == HV_OK; ++i) {
    d[i] = decode(words + (size_t)i * HV_DESC_WORD_BYTES);
    rc = validate(d[i], i);
    // the engine follows next_index; the compiled ROM is sequential (0)
    if (rc == HV_OK && d[i].next != 0 && d[i].next != i + 1)
      rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptor %d: branch to %d", i, d[i].next);
  }
  if (rc) {
    delete[] d;
    return rc;
  }
  hv_schedule sc;
  memset(&sc, 0, sizeof sc);
  hv_model_dev &m = sc.model;
  Reader r{d, n_desc};
  // patch stage (transformer.patch_embedding)
  const Desc *pf = r.take(OP_PATCHIFY, 768);
  const Desc *pg = r.take(OP_GEMM, 192, 768, 0, POST_NONE);
  const Desc *pos = r.take(OP_COPY_ADD_POS, 192);
  if (r.ok()) {
    if (!pf->has(F_SRC0_INPUT) || pf->m != 196 || pos->m != 197)
      r.rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "patch stage shape or source region");
    // PATCHIFY moves bytes: the GEMM reads them at its own src0 exponent
    r.same(pg->s0, pf->sdst, "patch matrix");
    m.patch.image_exp = pg->s0;
    m.patch.weight_exp = pg->s1;
    m.patch.activation_exp = pg->sdst;
    r.gemm_weights(pg, 768 * 192, 192 * 4, &sc.patch_w, &sc.patch_b);
    r.same(pos->s0, m.patch.activation_exp, "patch embedding -> position add");
    m.patch.pos_exp = pos->s1;
    m.patch.cls_exp = pos->saux;
    m.patch.tokens_exp = pos->sdst;
    sc.pos = r.weight(pos->src1, 197 * 192, !pos->has(F_SRC1_SCRATCH));
    sc.cls = r.weight(pos->aux, 192, pos->has(F_AUX_WEIGHT));
  }
  int stream_exp = m.patch.tokens_exp;
  for (int b = 1; b <= 12 && r.ok(); ++b) {
    const Desc *nx = r.peek();
    if (nx && nx->op == OP_GEMM && nx->heads == 3 && nx->n == 32 && nx->post() == POST_GELU) {
      if (m.n_selectors == 3) {
        r.rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "more than three selectors");
        break;
      }
      parse_selector(r, stream_exp, m.selectors[m.n_selectors], sc.selectors[m.n_selectors]);
      m.selector_blocks[m.n_selectors++] = b;
    }
    parse_block(r, stream_exp, m.blocks[b - 1], sc.blocks[b - 1]);
    stream_exp = m.blocks[b - 1].out_exp;
  }
  const Desc *ln = r.take(OP_LAYERNORM);
  const Desc *head = r.take(OP_GEMM, 1000, 192, 0, POST_NONE);
  r.take(OP_FINISH);
  if (r.ok()) {
    r.same(ln->s0, stream_exp, "final LayerNorm input");
    m.final_gamma_exp = ln->s1;
    m.final_beta_exp = ln->saux;
    m.final_ln_out_exp = ln->sdst;
    sc.final_gamma = r.weight(ln->src1, 192, !ln->has(F_SRC1_SCRATCH));
    sc.final_beta = r.weight(ln->aux, 192, ln->has(F_AUX_WEIGHT));
    if (head->m != 1 || !head->has(F_OUT_I32) || !head->has(F_DST_OUTPUT))
      r.rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "classifier shape or destination");
    r.same(head->s0, m.final_ln_out_exp, "final LayerNorm -> classifier");
    m.head_w_exp = head->s1;
    r.same(head->sdst, kLogit, "logits");
    r.gemm_weights(head, 192 * 1000, 1000 * 4, &sc.head_w, &sc.head_b, true);
  }
  if (r.ok() && r.pos != n_desc)
    r.rc = fail(HV_EVALUE, HV_ERR_DIMENSION, "descriptors after FINISH (%d)", r.pos);
  sc.weight_bytes = r.weight_end;
  delete[] d;
  if (r.rc) return r.rc;
  *out = sc;
  return HV_OK;
}

size_t hv_schedule_packed_bytes(const hv_schedule *s) {
  if (!s) return 0;
  hv_model_dev m = s->model;
  Binder b{nullptr, nullptr, nullptr};
  b.bind(*s, m);
  return b.slots.used;
}

int hv_schedule_bind(const hv_schedule *s, const uint8_t *weights, size_t weight_bytes,
                     void *packed, size_t packed_bytes, hv_model_dev *model, hv_stream_t stream) {
  clear_error();
  if (!s || !weights || !packed || !model)
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "schedule bind: null argument");
  if (weight_bytes < s->weight_bytes)
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "weight region of %zu bytes; the schedule reads %llu",
                weight_bytes, (unsigned long long)s->weight_bytes);
  if (packed_bytes < hv_schedule_packed_bytes(s) || ((uintptr_t)packed & 255))
    return fail(HV_EVALUE, HV_ERR_ADDRESS, "packed buffer too small or not 256-byte aligned");
  hv_model_dev m = s->model;
  Binder b{weights, static_cast<uint8_t *>(packed), (hipStream_t)stream};
  b.bind(*s, m);
  if (b.rc) return b.rc;
  *model = m;
  return HV_OK;
}

}  // extern "C"
