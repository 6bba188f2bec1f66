"""ctypes view of the CPU oracle (liboracle.so, built from hv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product package
(heatvit_amd) never imports this module.

Parameter objects are the heatvit_amd.params dataclasses (same field names
as the reference's verification/heatvit_ref dataclasses); they are viewed
here through C structs without copying the numpy buffers.
"""

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

OK, EVALUE, EOVERFLOW = 0, -2, -3
WARN_HEAD_DEN_ZERO, WARN_PACKAGE_DEN_ZERO, WARN_LN_NEGATIVE_VARIANCE = 1, 2, 4

_p8 = C.POINTER(C.c_int8)
_pu8 = C.POINTER(C.c_uint8)
_p32 = C.POINTER(C.c_int32)
_p64 = C.POINTER(C.c_int64)


class Patch(C.Structure):
    _fields_ = [("weight", _p8), ("bias", _p32), ("cls", _p8), ("pos", _p8),
                ("width", C.c_int32), ("height", C.c_int32), ("patch", C.c_int32),
                ("image_exp", C.c_int32), ("weight_exp", C.c_int32),
                ("activation_exp", C.c_int32), ("tokens_exp", C.c_int32),
                ("cls_exp", C.c_int32), ("pos_exp", C.c_int32)]


class Block(C.Structure):
    _fields_ = [("ln1_gamma", _p8), ("ln1_beta", _p8), ("wqkv", _p8), ("bqkv", _p32),
                ("wproj", _p8), ("bproj", _p32), ("ln2_gamma", _p8), ("ln2_beta", _p8),
                ("w1", _p8), ("b1", _p32), ("w2", _p8), ("b2", _p32)] + [
        (n, C.c_int32) for n in (
            "x_exp", "gamma1_exp", "beta1_exp", "ln1_out_exp", "wqkv_exp",
            "qkv_out_exp", "score_exp", "prob_exp", "context_out_exp",
            "wproj_exp", "msa_out_exp", "ffn_x_exp", "gamma2_exp", "beta2_exp",
            "ln2_out_exp", "w1_exp", "hidden_out_exp", "w2_exp", "ffn_out_exp",
            "out_exp")]


class Selector(C.Structure):
    _fields_ = [("local_w", _p8), ("local_b", _p32), ("w1", _p8), ("b1", _p32),
                ("w2", _p8), ("b2", _p32), ("w3", _p8), ("b3", _p32),
                ("hw_w1", _p8), ("hw_b1", _p32), ("hw_w2", _p8), ("hw_b2", _p32)] + [
        (n, C.c_int32) for n in (
            "in_exp", "local_w_exp", "local_out_exp", "concat_out_exp",
            "score_w1_exp", "score_w2_exp", "score_w3_exp", "h1_out_exp",
            "h2_out_exp", "logits_out_exp", "stats_out_exp", "hw_w1_exp",
            "hw_hidden_out_exp", "hw_w2_exp")]


class Model(C.Structure):
    _fields_ = [("patch", Patch), ("blocks", Block * 12), ("selectors", Selector * 3),
                ("n_selectors", C.c_int32), ("selector_blocks", C.c_int32 * 3),
                ("final_gamma", _p8), ("final_beta", _p8), ("head_w", _p8),
                ("head_b", _p32), ("final_gamma_exp", C.c_int32),
                ("final_beta_exp", C.c_int32), ("final_ln_out_exp", C.c_int32),
                ("head_w_exp", C.c_int32)]


class BlockCkpt(C.Structure):
    _fields_ = [("ln1", _p8), ("fused_qkv", _p8), ("score", _p32), ("prob", _pu8),
                ("context", _p8), ("concat", _p8), ("msa", _p8), ("y", _p8),
                ("ln2", _p8), ("hidden", _p8), ("ffn_out", _p8), ("warnings", _p32)]


class SelectorCkpt(C.Structure):
    _fields_ = [("local", _p8), ("global_", _p8), ("head_scores", _p32),
                ("head_stats", _p8), ("head_weights", _p32), ("fused", _p32), ("h2", _p8)]


class SelectorState(C.Structure):
    _fields_ = [("token_count", C.c_int32), ("package_present", C.c_int32),
                ("kept_normal_count", C.c_int32), ("pruned_normal_count", C.c_int32),
                ("warnings", C.c_int32)]


def build(force=False):
    """Compile liboracle.so with the committed Makefile (with
    HEATVIT_ORACLE_LIB set, that library is used as built)."""
    if os.environ.get("HEATVIT_ORACLE_LIB"):
        return
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-B" if force else "liboracle.so"], cwd=HERE,
                       check=True)


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.environ.get("HEATVIT_ORACLE_LIB")
        if not path:
            if not LIB_PATH.exists():
                build()
            path = str(LIB_PATH)
        L = C.CDLL(path)
        L.hvo_round_shift_away.restype = C.c_int64
        L.hvo_round_shift_away.argtypes = [C.c_int64, C.c_int]
        L.hvo_sat_signed.restype = C.c_int64
        L.hvo_sat_signed.argtypes = [C.c_int64, C.c_int]
        L.hvo_requant.restype = C.c_int64
        L.hvo_requant.argtypes = [C.c_int64, C.c_int, C.c_int, C.c_int]
        L.hvo_requant_array.restype = None
        L.hvo_requant_array.argtypes = [_p64, _p64, C.c_int64, C.c_int, C.c_int, C.c_int]
        L.hvo_round_div.argtypes = [C.c_int64, C.c_int64, _p64]
        L.hvo_udiv.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64),
                               C.POINTER(C.c_uint64)]
        L.hvo_isqrt.restype = C.c_uint64
        L.hvo_isqrt.argtypes = [C.c_uint64, C.POINTER(C.c_uint64)]
        L.hvo_gelu.restype = C.c_int32
        L.hvo_gelu.argtypes = [C.c_int32]
        L.hvo_gelu_array.restype = None
        L.hvo_gelu_array.argtypes = [_p32, _p32, C.c_int64]
        L.hvo_plan_sigmoid.restype = C.c_int32
        L.hvo_plan_sigmoid.argtypes = [C.c_int32]
        L.hvo_softmax_attention.argtypes = [_p32, C.c_int, _pu8]
        L.hvo_softmax_selector.argtypes = [_p32, C.c_int, _p32]
        L.hvo_layernorm.argtypes = [_p8, _p8, _p8, C.c_int, C.c_int, C.c_int, C.c_int,
                                    _p8, C.POINTER(C.c_int)]
        L.hvo_gemm.argtypes = [C.c_void_p, _p8, _p32, C.c_int, C.c_int, C.c_int,
                               C.c_int, C.c_int, _p64]
        L.hvo_gemm_writeback.argtypes = [_p64, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.c_void_p]
        L.hvo_patch_embedding.argtypes = [_p8, C.POINTER(Patch), _p8]
        L.hvo_transformer_block.argtypes = [_p8, C.c_int, C.POINTER(Block), _p8,
                                            C.POINTER(BlockCkpt)]
        L.hvo_fuse_head_scores.restype = None
        L.hvo_fuse_head_scores.argtypes = [_p32, _p32, C.c_int, _p32, C.POINTER(C.c_int)]
        L.hvo_finalize_tokens.argtypes = [_p8, _p8, C.c_int, _p8, _p32, C.c_int, C.c_int,
                                          _p8, _p32, C.POINTER(SelectorState)]
        L.hvo_token_selector.argtypes = [_p8, C.c_int, C.c_int, C.POINTER(Selector), _p8,
                                         _p32, C.POINTER(SelectorState),
                                         C.POINTER(SelectorCkpt)]
        L.hvo_patchify.argtypes = [_p8, C.c_int, C.c_int, C.c_int, _p8]
        L.hvo_quantize_image.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_int, C.c_int, _p8]
        L.hvo_model_infer.argtypes = [_p8, C.POINTER(Model), _p32, _p8, _p32,
                                      C.POINTER(SelectorState), _p32]
        L.hvo_model_infer_batch.argtypes = [_p8, C.c_int, C.POINTER(Model), C.c_int,
                                            _p32, _p32, _p32, _p32]
        _LIB = L
    return _LIB


def _ptr(arr, typ):
    if arr is None:
        return None
    assert arr.flags["C_CONTIGUOUS"]
    return arr.ctypes.data_as(typ)


def _check(rc, what):
    if rc == EVALUE:
        raise ValueError(f"oracle {what}: invalid input")
    if rc == EOVERFLOW:
        raise OverflowError(f"oracle {what}: GEMM accumulator exceeds int32")
    if rc != OK:
        raise RuntimeError(f"oracle {what}: status {rc}")


# ---------------------------------------------------------------- primitives

def round_shift_away(v, s):
    return lib().hvo_round_shift_away(int(v), int(s))


def sat_signed(v, bits):
    return lib().hvo_sat_signed(int(v), int(bits))


def requant(v, src, dst, bits):
    return lib().hvo_requant(int(v), int(src), int(dst), int(bits))


def requant_array(values, src, dst, bits):
    v = np.ascontiguousarray(values, np.int64)
    out = np.empty_like(v)
    lib().hvo_requant_array(_ptr(v, _p64), _ptr(out, _p64), v.size, src, dst, bits)
    return out


def round_div(n, d):
    out = C.c_int64()
    _check(lib().hvo_round_div(int(n), int(d), C.byref(out)), "round_div")
    return out.value


def udiv(n, d):
    q, r = C.c_uint64(), C.c_uint64()
    _check(lib().hvo_udiv(int(n), int(d), C.byref(q), C.byref(r)), "udiv")
    return q.value, r.value


def isqrt(x):
    rem = C.c_uint64()
    root = lib().hvo_isqrt(int(x), C.byref(rem))
    return root, rem.value


def gelu(x):
    return lib().hvo_gelu(int(x))


def gelu_array(xs):
    x = np.ascontiguousarray(xs, np.int32)
    out = np.empty_like(x)
    lib().hvo_gelu_array(_ptr(x, _p32), _ptr(out, _p32), x.size)
    return out


def plan_sigmoid(x):
    return lib().hvo_plan_sigmoid(int(x))


def softmax_attention(row):
    x = np.ascontiguousarray(row, dtype=np.int32)
    out = np.zeros(len(x), np.uint8)
    _check(lib().hvo_softmax_attention(_ptr(x, _p32), len(x), _ptr(out, _pu8)), "softmax")
    return out


def softmax_selector(row):
    x = np.ascontiguousarray(row, dtype=np.int32)
    out = np.zeros(len(x), np.int32)
    _check(lib().hvo_softmax_selector(_ptr(x, _p32), len(x), _ptr(out, _p32)), "softmax")
    return out


def layernorm(x, gamma, beta, x_exp, g_exp, b_exp, out_exp):
    x = np.ascontiguousarray(x, np.int8)
    g = np.ascontiguousarray(gamma, np.int8)
    b = np.ascontiguousarray(beta, np.int8)
    out = np.zeros(192, np.int8)
    neg = C.c_int()
    _check(lib().hvo_layernorm(_ptr(x, _p8), _ptr(g, _p8), _ptr(b, _p8), x_exp, g_exp,
                               b_exp, out_exp, _ptr(out, _p8), C.byref(neg)), "layernorm")
    return out, bool(neg.value)


def layernorm_rows(x, gamma, beta, x_exp, g_exp, b_exp, out_exp):
    x = np.ascontiguousarray(x, np.int8).reshape(-1, 192)
    return np.stack([layernorm(r, gamma, beta, x_exp, g_exp, b_exp, out_exp)[0]
                     for r in x]) if len(x) else np.zeros((0, 192), np.int8)


def gemm(a, b, bias, transpose_b=False, a_unsigned=False):
    a = np.ascontiguousarray(a, np.uint8 if a_unsigned else np.int8)
    b = np.ascontiguousarray(b, np.int8)
    m, k = a.shape
    n = b.shape[0] if transpose_b else b.shape[1]
    bias_arr = None if bias is None else np.ascontiguousarray(bias, np.int32)
    acc = np.zeros((m, n), np.int64)
    _check(lib().hvo_gemm(a.ctypes.data, _ptr(b, _p8), _ptr(bias_arr, _p32), m, n, k,
                          int(transpose_b), int(a_unsigned), _ptr(acc, _p64)), "gemm")
    return acc


def gemm_writeback(acc, src_exp, dst_exp, bits):
    acc = np.ascontiguousarray(acc, np.int64)
    out = np.zeros(acc.shape, np.int8 if bits == 8 else np.int32)
    _check(lib().hvo_gemm_writeback(_ptr(acc, _p64), acc.size, src_exp, dst_exp, bits,
                                    out.ctypes.data), "gemm_writeback")
    return out


def attention(fused_qkv, qkv_exp, score_exp, prob_exp, context_exp):
    """The attention core of mhsa (transformer.py:228-266) composed from the
    primitives above, for one image: fused_qkv [N][576] int8 with Q, K, V
    column blocks and heads of 64 lanes (layout.qkv_unpack,
    layout.py:92-129).  Returns (score [3][N][N] int32, prob [3][N][N]
    uint8, concat [N][192] int8), concat in head-major lane order
    (layout.head_concat, layout.py:132-155)."""
    x = np.ascontiguousarray(fused_qkv, np.int8)
    n = len(x)
    score = np.zeros((3, n, n), np.int32)
    prob = np.zeros((3, n, n), np.uint8)
    concat = np.zeros((n, 192), np.int8)
    for h in range(3):
        q, k, v = (x[:, blk * 192 + h * 64: blk * 192 + h * 64 + 64] for blk in range(3))
        # transformer.py:230-234
        score[h] = gemm_writeback(gemm(q, k, None, transpose_b=True), 2 * qkv_exp, score_exp, 32)
        # transformer.py:236-254: q16 = sat24(rsa(score, -(score_exp + 13)))
        q16 = requant_array(score[h], 0, -(score_exp + 13), 24)
        for r in range(n):
            prob[h, r] = softmax_attention(q16[r])
        # transformer.py:256-264
        concat[:, h * 64:(h + 1) * 64] = gemm_writeback(
            gemm(prob[h], v, None, a_unsigned=True), prob_exp + qkv_exp, context_exp, 8)
    return score, prob, concat


# ---------------------------------------------------------------- params

class _Keep:
    """Holds the numpy arrays a C struct points into."""

    def __init__(self):
        self.arrays = []

    def p(self, arr, dtype, typ):
        a = np.ascontiguousarray(arr, dtype)
        self.arrays.append(a)
        return a.ctypes.data_as(typ)


def patch_struct(pp, keep):
    return Patch(keep.p(pp.patch_weight, np.int8, _p8), keep.p(pp.patch_bias, np.int32, _p32),
                 keep.p(pp.cls, np.int8, _p8), keep.p(pp.pos, np.int8, _p8),
                 pp.width, pp.height, pp.patch, pp.image_scale_exp, pp.weight_scale_exp,
                 pp.activation_scale_exp, pp.tokens_scale_exp, pp.cls_scale_exp,
                 pp.pos_scale_exp)


def block_struct(bp, keep):
    m, f = bp.mhsa, bp.ffn
    s = Block()
    s.ln1_gamma = keep.p(m.ln_gamma, np.int8, _p8)
    s.ln1_beta = keep.p(m.ln_beta, np.int8, _p8)
    s.wqkv = keep.p(m.wqkv, np.int8, _p8)
    s.bqkv = keep.p(m.bqkv, np.int32, _p32)
    s.wproj = keep.p(m.wproj, np.int8, _p8)
    s.bproj = keep.p(m.bproj, np.int32, _p32)
    s.ln2_gamma = keep.p(f.ln_gamma, np.int8, _p8)
    s.ln2_beta = keep.p(f.ln_beta, np.int8, _p8)
    s.w1 = keep.p(f.w1, np.int8, _p8)
    s.b1 = keep.p(f.b1, np.int32, _p32)
    s.w2 = keep.p(f.w2, np.int8, _p8)
    s.b2 = keep.p(f.b2, np.int32, _p32)
    s.x_exp, s.gamma1_exp, s.beta1_exp = m.x_scale_exp, m.gamma1_scale_exp, m.beta1_scale_exp
    s.ln1_out_exp, s.wqkv_exp, s.qkv_out_exp = (m.ln1_out_scale_exp, m.wqkv_scale_exp,
                                                m.qkv_out_scale_exp)
    s.score_exp, s.prob_exp = m.score_scale_exp, m.prob_scale_exp
    s.context_out_exp, s.wproj_exp, s.msa_out_exp = (m.context_out_scale_exp,
                                                     m.wproj_scale_exp, m.msa_out_scale_exp)
    s.ffn_x_exp, s.gamma2_exp, s.beta2_exp = f.x_scale_exp, f.gamma2_scale_exp, f.beta2_scale_exp
    s.ln2_out_exp, s.w1_exp, s.hidden_out_exp = (f.ln2_out_scale_exp, f.w1_scale_exp,
                                                 f.hidden_out_scale_exp)
    s.w2_exp, s.ffn_out_exp, s.out_exp = f.w2_scale_exp, f.ffn_out_scale_exp, f.out_scale_exp
    return s


def selector_struct(sp, keep):
    s = Selector()
    s.local_w = keep.p(sp.local.w, np.int8, _p8)
    s.local_b = keep.p(sp.local.b, np.int32, _p32)
    s.w1 = keep.p(sp.score.w1, np.int8, _p8)
    s.b1 = keep.p(sp.score.b1, np.int32, _p32)
    s.w2 = keep.p(sp.score.w2, np.int8, _p8)
    s.b2 = keep.p(sp.score.b2, np.int32, _p32)
    s.w3 = keep.p(sp.score.w3, np.int8, _p8)
    s.b3 = keep.p(sp.score.b3, np.int32, _p32)
    s.hw_w1 = keep.p(sp.head_weight.w1, np.int8, _p8)
    s.hw_b1 = keep.p(sp.head_weight.b1, np.int32, _p32)
    s.hw_w2 = keep.p(sp.head_weight.w2, np.int8, _p8)
    s.hw_b2 = keep.p(sp.head_weight.b2, np.int32, _p32)
    for cname, pname in (("in_exp", "in_scale_exp"), ("local_w_exp", "local_w_scale_exp"),
                         ("local_out_exp", "local_out_scale_exp"),
                         ("concat_out_exp", "concat_out_scale_exp"),
                         ("score_w1_exp", "score_w1_scale_exp"),
                         ("score_w2_exp", "score_w2_scale_exp"),
                         ("score_w3_exp", "score_w3_scale_exp"),
                         ("h1_out_exp", "h1_out_scale_exp"), ("h2_out_exp", "h2_out_scale_exp"),
                         ("logits_out_exp", "logits_out_scale_exp"),
                         ("stats_out_exp", "stats_out_scale_exp"),
                         ("hw_w1_exp", "hw_w1_scale_exp"),
                         ("hw_hidden_out_exp", "hw_hidden_out_scale_exp"),
                         ("hw_w2_exp", "hw_w2_scale_exp")):
        setattr(s, cname, getattr(sp, pname))
    return s


def model_struct(params, keep):
    s = Model()
    s.patch = patch_struct(params.patch, keep)
    for i, bp in enumerate(params.blocks):
        s.blocks[i] = block_struct(bp, keep)
    for i, sp in enumerate(params.selectors):
        s.selectors[i] = selector_struct(sp, keep)
    s.n_selectors = len(params.selectors)
    for i, b in enumerate(params.selector_blocks):
        s.selector_blocks[i] = b
    s.final_gamma = keep.p(params.final_gamma, np.int8, _p8)
    s.final_beta = keep.p(params.final_beta, np.int8, _p8)
    s.head_w = keep.p(params.head_w, np.int8, _p8)
    s.head_b = keep.p(params.head_b, np.int32, _p32)
    s.final_gamma_exp = params.final_gamma_scale_exp
    s.final_beta_exp = params.final_beta_scale_exp
    s.final_ln_out_exp = params.final_ln_out_scale_exp
    s.head_w_exp = params.head_w_scale_exp
    return s


# ---------------------------------------------------------------- composites

def quantize_image(chw, input_exp):
    """p2_export_weights.real_image_list: float CHW [3][H][W] -> int8 NHWC
    [H*W*3]."""
    chw = np.ascontiguousarray(chw, np.float32)
    _, h, w = chw.shape
    out = np.zeros(h * w * 3, np.int8)
    _check(lib().hvo_quantize_image(chw.ctypes.data_as(C.POINTER(C.c_float)), w, h, input_exp,
                                    _ptr(out, _p8)), "quantize_image")
    return out


def patchify(image, width=224, height=224, patch=16):
    """layout.patchify: flat NHWC int8 image -> [(H/P)*(W/P)][P*P*3]."""
    img = np.ascontiguousarray(image, np.int8).reshape(-1)
    out = np.zeros(((height // patch) * (width // patch), patch * patch * 3), np.int8)
    _check(lib().hvo_patchify(_ptr(img, _p8), width, height, patch, _ptr(out, _p8)), "patchify")
    return out


def patch_embedding(image, pp):
    keep = _Keep()
    img = np.ascontiguousarray(image, np.int8).reshape(-1)
    st = patch_struct(pp, keep)
    out = np.zeros((197, 192), np.int8)
    _check(lib().hvo_patch_embedding(_ptr(img, _p8), C.byref(st), _ptr(out, _p8)), "patch")
    return out


BLOCK_KEYS = ("ln1", "fused_qkv", "score", "prob", "context", "concat", "msa", "y",
              "ln2", "hidden", "ffn_out")


def transformer_block(x, bp, checkpoints=True):
    """Returns (z, checkpoints) with the reference's checkpoint keys
    (transformer.py:274-283, 378-383, 428-431); qkv is derived from
    fused_qkv by layout.qkv_unpack semantics.  checkpoints["warnings"] is
    the engine's LayerNorm warning bit of the block (WARN_LN_NEGATIVE_VARIANCE
    or 0)."""
    keep = _Keep()
    x = np.ascontiguousarray(x, np.int8).reshape(-1, 192)
    n = len(x)
    st = block_struct(bp, keep)
    z = np.zeros((n, 192), np.int8)
    warn = np.zeros(1, np.int32)
    ck = BlockCkpt(warnings=_ptr(warn, _p32))
    bufs = {}
    if checkpoints:
        bufs = dict(ln1=np.zeros((n, 192), np.int8), fused_qkv=np.zeros((n, 576), np.int8),
                    score=np.zeros((3, n, n), np.int32), prob=np.zeros((3, n, n), np.uint8),
                    context=np.zeros((3, n, 64), np.int8), concat=np.zeros((n, 192), np.int8),
                    msa=np.zeros((n, 192), np.int8), y=np.zeros((n, 192), np.int8),
                    ln2=np.zeros((n, 192), np.int8), hidden=np.zeros((n, 768), np.int8),
                    ffn_out=np.zeros((n, 192), np.int8))
        ck = BlockCkpt(*[
            _ptr(bufs[k], {np.int8: _p8, np.int32: _p32, np.uint8: _pu8}[bufs[k].dtype.type])
            for k in BLOCK_KEYS], _ptr(warn, _p32))
    _check(lib().hvo_transformer_block(_ptr(x, _p8), n, C.byref(st), _ptr(z, _p8),
                                       C.byref(ck)), "block")
    if checkpoints:
        bufs["qkv"] = bufs["fused_qkv"].reshape(n, 3, 3, 64).transpose(1, 2, 0, 3).copy()
        bufs["z"] = z
    bufs["warnings"] = int(warn[0])
    return z, bufs


def fuse_head_scores(head_scores, head_weights):
    """head_scores [3][C], head_weights [C][3] -> (fused [C], warn 0/1)."""
    hs = np.ascontiguousarray(head_scores, np.int32)
    hw = np.ascontiguousarray(head_weights, np.int32)
    c = hs.shape[1]
    fused = np.zeros(c, np.int32)
    warn = C.c_int()
    lib().hvo_fuse_head_scores(_ptr(hs, _p32), _ptr(hw, _p32), c, _ptr(fused, _p32),
                               C.byref(warn))
    return fused, warn.value


def finalize_tokens(cls, normal, incoming, scores):
    cls = np.ascontiguousarray(cls, np.int8)
    width = len(cls)
    normal = np.ascontiguousarray(normal, np.int8).reshape(-1, width)
    inc = None if incoming is None else np.ascontiguousarray(incoming, np.int8)
    sc = np.ascontiguousarray(scores, np.int32)
    out = np.zeros((len(normal) + 2, width), np.int8)
    kept = np.zeros(max(len(normal), 1), np.int32)
    st = SelectorState()
    _check(lib().hvo_finalize_tokens(_ptr(cls, _p8), _ptr(normal, _p8), len(normal),
                                     _ptr(inc, _p8), _ptr(sc, _p32), len(sc), width,
                                     _ptr(out, _p8), _ptr(kept, _p32), C.byref(st)),
           "finalize")
    return out[:st.token_count].copy(), kept[:st.kept_normal_count].copy(), st


SELECTOR_KEYS = ("local", "global_features", "head_scores", "head_stats", "head_weights",
                 "fused_scores", "h2")


def token_selector(tokens, package_present, sp, checkpoints=True):
    keep = _Keep()
    tokens = np.ascontiguousarray(tokens, np.int8).reshape(-1, 192)
    n = len(tokens)
    c = n - 1
    st = selector_struct(sp, keep)
    out = np.zeros((n + 1, 192), np.int8)
    kept = np.zeros(max(c, 1), np.int32)
    state = SelectorState()
    bufs = dict(local=np.zeros((3, c, 32), np.int8), global_features=np.zeros((3, 32), np.int8),
                head_scores=np.zeros((3, c), np.int32), head_stats=np.zeros((c, 3), np.int8),
                head_weights=np.zeros((c, 3), np.int32), fused_scores=np.zeros(c, np.int32),
                h2=np.zeros((3, c, 16), np.int8))
    ck = SelectorCkpt(_ptr(bufs["local"], _p8), _ptr(bufs["global_features"], _p8),
                      _ptr(bufs["head_scores"], _p32), _ptr(bufs["head_stats"], _p8),
                      _ptr(bufs["head_weights"], _p32), _ptr(bufs["fused_scores"], _p32),
                      _ptr(bufs["h2"], _p8))
    _check(lib().hvo_token_selector(_ptr(tokens, _p8), n, int(bool(package_present)),
                                    C.byref(st), _ptr(out, _p8), _ptr(kept, _p32),
                                    C.byref(state), C.byref(ck) if checkpoints else None),
           "token_selector")
    result = dict(tokens=out[:state.token_count].copy(), token_count=state.token_count,
                  package_present=bool(state.package_present),
                  kept_normal_count=state.kept_normal_count,
                  pruned_normal_count=state.pruned_normal_count, warnings=state.warnings,
                  kept_index=kept[:state.kept_normal_count].copy())
    if checkpoints:
        result.update(bufs)
    return result


CKPT_NAMES = (["patch"] + [f"selector_{i:02d}" for i in range(1, 4)] +
              [f"block_{i:02d}" for i in range(1, 13)] + ["final_ln"])


def model_infer(image, params, checkpoints=True):
    """Returns (logits[1000] int32, checkpoints dict, selector summary list,
    warning bits of the forward)."""
    keep = _Keep()
    st = model_struct(params, keep)
    img = np.ascontiguousarray(image, np.int8).reshape(-1)
    logits = np.zeros(1000, np.int32)
    ck = np.zeros((17, 197, 192), np.int8) if checkpoints else None
    rows = np.zeros(17, np.int32)
    summ = (SelectorState * 3)()
    warn = np.zeros(1, np.int32)
    _check(lib().hvo_model_infer(_ptr(img, _p8), C.byref(st), _ptr(logits, _p32),
                                 _ptr(ck, _p8), _ptr(rows, _p32), summ, _ptr(warn, _p32)),
           "infer")
    cks = {}
    if checkpoints:
        for i, name in enumerate(CKPT_NAMES):
            if rows[i]:
                cks[name] = ck[i, :rows[i]].copy()
        cks["logits"] = logits.copy()
    summary = [dict(token_count=s.token_count, package_present=s.package_present,
                    kept_normal=s.kept_normal_count, pruned_normal=s.pruned_normal_count,
                    warnings=s.warnings) for s in list(summ)[:len(params.selectors)]]
    return logits, cks, summary, int(warn[0])


def model_infer_batch(images, params, threads=None):
    """Oracle over a batch with OpenMP; returns (logits [B][1000],
    token_counts [B][4], status [B], warnings [B])."""
    keep = _Keep()
    st = model_struct(params, keep)
    imgs = np.ascontiguousarray(images, np.int8)
    b = imgs.shape[0]
    logits = np.zeros((b, 1000), np.int32)
    counts = np.zeros((b, 4), np.int32)
    status = np.zeros(b, np.int32)
    warnings = np.zeros(b, np.int32)
    threads = threads or os.cpu_count() or 1
    lib().hvo_model_infer_batch(_ptr(imgs, _p8), b, C.byref(st), threads,
                                _ptr(logits, _p32), _ptr(counts, _p32), _ptr(status, _p32),
                                _ptr(warnings, _p32))
    return logits, counts, status, warnings
