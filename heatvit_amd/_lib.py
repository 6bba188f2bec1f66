"""ctypes binding of libheatvit_hip.so (include/heatvit_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in heatvit_amd.
Status codes map onto the golden model's exception types (HV_EVALUE ->
ValueError, HV_EOVERFLOW -> OverflowError, HIP errors -> RuntimeError);
each raised exception carries `error_class`, the reference engine's error
code of the failure (HV_ERR_*, heatvit_pkg.sv:109-118).
"""

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libheatvit_hip.so"

HV_OK, HV_EVALUE, HV_EOVERFLOW, HV_EHIP = 0, -2, -3, -4
(HV_ERR_NONE, HV_ERR_OPCODE, HV_ERR_DIMENSION, HV_ERR_ADDRESS, HV_ERR_TOKEN_COUNT,
 HV_ERR_MEMORY_PROTOCOL, HV_ERR_SOFTMAX_ZERO_SUM, HV_ERR_BUSY_START) = range(8)
HV_WARN_HEAD_DEN_ZERO, HV_WARN_PACKAGE_DEN_ZERO, HV_WARN_LN_NEGATIVE_VARIANCE = 1, 2, 4
HV_PRIM_REQUANT, HV_PRIM_GELU, HV_PRIM_PLAN, HV_PRIM_RSA = 0, 1, 2, 3
HV_PRIM_GELU_POST, HV_PRIM_GELU_TABLE = 4, 5
GELU_TABLE_SO = range(3, 13)
HV_EPI_I8, HV_EPI_I32, HV_EPI_GELU, HV_EPI_RESIDUAL = 0, 1, 2, 3
HV_A_ROWS, HV_A_GATHER, HV_A_UNSIGNED = 0, 1, 4
HV_SELECTOR_NOALLOC_MAX_BATCH = 1024
HV_FWD_PIPELINED = 1
ABI_VERSION = 5
PROF_CLASSES = ("patch", "layernorm", "gemm_qkv", "attention", "gemm_proj", "gemm_ffn1",
                "gemm_ffn2", "selector", "head", "other", "ffn")

_vp = C.c_void_p
_i32 = C.c_int32


class GemmDesc(C.Structure):
    _fields_ = [("a", _vp), ("a_rows", _vp), ("b_packed", _vp), ("bias", _vp), ("c", _vp),
                ("residual", _vp), ("aux", _vp), ("m_dev", _vp)] + [
        (n, _i32) for n in ("m", "n", "k", "lda", "ldc", "ldr", "a_mode", "epilogue",
                            "src_exp", "dst_exp", "mid_exp", "res_exp")]


PATCH_EXPS = ("image_exp", "weight_exp", "activation_exp", "tokens_exp", "cls_exp", "pos_exp")
BLOCK_EXPS = ("x_exp", "gamma1_exp", "beta1_exp", "ln1_out_exp", "wqkv_exp", "qkv_out_exp",
              "score_exp", "prob_exp", "context_out_exp", "wproj_exp", "msa_out_exp",
              "ffn_x_exp", "gamma2_exp", "beta2_exp", "ln2_out_exp", "w1_exp",
              "hidden_out_exp", "w2_exp", "ffn_out_exp", "out_exp")
SELECTOR_EXPS = ("in_exp", "local_w_exp", "local_out_exp", "concat_out_exp", "score_w1_exp",
                 "score_w2_exp", "score_w3_exp", "h1_out_exp", "h2_out_exp",
                 "logits_out_exp", "stats_out_exp", "hw_w1_exp", "hw_hidden_out_exp",
                 "hw_w2_exp")


class PatchDev(C.Structure):
    _fields_ = [("weight_p", _vp), ("bias", _vp), ("cls", _vp), ("pos", _vp)] + [
        (n, _i32) for n in PATCH_EXPS]


class BlockDev(C.Structure):
    _fields_ = [(n, _vp) for n in ("ln1_gamma", "ln1_beta", "wqkv_p", "wproj_p", "ln2_gamma",
                                   "ln2_beta", "w1_p", "w2_p", "bqkv", "bproj", "b1", "b2")] + [
        (n, _i32) for n in BLOCK_EXPS]


class SelectorDev(C.Structure):
    _fields_ = [(n, _vp) for n in ("local_wt", "w1t", "w2t", "w3t", "hw_w1t", "hw_w2t",
                                   "local_b", "b1", "b2", "b3", "hw_b1", "hw_b2")] + [
        (n, _i32) for n in SELECTOR_EXPS]


class ModelDev(C.Structure):
    _fields_ = [("patch", PatchDev), ("blocks", BlockDev * 12), ("selectors", SelectorDev * 3),
                ("n_selectors", _i32), ("selector_blocks", _i32 * 3),
                ("final_gamma", _vp), ("final_beta", _vp), ("head_w_p", _vp), ("head_b", _vp),
                ("final_gamma_exp", _i32), ("final_beta_exp", _i32),
                ("final_ln_out_exp", _i32), ("head_w_exp", _i32)]


SCHEDULE_BLOCK_TENSORS = ("gamma1", "beta1", "wqkv", "bqkv", "wproj", "bproj", "gamma2", "beta2",
                          "w1", "b1", "w2", "b2")
SCHEDULE_SELECTOR_TENSORS = ("local_w", "local_b", "score_w1", "score_b1", "score_w2", "score_b2",
                             "score_w3", "score_b3", "hw_w1", "hw_b1", "hw_w2", "hw_b2")
HV_DESC_WORD_BYTES = 40


class ScheduleBlock(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in SCHEDULE_BLOCK_TENSORS]


class ScheduleSelector(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in SCHEDULE_SELECTOR_TENSORS]


class Schedule(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("patch_w", "patch_b", "cls", "pos")] + [
        ("blocks", ScheduleBlock * 12), ("selectors", ScheduleSelector * 3)] + [
        (n, C.c_uint32) for n in ("final_gamma", "final_beta", "head_w", "head_b")] + [
        ("weight_bytes", C.c_uint64), ("model", ModelDev)]


class SelectorCkpt(C.Structure):
    _fields_ = [(n, _vp) for n in ("local", "global_", "head_scores", "head_stats",
                                   "head_weights", "h2")]


class BlockCkpt(C.Structure):
    _fields_ = [(n, _vp) for n in ("ln1", "fused_qkv", "concat", "msa", "y", "ln2", "hidden",
                                   "ffn_out", "score", "prob")]


_LIB = None


def lib():
    """The loaded library; raises if it is missing or no GPU is visible."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m heatvit_amd.build`")
    import torch  # noqa: F401  (initialises the HIP runtime the library shares)
    if not torch.cuda.is_available():
        raise RuntimeError("heatvit_amd needs a ROCm GPU (gfx950); none is visible")
    L = C.CDLL(str(LIB_PATH))
    _declare(L)
    if L.hv_abi_version() != ABI_VERSION:
        raise RuntimeError("libheatvit_hip.so ABI version mismatch; rebuild it")
    _LIB = L
    return L


def _declare(L):
    """ctypes signatures of every entry point of include/heatvit_hip.h."""
    L.hv_last_error.restype = C.c_char_p
    L.hv_last_error_class.restype = C.c_int
    L.hv_abi_version.restype = C.c_int
    L.hv_eval_primitive.argtypes = [C.c_int, _vp, _vp, C.c_int64, C.c_int, C.c_int, C.c_int, _vp]
    L.hv_softmax_rows.argtypes = [_vp, _vp, C.c_int, _vp, _vp, _vp]
    L.hv_layernorm_i8.argtypes = [_vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int, C.c_int, C.c_int,
                                  C.c_int, _vp, _vp]
    L.hv_attention_i8.argtypes = [_vp, _vp, C.c_int, C.c_int, _vp, _vp, _vp, C.c_int, C.c_int,
                                  C.c_int, C.c_int, _vp, _vp]
    L.hv_gemm_i8.argtypes = [C.POINTER(GemmDesc), _vp]
    L.hv_block_workspace_bytes.restype = C.c_size_t
    L.hv_block_workspace_bytes.argtypes = [C.c_int, C.c_int]
    L.hv_block_forward.argtypes = [C.POINTER(BlockDev), _vp, _vp, C.c_int, C.c_int, _vp,
                                   C.POINTER(BlockCkpt), _vp, _vp, _vp, C.c_size_t, _vp]
    L.hv_selector_workspace_bytes.restype = C.c_size_t
    L.hv_selector_workspace_bytes.argtypes = [C.c_int]
    L.hv_selector_forward.argtypes = [C.POINTER(SelectorDev), _vp, _vp, _vp, C.c_int, _vp, _vp,
                                      _vp, _vp, _vp, _vp, C.POINTER(SelectorCkpt), _vp,
                                      C.c_size_t, _vp]
    L.hv_selector_forward_noalloc.argtypes = [C.POINTER(SelectorDev), _vp, _vp, _vp, C.c_int,
                                              _vp, _vp, _vp, _vp, _vp, _vp,
                                              C.POINTER(SelectorCkpt), _vp]
    L.hv_selector_finalize.argtypes = [_vp, _vp, _vp, _vp, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp]
    L.hv_patch_embedding.argtypes = [C.POINTER(PatchDev), _vp, C.c_int, _vp, _vp]
    L.hv_model_workspace_bytes.restype = C.c_size_t
    L.hv_model_workspace_bytes.argtypes = [C.c_int]
    L.hv_model_forward.argtypes = [C.POINTER(ModelDev), _vp, C.c_int, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _vp, C.c_size_t, _vp]
    L.hv_model_forward_f32.argtypes = L.hv_model_forward.argtypes
    L.hv_model_forward_ex.argtypes = [C.POINTER(ModelDev), _vp, C.c_int, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _vp, C.c_size_t, C.c_int, _vp]
    L.hv_model_forward_f32_ex.argtypes = L.hv_model_forward_ex.argtypes
    L.hv_quantize_images.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]
    L.hv_schedule_compile.argtypes = [_vp, C.c_int, C.POINTER(Schedule)]
    L.hv_schedule_packed_bytes.restype = C.c_size_t
    L.hv_schedule_packed_bytes.argtypes = [C.POINTER(Schedule)]
    L.hv_schedule_bind.argtypes = [C.POINTER(Schedule), _vp, C.c_size_t, _vp, C.c_size_t,
                                   C.POINTER(ModelDev), _vp]
    L.hv_profile_enable.argtypes = [C.c_int]
    L.hv_profile_read.argtypes = [_vp, _vp, C.c_int]


def error(rc, what, L=None):
    """The exception for status rc of the last call on this thread."""
    L = L or lib()
    exc = {HV_EVALUE: ValueError, HV_EOVERFLOW: OverflowError}.get(rc, RuntimeError)
    e = exc(f"{what}: {L.hv_last_error().decode(errors='replace')}")
    e.error_class = L.hv_last_error_class()
    return e


def check(rc, what):
    if rc != HV_OK:
        raise error(rc, what)


def exported_symbols():
    """Names declared in include/heatvit_hip.h (checked by the CPU tests)."""
    return ("hv_last_error", "hv_last_error_class", "hv_abi_version", "hv_eval_primitive",
            "hv_softmax_rows",
            "hv_layernorm_i8", "hv_attention_i8", "hv_gemm_i8", "hv_block_workspace_bytes", "hv_block_forward",
            "hv_selector_workspace_bytes", "hv_selector_forward", "hv_selector_forward_noalloc",
            "hv_selector_finalize",
            "hv_patch_embedding", "hv_profile_enable", "hv_profile_read",
            "hv_model_workspace_bytes", "hv_model_forward", "hv_model_forward_f32",
            "hv_model_forward_ex", "hv_model_forward_f32_ex",
            "hv_quantize_images", "hv_schedule_compile", "hv_schedule_packed_bytes",
            "hv_schedule_bind")
