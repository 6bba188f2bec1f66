"""Device-resident, kernel-ready parameter sets.

The reference keeps weights as nested tuples in row-major [K][N]
(docs/heatvit.md:181-190).  Here every GEMM weight is packed once into the
"mfma32" operand layout (include/heatvit_hip.h), selector MLP weights are
stored output-major for v_dot4, and the C parameter views hold the device
pointers plus the per-tensor scale exponents.
"""

import numpy as np
import torch

from . import _lib
from .params import BlockParams, HeatViTParams, SelectorParams, check_scale_exps, coerce


# Position of output channel c (0..31) of a weight tile among the MFMA
# operand rows: channel 16*h + 4*a + b sits at row 8*a + 4*h + b, so result
# lane l of the transposed product holds channels 16*(l//32) .. +15.
MFMA32_ROW_OF_CHANNEL = np.array([8 * ((c % 16) // 4) + 4 * (c // 16) + c % 4 for c in range(32)])
MFMA32_CHANNEL_OF_ROW = np.argsort(MFMA32_ROW_OF_CHANNEL)


def pack_mfma32(w):
    """Pack an int8 matrix W[K][N] (K % 32 == 0) into the mfma32 layout:
    [ceil(N/32)][K/32][64 lanes][16 bytes], element (k, n) at tile
    (n // 32, k // 32), lane MFMA32_ROW_OF_CHANNEL[n % 32] + 32 * ((k % 32) // 16),
    byte k % 16, zero-padded columns."""
    w = np.asarray(w, np.int8)
    k, n = w.shape
    if k % 32:
        raise ValueError(f"mfma32 packing needs K % 32 == 0 (K={k})")
    n32 = -(-n // 32) * 32
    wp = np.zeros((k, n32), np.int8)
    wp[:, :n] = w
    wp = wp.reshape(k, n32 // 32, 32)[:, :, MFMA32_CHANNEL_OF_ROW].reshape(k, n32)
    t = wp.reshape(k // 32, 2, 16, n32 // 32, 32).transpose(3, 0, 1, 4, 2)
    return np.ascontiguousarray(t).reshape(-1)


def unpack_mfma32(packed, k, n):
    """Inverse of pack_mfma32 (used by tests)."""
    n32 = -(-n // 32) * 32
    t = np.asarray(packed, np.int8).reshape(n32 // 32, k // 32, 2, 32, 16)
    wp = t.transpose(1, 2, 4, 0, 3).reshape(k, n32 // 32, 32)[:, :, MFMA32_ROW_OF_CHANNEL]
    return np.ascontiguousarray(wp.reshape(k, n32)[:, :n])


class _Holder:
    """Keeps the device tensors a C struct points into."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.tensors = []

    def put(self, arr, dtype):
        t = torch.from_numpy(np.array(arr, dtype=dtype, copy=True, order="C")).to(self.device)
        self.tensors.append(t)
        return t.data_ptr()


def _block_struct(bp, h):
    m, f = bp.mhsa, bp.ffn
    s = _lib.BlockDev()
    s.ln1_gamma = h.put(m.ln_gamma, np.int8)
    s.ln1_beta = h.put(m.ln_beta, np.int8)
    s.wqkv_p = h.put(pack_mfma32(m.wqkv), np.int8)
    s.wproj_p = h.put(pack_mfma32(m.wproj), np.int8)
    s.ln2_gamma = h.put(f.ln_gamma, np.int8)
    s.ln2_beta = h.put(f.ln_beta, np.int8)
    s.w1_p = h.put(pack_mfma32(f.w1), np.int8)
    s.w2_p = h.put(pack_mfma32(f.w2), np.int8)
    s.bqkv = h.put(m.bqkv, np.int32)
    s.bproj = h.put(m.bproj, np.int32)
    s.b1 = h.put(f.b1, np.int32)
    s.b2 = h.put(f.b2, np.int32)
    exps = (m.x_scale_exp, m.gamma1_scale_exp, m.beta1_scale_exp, m.ln1_out_scale_exp,
            m.wqkv_scale_exp, m.qkv_out_scale_exp, m.score_scale_exp, m.prob_scale_exp,
            m.context_out_scale_exp, m.wproj_scale_exp, m.msa_out_scale_exp,
            f.x_scale_exp, f.gamma2_scale_exp, f.beta2_scale_exp, f.ln2_out_scale_exp,
            f.w1_scale_exp, f.hidden_out_scale_exp, f.w2_scale_exp, f.ffn_out_scale_exp,
            f.out_scale_exp)
    for name, v in zip(_lib.BLOCK_EXPS, exps):
        setattr(s, name, int(v))
    return s


def _selector_struct(sp, h):
    s = _lib.SelectorDev()
    t = lambda w: np.swapaxes(np.asarray(w), -1, -2)  # noqa: E731  output-major
    s.local_wt = h.put(t(sp.local.w), np.int8)
    s.w1t = h.put(t(sp.score.w1), np.int8)
    s.w2t = h.put(t(sp.score.w2), np.int8)
    s.w3t = h.put(t(sp.score.w3), np.int8)
    s.hw_w1t = h.put(t(sp.head_weight.w1), np.int8)
    s.hw_w2t = h.put(t(sp.head_weight.w2), np.int8)
    s.local_b = h.put(sp.local.b, np.int32)
    s.b1 = h.put(sp.score.b1, np.int32)
    s.b2 = h.put(sp.score.b2, np.int32)
    s.b3 = h.put(sp.score.b3, np.int32)
    s.hw_b1 = h.put(sp.head_weight.b1, np.int32)
    s.hw_b2 = h.put(sp.head_weight.b2, np.int32)
    exps = (sp.in_scale_exp, sp.local_w_scale_exp, sp.local_out_scale_exp,
            sp.concat_out_scale_exp, sp.score_w1_scale_exp, sp.score_w2_scale_exp,
            sp.score_w3_scale_exp, sp.h1_out_scale_exp, sp.h2_out_scale_exp,
            sp.logits_out_scale_exp, sp.stats_out_scale_exp, sp.hw_w1_scale_exp,
            sp.hw_hidden_out_scale_exp, sp.hw_w2_scale_exp)
    for name, v in zip(_lib.SELECTOR_EXPS, exps):
        setattr(s, name, int(v))
    return s


def _patch_struct(pp, h):
    s = _lib.PatchDev()
    s.weight_p = h.put(pack_mfma32(pp.patch_weight), np.int8)
    s.bias = h.put(pp.patch_bias, np.int32)
    s.cls = h.put(pp.cls, np.int8)
    s.pos = h.put(pp.pos, np.int8)
    exps = (pp.image_scale_exp, pp.weight_scale_exp, pp.activation_scale_exp,
            pp.tokens_scale_exp, pp.cls_scale_exp, pp.pos_scale_exp)
    for name, v in zip(_lib.PATCH_EXPS, exps):
        setattr(s, name, int(v))
    return s


class DeviceBlock:
    def __init__(self, params, device="cuda"):
        params = coerce(params, BlockParams)
        check_scale_exps(params)
        self.params = params
        self.holder = _Holder(device)
        self.struct = _block_struct(params, self.holder)


class DeviceSelector:
    def __init__(self, params, device="cuda"):
        params = coerce(params, SelectorParams)
        check_scale_exps(params)
        self.params = params
        self.holder = _Holder(device)
        self.struct = _selector_struct(params, self.holder)


class DeviceModel:
    """HeatViTParams uploaded once (about 6 MB of packed weights)."""

    def __init__(self, params, device="cuda"):
        params = coerce(params, HeatViTParams)
        if (params.patch.width, params.patch.height, params.patch.patch) != (224, 224, 16):
            raise ValueError("the HIP patch embedding handles 224x224x3 images with 16x16 patches")
        check_scale_exps(params)
        self.params = params
        self.holder = _Holder(device)
        s = _lib.ModelDev()
        s.patch = _patch_struct(params.patch, self.holder)
        for i, bp in enumerate(params.blocks):
            s.blocks[i] = _block_struct(bp, self.holder)
        for i, sp in enumerate(params.selectors):
            s.selectors[i] = _selector_struct(sp, self.holder)
        s.n_selectors = len(params.selectors)
        for i, b in enumerate(params.selector_blocks):
            s.selector_blocks[i] = b
        s.final_gamma = self.holder.put(params.final_gamma, np.int8)
        s.final_beta = self.holder.put(params.final_beta, np.int8)
        s.head_w_p = self.holder.put(pack_mfma32(params.head_w), np.int8)
        s.head_b = self.holder.put(params.head_b, np.int32)
        s.final_gamma_exp = params.final_gamma_scale_exp
        s.final_beta_exp = params.final_beta_scale_exp
        s.final_ln_out_exp = params.final_ln_out_scale_exp
        s.head_w_exp = params.head_w_scale_exp
        self.struct = s
        self.device = self.holder.device
