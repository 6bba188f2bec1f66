"""Deterministic synthetic HeatViT-T workloads (inputs, weights, exponents).

The five workloads are:
  block     one Pre-LN block, x [197][192] uniform int8 (batch 1)
  full      full model, selectors disabled, one 224x224x3 image
  selector  token selector alone, 64 x [197][192] uniform int8 tokens
  pruned    full model with selectors before blocks 4/7/10, calibrated to the
            197 -> 88 -> 45 -> 32 token budget, 32 images
  throughput  the pruned model over 256 images (images 0..31 equal the
            pruned workload's), plus an unpruned control with the same
            weights and no selectors

Random numbers come from a counter-based generator: the n-th 64-bit word of
tensor `name` under seed `s` is splitmix64_mix(key(s, name) + (n+1)*phi),
phi = 0x9E3779B97F4A7C15, key(s, name) = splitmix64_mix(s ^ fnv1a64(name)).
It is order-independent (every tensor has its own stream) and vectorises in
numpy.

Distributions (integer only, no floating point):
  uniform int8     every byte of the word stream, minus 128
  normal(sigma)    s = sum of the twelve 16-bit chunks of three words minus
                   6*65535 (Irwin-Hall, variance ~65536^2), value =
                   round_div(sigma * s, 65536) (ties away), int8 weights
                   clipped to [-127, 127]; sigma 40 for int8 tensors
                   (weights, gamma, beta, cls, pos), 1024 for int32 biases
  scale exps       uniform integer in [-12, -4] per tensor, except the
                   derived ones: score = 2*qkv_out - 3, prob = -8, chained
                   inputs equal the producing tensor's output exponent,
                   selector concat_out = local_out and stats_out = in
                   (the selector relabels these without rescaling).
  selectors        the calibration (tests/golden/calibrate.py, stored in
                   data/calibration.json) picks, per selector, one of 16
                   independent uniform exponent draws -- the one whose fused
                   keep scores are most diverse on the calibration inputs,
                   since saturated draws leave every candidate on one score
                   level -- and then the keep-logit biases.
"""

import json
from dataclasses import replace
from pathlib import Path

import numpy as np

from .params import (BlockParams, FfnParams, HeatViTParams, MhsaParams, PatchParams,
                     SelectorHeadWeightParams, SelectorLocalParams, SelectorParams,
                     SelectorScoreParams)

BASE_SEED = 20260815
STREAM_STRIDE = 1000003
WORKLOAD_SEED = {
    "block": BASE_SEED + 0 * STREAM_STRIDE,
    "full": BASE_SEED + 1 * STREAM_STRIDE,
    "selector": BASE_SEED + 2 * STREAM_STRIDE,
    "pruned": BASE_SEED + 3 * STREAM_STRIDE,
}
WORKLOAD_BATCH = {"block": 1, "full": 1, "selector": 64, "pruned": 32, "throughput": 256}
TOKEN_TARGETS = (88, 45, 32)
SELECTOR_KEEP_FRACTION = 0.45
EXP_RANGE = (-12, -4)
CALIBRATION_FILE = Path(__file__).resolve().parent / "data" / "calibration.json"

_M64 = (1 << 64) - 1
_PHI = np.uint64(0x9E3779B97F4A7C15)


def _mix(z):
    """splitmix64 finaliser on a uint64 numpy array (wrapping arithmetic)."""
    z = z.astype(np.uint64, copy=True)
    with np.errstate(over="ignore"):
        z ^= z >> np.uint64(30)
        z *= np.uint64(0xBF58476D1CE4E5B9)
        z ^= z >> np.uint64(27)
        z *= np.uint64(0x94D049BB133111EB)
        z ^= z >> np.uint64(31)
    return z


def _fnv1a64(text):
    h = 0xCBF29CE484222325
    for b in text.encode():
        h = ((h ^ b) * 0x100000001B3) & _M64
    return h


def stream_key(seed, name):
    return int(_mix(np.array([(int(seed) ^ _fnv1a64(name)) & _M64], np.uint64))[0])


def words(seed, name, count, offset=0):
    """`count` uint64 words of stream (seed, name) starting at word `offset`."""
    idx = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(stream_key(seed, name)) + idx * _PHI
    return _mix(z)


def uniform_i8(seed, name, shape, offset=0):
    n = int(np.prod(shape))
    w = words(seed, name, (n + 7) // 8, offset)
    b = w.view(np.uint8)[:n].astype(np.int16) - 128
    return b.astype(np.int8).reshape(shape)


def _irwin_hall(seed, name, n):
    w = words(seed, name, 3 * n).reshape(n, 3)
    chunks = w.view(np.uint16).reshape(n, 12).astype(np.int64)
    return chunks.sum(axis=1) - 6 * 65535


def _round_div_pow2(num, shift):
    mag = (np.abs(num) + (1 << (shift - 1))) >> shift
    return np.where(num < 0, -mag, mag)


def normal_i8(seed, name, shape, sigma=40):
    n = int(np.prod(shape))
    v = _round_div_pow2(sigma * _irwin_hall(seed, name, n), 16)
    return np.clip(v, -127, 127).astype(np.int8).reshape(shape)


def normal_i32(seed, name, shape, sigma=1024):
    n = int(np.prod(shape))
    v = _round_div_pow2(sigma * _irwin_hall(seed, name, n), 16)
    return np.clip(v, -(1 << 31), (1 << 31) - 1).astype(np.int32).reshape(shape)


class _Exps:
    """Per-tensor scale exponents drawn uniformly from EXP_RANGE."""

    def __init__(self, seed, prefix):
        self.seed, self.prefix = seed, prefix

    def __call__(self, name):
        lo, hi = EXP_RANGE
        u = int(words(self.seed, f"{self.prefix}.exp.{name}", 1)[0])
        return lo + (((u >> 32) * (hi - lo + 1)) >> 32)


# --------------------------------------------------------------- builders

def make_patch(seed, tokens_exp=None):
    e = _Exps(seed, "patch")
    return PatchParams(
        patch_weight=normal_i8(seed, "patch.w", (768, 192)),
        patch_bias=normal_i32(seed, "patch.b", (192,)),
        cls=normal_i8(seed, "patch.cls", (192,)),
        pos=normal_i8(seed, "patch.pos", (197, 192)),
        image_scale_exp=e("image"), weight_scale_exp=e("weight"),
        activation_scale_exp=e("activation"),
        tokens_scale_exp=e("tokens") if tokens_exp is None else tokens_exp,
        cls_scale_exp=e("cls"), pos_scale_exp=e("pos"),
    )


def make_block(seed, index, x_exp):
    p = f"block{index}"
    e = _Exps(seed, p)
    qkv = e("qkv_out")
    mhsa = MhsaParams(
        ln_gamma=normal_i8(seed, f"{p}.ln1.gamma", (192,)),
        ln_beta=normal_i8(seed, f"{p}.ln1.beta", (192,)),
        wqkv=normal_i8(seed, f"{p}.wqkv", (192, 576)),
        bqkv=normal_i32(seed, f"{p}.bqkv", (576,)),
        wproj=normal_i8(seed, f"{p}.wproj", (192, 192)),
        bproj=normal_i32(seed, f"{p}.bproj", (192,)),
        x_scale_exp=x_exp, gamma1_scale_exp=e("gamma1"), beta1_scale_exp=e("beta1"),
        ln1_out_scale_exp=e("ln1_out"), wqkv_scale_exp=e("wqkv"), qkv_out_scale_exp=qkv,
        score_scale_exp=2 * qkv - 3, prob_scale_exp=-8,
        context_out_scale_exp=e("context_out"), wproj_scale_exp=e("wproj"),
        msa_out_scale_exp=e("msa_out"),
    )
    ffn = FfnParams(
        ln_gamma=normal_i8(seed, f"{p}.ln2.gamma", (192,)),
        ln_beta=normal_i8(seed, f"{p}.ln2.beta", (192,)),
        w1=normal_i8(seed, f"{p}.w1", (192, 768)),
        b1=normal_i32(seed, f"{p}.b1", (768,)),
        w2=normal_i8(seed, f"{p}.w2", (768, 192)),
        b2=normal_i32(seed, f"{p}.b2", (192,)),
        x_scale_exp=e("y"), gamma2_scale_exp=e("gamma2"), beta2_scale_exp=e("beta2"),
        ln2_out_scale_exp=e("ln2_out"), w1_scale_exp=e("w1"),
        hidden_out_scale_exp=e("hidden_out"), w2_scale_exp=e("w2"),
        ffn_out_scale_exp=e("ffn_out"), out_scale_exp=e("out"),
    )
    return BlockParams(mhsa=mhsa, ffn=ffn)


def make_selector(seed, index, in_exp, keep_bias=0, exp_draw=0):
    """Selector `index` with the keep-logit biases b3[h][1] set to `keep_bias`
    (one int for every head, or three per-head ints); b3[h][0] keeps its
    drawn value.  `exp_draw` selects one of several independent uniform
    draws of the selector's scale exponents (draw 0 is the default)."""
    p = f"selector{index}"
    e = _Exps(seed, p if exp_draw == 0 else f"{p}.draw{exp_draw}")
    local_out = e("local_out")
    b3 = normal_i32(seed, f"{p}.score.b3", (3, 2)).copy()
    b3[:, 1] = np.broadcast_to(np.asarray(keep_bias, np.int64), (3,))
    return SelectorParams(
        local=SelectorLocalParams(w=normal_i8(seed, f"{p}.local.w", (3, 64, 32)),
                                  b=normal_i32(seed, f"{p}.local.b", (3, 32))),
        score=SelectorScoreParams(
            w1=normal_i8(seed, f"{p}.score.w1", (3, 64, 32)),
            b1=normal_i32(seed, f"{p}.score.b1", (3, 32)),
            w2=normal_i8(seed, f"{p}.score.w2", (3, 32, 16)),
            b2=normal_i32(seed, f"{p}.score.b2", (3, 16)),
            w3=normal_i8(seed, f"{p}.score.w3", (3, 16, 2)),
            b3=b3),
        head_weight=SelectorHeadWeightParams(
            w1=normal_i8(seed, f"{p}.hw.w1", (3, 3)),
            b1=normal_i32(seed, f"{p}.hw.b1", (3,)),
            w2=normal_i8(seed, f"{p}.hw.w2", (3, 3)),
            b2=normal_i32(seed, f"{p}.hw.b2", (3,))),
        in_scale_exp=in_exp, local_w_scale_exp=e("local_w"), local_out_scale_exp=local_out,
        concat_out_scale_exp=local_out, score_w1_scale_exp=e("score_w1"),
        score_w2_scale_exp=e("score_w2"), score_w3_scale_exp=e("score_w3"),
        h1_out_scale_exp=e("h1_out"), h2_out_scale_exp=e("h2_out"),
        logits_out_scale_exp=e("logits_out"), stats_out_scale_exp=in_exp,
        hw_w1_scale_exp=e("hw_w1"), hw_hidden_out_scale_exp=e("hw_hidden_out"),
        hw_w2_scale_exp=e("hw_w2"),
    )


def make_model(seed, selector_blocks=(4, 7, 10), keep_biases=(0, 0, 0), exp_draws=(0, 0, 0)):
    """Full model; keep_biases[s] is selector s's keep bias (int or 3 ints)
    and exp_draws[s] its exponent draw."""
    patch = make_patch(seed)
    blocks, selectors = [], []
    x_exp = patch.tokens_scale_exp
    for b in range(1, 13):
        if b in selector_blocks:
            s = len(selectors)
            selectors.append(make_selector(seed, s + 1, x_exp, keep_biases[s], exp_draws[s]))
        blk = make_block(seed, b, x_exp)
        blocks.append(blk)
        x_exp = blk.ffn.out_scale_exp
    e = _Exps(seed, "head")
    return HeatViTParams(
        patch=patch, blocks=tuple(blocks), selectors=tuple(selectors),
        final_gamma=normal_i8(seed, "final.gamma", (192,)),
        final_beta=normal_i8(seed, "final.beta", (192,)),
        head_w=normal_i8(seed, "head.w", (192, 1000)),
        head_b=normal_i32(seed, "head.b", (1000,)),
        final_gamma_scale_exp=e("final_gamma"), final_beta_scale_exp=e("final_beta"),
        final_ln_out_scale_exp=e("final_ln_out"), head_w_scale_exp=e("head_w"),
        selector_blocks=tuple(selector_blocks),
    )


def images(seed, count, start=0):
    """`count` NHWC 224x224x3 int8 images; image i has its own stream."""
    return np.stack([uniform_i8(seed, f"image{start + i}", (224, 224, 3))
                     for i in range(count)])


def token_batch(seed, count):
    return np.stack([uniform_i8(seed, f"tokens{i}", (197, 192)) for i in range(count)])


# --------------------------------------------------------------- workloads

def load_calibration():
    if CALIBRATION_FILE.exists():
        return json.loads(CALIBRATION_FILE.read_text())
    return {}


def block_workload():
    seed = WORKLOAD_SEED["block"]
    x_exp = _Exps(seed, "input")("x")
    return uniform_i8(seed, "x", (197, 192)), make_block(seed, 1, x_exp)


def full_workload():
    seed = WORKLOAD_SEED["full"]
    return images(seed, 1), make_model(seed, selector_blocks=())


def selector_workload(keep_bias=None, exp_draw=None):
    seed = WORKLOAD_SEED["selector"]
    cal = load_calibration().get("selector", {})
    keep_bias = cal.get("keep_bias", 0) if keep_bias is None else keep_bias
    exp_draw = cal.get("exp_draw", 0) if exp_draw is None else exp_draw
    in_exp = _Exps(seed, "input")("tokens")
    return token_batch(seed, WORKLOAD_BATCH["selector"]), make_selector(seed, 1, in_exp,
                                                                        keep_bias, exp_draw)


def pruned_params(keep_biases=None, exp_draws=None):
    seed = WORKLOAD_SEED["pruned"]
    cal = load_calibration().get("pruned", {})
    keep_biases = cal.get("keep_biases", (0, 0, 0)) if keep_biases is None else keep_biases
    exp_draws = cal.get("exp_draws", (0, 0, 0)) if exp_draws is None else exp_draws
    return make_model(seed, (4, 7, 10), tuple(keep_biases), tuple(exp_draws))


def unpruned_control(params):
    """The same weights with every selector removed."""
    return replace(params, selectors=(), selector_blocks=())


def pruned_workload(count=None):
    seed = WORKLOAD_SEED["pruned"]
    count = WORKLOAD_BATCH["pruned"] if count is None else count
    return images(seed, count), pruned_params()


def throughput_workload(count=None):
    seed = WORKLOAD_SEED["pruned"]
    count = WORKLOAD_BATCH["throughput"] if count is None else count
    return images(seed, count), pruned_params()
