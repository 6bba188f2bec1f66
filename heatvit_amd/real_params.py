"""Golden parameters from real (float) weights and a per-tensor scale table.

  golden_params_from_real(floats, table, selector_payload)
      p2_export_weights.golden_params_from_real
      (tools/p2/p2_export_weights.py:110-243)
  merge_selector_scales(table, payload)   the same file, :96-107
  quantize_int8 / quantize_bias           p2_quantize.py:102-109

`floats` maps the reference's tensor names (p2_quantize.to_heatvit_tensors,
tools/p2/p2_quantize.py:65-92: GEMM weights as [K][N], e.g. "b3_wqkv"
[192][576], biases "b3_bqkv" [576], "patch_w" [768][192], "head_w"
[192][1000], ...) to float tensors; the selector payload carries the
already-integer trained selectors ({"selectors": [{"local_w": [3][64][32],
"local_b": [3][32], "score_w1" ... "hw_b2": [3]}] * 3}, plus optionally
"weight_exps"/"sel_acts" per selector).  The result is the HeatViTParams the
GPU forward takes: with HeatViTModel.infer_float_batch it replaces the
reference's per-image accuracy engine (p2_sim.forward_image / p2_sim_ivit.
forward_image_cfg in its contract configuration) with pruning batched on
the device.
"""

import numpy as np

from .params import (BlockParams, FfnParams, HeatViTParams, MhsaParams, PatchParams,
                     SelectorHeadWeightParams, SelectorLocalParams, SelectorParams,
                     SelectorScoreParams)

PROB_SCALE_EXP = -8


def _float(t):
    """float64 tensors stay float64; everything else is taken as float32
    (the dtype of the reference's state-dict tensors)."""
    if hasattr(t, "detach"):
        t = t.detach().cpu().numpy()
    a = np.asarray(t)
    return a if a.dtype == np.float64 else a.astype(np.float32)


def _steps(t, exp):
    """round_half_even(t / 2^exp) in the tensor's precision, as torch.round
    of the reference's quotient."""
    a = _float(t)
    return np.rint(a / a.dtype.type(2.0 ** exp))


def quantize_int8(t, exp):
    return np.clip(_steps(t, exp), -128, 127).astype(np.int8)


def quantize_bias(t, exp):
    """int32 biases; quotients at or beyond 2^31 saturate to 2^31 - 1 (the
    reference's float32 clamp bound rounds to 2^31 there, whose int32 cast
    is undefined)."""
    q = _steps(t, exp).astype(np.float64)
    return np.clip(q, -(2.0 ** 31), 2.0 ** 31 - 1).astype(np.int32)


def block_input_exp(table, n):
    """Exponent of block n's input rows: the patch tokens, then block n-1's
    output."""
    return table.activation_exp("act_tokens" if n == 1 else f"b{n - 1}_out")


def selector_input_exp(table, s):
    """Selector s (1..3) sits before block 3s+1 and reads block 3s's output."""
    return table.activation_exp(f"b{3 * s}_out")


def merge_selector_scales(table, payload):
    """Copies the selector exponents a trained-selector payload carries into
    the table (idempotent) and validates the result."""
    if "weight_exps" not in payload:
        return table
    for s in (1, 2, 3):
        for name, exp in payload["weight_exps"][str(s)].items():
            table.weights[f"s{s}_{name}"] = int(exp)
        for name, exp in payload["sel_acts"][str(s)].items():
            table.activations[f"s{s}_{name}"] = int(exp)
    table.validate()
    return table


def _ints(t, dtype):
    if hasattr(t, "detach"):
        t = t.detach().cpu().numpy()
    return np.asarray(t).astype(dtype)


def _selector(sel, table, s):
    w, a = table.weight_exp, table.activation_exp
    i8 = lambda k: _ints(sel[k], np.int8)  # noqa: E731
    i32 = lambda k: _ints(sel[k], np.int32)  # noqa: E731
    return SelectorParams(
        local=SelectorLocalParams(w=i8("local_w"), b=i32("local_b")),
        score=SelectorScoreParams(w1=i8("score_w1"), b1=i32("score_b1"), w2=i8("score_w2"),
                                  b2=i32("score_b2"), w3=i8("score_w3"), b3=i32("score_b3")),
        head_weight=SelectorHeadWeightParams(w1=i8("hw_w1"), b1=i32("hw_b1"), w2=i8("hw_w2"),
                                             b2=i32("hw_b2")),
        in_scale_exp=selector_input_exp(table, s),
        local_w_scale_exp=w(f"s{s}_local_w"),
        local_out_scale_exp=a(f"s{s}_local_out"),
        concat_out_scale_exp=a(f"s{s}_concat_out"),
        score_w1_scale_exp=w(f"s{s}_score_w1"),
        score_w2_scale_exp=w(f"s{s}_score_w2"),
        score_w3_scale_exp=w(f"s{s}_score_w3"),
        h1_out_scale_exp=a(f"s{s}_h1_out"),
        h2_out_scale_exp=a(f"s{s}_h2_out"),
        logits_out_scale_exp=a(f"s{s}_logits_out"),
        stats_out_scale_exp=a(f"s{s}_stats_out"),
        hw_w1_scale_exp=w(f"s{s}_hw_w1"),
        hw_hidden_out_scale_exp=a(f"s{s}_hw_hidden_out"),
        hw_w2_scale_exp=w(f"s{s}_hw_w2"))


def _block(floats, table, n):
    w, a = table.weight_exp, table.activation_exp
    q8 = lambda k: quantize_int8(floats[f"b{n}_{k}"], w(f"b{n}_{k}"))  # noqa: E731
    # each bias sits at the exponent of its GEMM's accumulator
    qb = lambda k, act, wt: quantize_bias(floats[f"b{n}_{k}"],  # noqa: E731
                                          a(f"b{n}_{act}") + w(f"b{n}_{wt}"))
    qkv = a(f"b{n}_qkv_out")
    mhsa = MhsaParams(
        ln_gamma=q8("gamma1"), ln_beta=q8("beta1"), wqkv=q8("wqkv"),
        bqkv=qb("bqkv", "ln1_out", "wqkv"), wproj=q8("wproj"),
        bproj=qb("bproj", "context_out", "wproj"),
        x_scale_exp=block_input_exp(table, n), gamma1_scale_exp=w(f"b{n}_gamma1"),
        beta1_scale_exp=w(f"b{n}_beta1"), ln1_out_scale_exp=a(f"b{n}_ln1_out"),
        wqkv_scale_exp=w(f"b{n}_wqkv"), qkv_out_scale_exp=qkv, score_scale_exp=2 * qkv - 3,
        prob_scale_exp=PROB_SCALE_EXP, context_out_scale_exp=a(f"b{n}_context_out"),
        wproj_scale_exp=w(f"b{n}_wproj"), msa_out_scale_exp=a(f"b{n}_msa_out"))
    ffn = FfnParams(
        ln_gamma=q8("gamma2"), ln_beta=q8("beta2"), w1=q8("w1"), b1=qb("b1", "ln2_out", "w1"),
        w2=q8("w2"), b2=qb("b2", "hidden", "w2"),
        x_scale_exp=a(f"b{n}_y"), gamma2_scale_exp=w(f"b{n}_gamma2"),
        beta2_scale_exp=w(f"b{n}_beta2"), ln2_out_scale_exp=a(f"b{n}_ln2_out"),
        w1_scale_exp=w(f"b{n}_w1"), hidden_out_scale_exp=a(f"b{n}_hidden"),
        w2_scale_exp=w(f"b{n}_w2"), ffn_out_scale_exp=a(f"b{n}_ffn_out"),
        out_scale_exp=a(f"b{n}_out"))
    return BlockParams(mhsa=mhsa, ffn=ffn)


def golden_params_from_real(floats, table, selector_payload):
    """HeatViTParams (selectors before blocks 4, 7, 10) from float tensors,
    the scale table and the trained selectors."""
    w, a = table.weight_exp, table.activation_exp
    q8 = lambda k: quantize_int8(floats[k], w(k))  # noqa: E731
    patch = PatchParams(
        patch_weight=q8("patch_w"),
        patch_bias=quantize_bias(floats["patch_b"], a("input") + w("patch_w")),
        cls=q8("cls"), pos=q8("pos"),
        image_scale_exp=a("input"), weight_scale_exp=w("patch_w"),
        activation_scale_exp=a("act_patch_embed"), tokens_scale_exp=a("act_tokens"),
        cls_scale_exp=w("cls"), pos_scale_exp=w("pos"))
    blocks = tuple(_block(floats, table, n) for n in range(1, 13))
    selectors = tuple(_selector(selector_payload["selectors"][s - 1], table, s)
                      for s in (1, 2, 3))
    return HeatViTParams(
        patch=patch, blocks=blocks, selectors=selectors,
        final_gamma=q8("final_gamma"), final_beta=q8("final_beta"), head_w=q8("head_w"),
        head_b=quantize_bias(floats["head_b"], a("final_ln_out") + w("head_w")),
        final_gamma_scale_exp=w("final_gamma"), final_beta_scale_exp=w("final_beta"),
        final_ln_out_scale_exp=a("final_ln_out"), head_w_scale_exp=w("head_w"))
