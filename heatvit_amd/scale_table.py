"""Per-tensor scale exponents of a real-weight model.

The reference keeps one JSON table of power-of-two exponents per weight and
per activation tensor (tools/p2/scale_table.py:1-126): PTQ calibration
writes it, and the golden parameters, the descriptor scale fields and the
accuracy engine read it.  This module keeps the same JSON document and
tensor names, so a table written for the reference loads here unchanged:

    {"weights": {"patch_w": -9, "b1_wqkv": -8, ...},
     "activations": {"input": -5, "b1_ln1_out": -4, ...}}

Bias exponents are derived (activation + weight) and fixed internal
exponents (Q8.16 = -16, attention probabilities -8, selector Q0.16 -16,
attention score 2*qkv - 3, logits -14) are not stored.
"""

import json
from pathlib import Path

EXP_MIN, EXP_MAX = -32, 31

BLOCK_WEIGHTS = ("wqkv", "wproj", "gamma1", "beta1", "w1", "w2", "gamma2", "beta2")
SELECTOR_WEIGHTS = ("local_w", "score_w1", "score_w2", "score_w3", "hw_w1", "hw_w2")
BLOCK_ACTIVATIONS = ("ln1_out", "qkv_out", "context_out", "msa_out", "y", "ln2_out", "hidden",
                     "ffn_out", "out")
SELECTOR_ACTIVATIONS = ("local_out", "concat_out", "h1_out", "h2_out", "logits_out",
                        "stats_out", "hw_hidden_out")

WEIGHT_NAMES = tuple(
    ["patch_w", "cls", "pos"]
    + [f"b{n}_{w}" for n in range(1, 13) for w in BLOCK_WEIGHTS]
    + [f"s{s}_{w}" for s in range(1, 4) for w in SELECTOR_WEIGHTS]
    + ["final_gamma", "final_beta", "head_w"])

ACTIVATION_NAMES = tuple(
    ["input", "act_patch_matrix", "act_patch_embed", "act_tokens"]
    + [f"b{n}_{a}" for n in range(1, 13) for a in BLOCK_ACTIVATIONS]
    + [f"s{s}_{a}" for s in range(1, 4) for a in SELECTOR_ACTIVATIONS]
    + ["final_ln_out"])


def check_exp(name, value):
    """The exponent itself; ValueError unless it is an int in [-32, 31]."""
    if isinstance(value, bool) or not isinstance(value, int):
        raise ValueError(f"scale_exp {name} must be an integer, got {value!r}")
    if not EXP_MIN <= value <= EXP_MAX:
        raise ValueError(f"scale_exp {name}={value} outside [{EXP_MIN}, {EXP_MAX}]")
    return value


class ScaleTable:
    """Weight and activation exponents by tensor name."""

    def __init__(self, weights=None, activations=None):
        self.weights = dict(weights or {})
        self.activations = dict(activations or {})

    @classmethod
    def load(cls, path):
        doc = json.loads(Path(path).read_text(encoding="utf-8"))
        if not isinstance(doc, dict):
            raise ValueError("scale table root must be an object")
        return cls(doc.get("weights"), doc.get("activations"))

    def save(self, path):
        doc = {"weights": dict(sorted(self.weights.items())),
               "activations": dict(sorted(self.activations.items()))}
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(doc, indent=2) + "\n", encoding="utf-8", newline="\n")

    def validate(self):
        """Every schema name present, no unknown name, every value in range."""
        for kind, table, names in (("weight", self.weights, WEIGHT_NAMES),
                                   ("activation", self.activations, ACTIVATION_NAMES)):
            missing = [n for n in names if n not in table]
            if missing:
                raise ValueError(f"missing {kind} scale_exp: {missing[0]}")
            known = set(names)
            for name, value in table.items():
                if name not in known:
                    raise ValueError(f"unknown {kind} tensor: {name}")
                check_exp(name, value)
        return self

    def weight_exp(self, name):
        try:
            return self.weights[name]
        except KeyError:
            raise KeyError(f"no scale_exp for weight tensor {name}") from None

    def activation_exp(self, name):
        try:
            return self.activations[name]
        except KeyError:
            raise KeyError(f"no scale_exp for activation tensor {name}") from None

    @classmethod
    def from_params(cls, params):
        """The table whose golden_params_from_real exponents are those of
        `params` (a HeatViTParams with three selectors before blocks 4/7/10
        and the fixed derived exponents)."""
        p = params.patch
        w = {"patch_w": p.weight_scale_exp, "cls": p.cls_scale_exp, "pos": p.pos_scale_exp,
             "final_gamma": params.final_gamma_scale_exp,
             "final_beta": params.final_beta_scale_exp, "head_w": params.head_w_scale_exp}
        a = {"input": p.image_scale_exp, "act_patch_matrix": p.image_scale_exp,
             "act_patch_embed": p.activation_scale_exp, "act_tokens": p.tokens_scale_exp,
             "final_ln_out": params.final_ln_out_scale_exp}
        for n, blk in enumerate(params.blocks, 1):
            m, f = blk.mhsa, blk.ffn
            w.update({f"b{n}_wqkv": m.wqkv_scale_exp, f"b{n}_wproj": m.wproj_scale_exp,
                      f"b{n}_gamma1": m.gamma1_scale_exp, f"b{n}_beta1": m.beta1_scale_exp,
                      f"b{n}_w1": f.w1_scale_exp, f"b{n}_w2": f.w2_scale_exp,
                      f"b{n}_gamma2": f.gamma2_scale_exp, f"b{n}_beta2": f.beta2_scale_exp})
            a.update({f"b{n}_ln1_out": m.ln1_out_scale_exp, f"b{n}_qkv_out": m.qkv_out_scale_exp,
                      f"b{n}_context_out": m.context_out_scale_exp,
                      f"b{n}_msa_out": m.msa_out_scale_exp, f"b{n}_y": f.x_scale_exp,
                      f"b{n}_ln2_out": f.ln2_out_scale_exp,
                      f"b{n}_hidden": f.hidden_out_scale_exp,
                      f"b{n}_ffn_out": f.ffn_out_scale_exp, f"b{n}_out": f.out_scale_exp})
        for s, sp in enumerate(params.selectors, 1):
            w.update({f"s{s}_local_w": sp.local_w_scale_exp,
                      f"s{s}_score_w1": sp.score_w1_scale_exp,
                      f"s{s}_score_w2": sp.score_w2_scale_exp,
                      f"s{s}_score_w3": sp.score_w3_scale_exp,
                      f"s{s}_hw_w1": sp.hw_w1_scale_exp, f"s{s}_hw_w2": sp.hw_w2_scale_exp})
            a.update({f"s{s}_local_out": sp.local_out_scale_exp,
                      f"s{s}_concat_out": sp.concat_out_scale_exp,
                      f"s{s}_h1_out": sp.h1_out_scale_exp, f"s{s}_h2_out": sp.h2_out_scale_exp,
                      f"s{s}_logits_out": sp.logits_out_scale_exp,
                      f"s{s}_stats_out": sp.stats_out_scale_exp,
                      f"s{s}_hw_hidden_out": sp.hw_hidden_out_scale_exp})
        return cls(w, a)
