"""Deterministic stand-in for a real-weight model: float tensors in the
reference's real-weight layout (p2_quantize.to_heatvit_tensors), a scale
table, an integer selector payload and float CHW images.

No trained DeiT-T checkpoint or scale table ships with the reference, so the
floats are built around this build's calibrated synthetic model: every
integer q at exponent e becomes (q + u) * 2^e with u uniform in (-1/2, 1/2),
except for planted exact ties (u = +-1/2, resolved to even by the
quantiser) and out-of-range values (|q + u| > 128, clamped).  The table is
the synthetic model's own exponents, so the pipeline keeps the calibrated
pruning behaviour.
"""

import hashlib

import numpy as np

from heatvit_amd import synth
from heatvit_amd.scale_table import ScaleTable

SEED = 20251130


def _perturb(rng, q, exp, ties=0.02, wild=0.002, dtype=np.float32):
    q = np.asarray(q, np.float64)
    u = rng.uniform(-0.49, 0.49, q.shape)
    r = rng.random(q.shape)
    u = np.where(r < ties, np.where(rng.random(q.shape) < 0.5, -0.5, 0.5), u)
    big = (r >= ties) & (r < ties + wild)
    u = np.where(big, np.sign(q + 0.1) * rng.uniform(1.0, 64.0, q.shape), u)
    return ((q + u) * 2.0 ** exp).astype(dtype)


def make(images=4):
    """Returns (floats dict, ScaleTable, selector payload, float images
    [B][3][224][224], the synthetic HeatViTParams they were built from)."""
    params = synth.pruned_params()
    table = ScaleTable.from_params(params).validate()
    rng = np.random.default_rng(SEED)
    w, a = table.weights, table.activations
    f = {}
    p = params.patch
    f["patch_w"] = _perturb(rng, p.patch_weight, w["patch_w"])
    f["patch_b"] = _perturb(rng, p.patch_bias, a["input"] + w["patch_w"], wild=0)
    f["cls"] = _perturb(rng, p.cls, w["cls"])
    f["pos"] = _perturb(rng, p.pos, w["pos"])
    for n, blk in enumerate(params.blocks, 1):
        m, ff = blk.mhsa, blk.ffn
        for key, q in (("gamma1", m.ln_gamma), ("beta1", m.ln_beta), ("wqkv", m.wqkv),
                       ("wproj", m.wproj), ("gamma2", ff.ln_gamma), ("beta2", ff.ln_beta),
                       ("w1", ff.w1), ("w2", ff.w2)):
            f[f"b{n}_{key}"] = _perturb(rng, q, w[f"b{n}_{key}"])
        for key, q, act, wt in (("bqkv", m.bqkv, "ln1_out", "wqkv"),
                                ("bproj", m.bproj, "context_out", "wproj"),
                                ("b1", ff.b1, "ln2_out", "w1"), ("b2", ff.b2, "hidden", "w2")):
            f[f"b{n}_{key}"] = _perturb(rng, q, a[f"b{n}_{act}"] + w[f"b{n}_{wt}"], wild=0)
    f["final_gamma"] = _perturb(rng, params.final_gamma, w["final_gamma"])
    f["final_beta"] = _perturb(rng, params.final_beta, w["final_beta"])
    f["head_w"] = _perturb(rng, params.head_w, w["head_w"])
    f["head_b"] = _perturb(rng, params.head_b, a["final_ln_out"] + w["head_w"], wild=0)
    payload = {"selectors": []}
    for sp in params.selectors:
        payload["selectors"].append({
            "local_w": np.asarray(sp.local.w), "local_b": np.asarray(sp.local.b),
            "score_w1": np.asarray(sp.score.w1), "score_b1": np.asarray(sp.score.b1),
            "score_w2": np.asarray(sp.score.w2), "score_b2": np.asarray(sp.score.b2),
            "score_w3": np.asarray(sp.score.w3), "score_b3": np.asarray(sp.score.b3),
            "hw_w1": np.asarray(sp.head_weight.w1), "hw_b1": np.asarray(sp.head_weight.b1),
            "hw_w2": np.asarray(sp.head_weight.w2), "hw_b2": np.asarray(sp.head_weight.b2)})
    q_imgs = np.asarray(synth.images(SEED, images)).reshape(images, 224, 224, 3)
    chw = np.ascontiguousarray(q_imgs.transpose(0, 3, 1, 2))
    imgs = _perturb(rng, chw, a["input"], wild=0.001)
    return f, table, payload, imgs, params


# int32 parameter tensors by field name (biases); every other tensor is int8
INT32_FIELDS = {"patch_bias", "bqkv", "bproj", "b1", "b2", "b3", "b", "head_b"}


def digest(arr, dtype):
    return hashlib.sha256(np.ascontiguousarray(np.asarray(arr), dtype=dtype).tobytes()).hexdigest()


def param_digests(p):
    """{field path: SHA-256 of the tensor, or the integer} over a
    HeatViTParams-shaped dataclass tree (the reference's or this build's)."""
    out = {}

    def walk(obj, path):
        for name in obj.__dataclass_fields__:
            v = getattr(obj, name)
            key = f"{path}.{name}" if path else name
            if hasattr(v, "__dataclass_fields__"):
                walk(v, key)
            elif name in ("blocks", "selectors"):
                for i, item in enumerate(v):
                    walk(item, f"{key}[{i}]")
            elif name == "selector_blocks":
                out[key] = [int(b) for b in v]
            elif isinstance(v, (int, np.integer)) and not isinstance(v, bool):
                out[key] = int(v)
            else:
                out[key] = digest(v, np.int32 if name in INT32_FIELDS else np.int8)
    walk(p, "")
    return out
