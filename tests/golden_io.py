"""Loaders for the composite-stage golden fixtures (tests/golden/*.json|npz),
written by tests/golden/make_golden.py from the reference's golden model."""

import hashlib
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

BLOCK_DTYPES = dict(ln1=np.int8, fused_qkv=np.int8, qkv=np.int8, score="<i4", prob=np.uint8,
                    context=np.int8, concat=np.int8, msa=np.int8, y=np.int8, ln2=np.int8,
                    hidden=np.int8, ffn_out=np.int8, z=np.int8)


def digest(arr, dtype):
    return hashlib.sha256(np.ascontiguousarray(np.asarray(arr), dtype=dtype).tobytes()).hexdigest()


def load(name):
    meta = json.loads((GOLDEN / f"{name}.json").read_text())
    arrays = dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))
    return meta, arrays


def available(name):
    return (GOLDEN / f"{name}.json").exists() and (GOLDEN / f"{name}.npz").exists()


def model_checkpoint_digests(cks):
    return {k: digest(v, "<i4" if k == "logits" else np.int8) for k, v in cks.items()}


def param_digests(p):
    """SHA-256 of every tensor of a HeatViTParams-shaped object (this
    package's or the reference's): int8 tensors as bytes, int32 biases
    little-endian, row-major; keys name the tensor."""
    out = {}
    i8, i32 = np.int8, "<i4"
    pp = p.patch
    for name, arr, dt in (("patch_weight", pp.patch_weight, i8), ("patch_bias", pp.patch_bias, i32),
                          ("cls", pp.cls, i8), ("pos", pp.pos, i8)):
        out[f"patch.{name}"] = digest(arr, dt)
    for b, blk in enumerate(p.blocks):
        m, f = blk.mhsa, blk.ffn
        for name, arr, dt in (("ln1_gamma", m.ln_gamma, i8), ("ln1_beta", m.ln_beta, i8),
                              ("wqkv", m.wqkv, i8), ("bqkv", m.bqkv, i32),
                              ("wproj", m.wproj, i8), ("bproj", m.bproj, i32),
                              ("ln2_gamma", f.ln_gamma, i8), ("ln2_beta", f.ln_beta, i8),
                              ("w1", f.w1, i8), ("b1", f.b1, i32), ("w2", f.w2, i8),
                              ("b2", f.b2, i32)):
            out[f"block{b + 1}.{name}"] = digest(arr, dt)
    for s, sp in enumerate(p.selectors):
        for name, arr, dt in (("local_w", sp.local.w, i8), ("local_b", sp.local.b, i32),
                              ("w1", sp.score.w1, i8), ("b1", sp.score.b1, i32),
                              ("w2", sp.score.w2, i8), ("b2", sp.score.b2, i32),
                              ("w3", sp.score.w3, i8), ("b3", sp.score.b3, i32),
                              ("hw_w1", sp.head_weight.w1, i8), ("hw_b1", sp.head_weight.b1, i32),
                              ("hw_w2", sp.head_weight.w2, i8), ("hw_b2", sp.head_weight.b2, i32)):
            out[f"selector{s + 1}.{name}"] = digest(arr, dt)
    for name, arr, dt in (("final_gamma", p.final_gamma, i8), ("final_beta", p.final_beta, i8),
                          ("head_w", p.head_w, i8), ("head_b", p.head_b, i32)):
        out[name] = digest(arr, dt)
    return out
