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
