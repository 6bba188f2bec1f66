"""Memory-image writer for the descriptor front end's tests: the weight
region of a HeatViTParams at the offsets a compiled ROM names, and an e2e
vector directory in the layout tools/generate_e2e_vectors.py writes
(.mem files of 64-bit little-endian beats, manifest.json, checkpoints/).
The weight region is pinned against the reference's serialize_weights by
SHA-256 (tests/golden/e2e.json)."""

import json
from pathlib import Path

import numpy as np


def mem_text(raw):
    raw = bytes(raw) + b"\x00" * ((-len(raw)) % 8)
    return "".join(f"{int.from_bytes(raw[i:i + 8], 'little'):016x}\n" for i in range(0, len(raw), 8))


def weight_region(params, sched):
    """Bytes of the weight region: int8 tensors row-major ([K][N] for GEMM
    weights, [3][K][N] per selector head), int32 biases little-endian."""
    buf = bytearray(int(sched.weight_bytes))

    def put(off, arr, dtype):
        b = np.ascontiguousarray(np.asarray(arr), dtype=dtype).tobytes()
        buf[off:off + len(b)] = b

    p = params.patch
    put(sched.patch_w, p.patch_weight, np.int8)
    put(sched.patch_b, p.patch_bias, "<i4")
    put(sched.cls, p.cls, np.int8)
    put(sched.pos, p.pos, np.int8)
    for o, blk in zip(sched.blocks, params.blocks):
        m, f = blk.mhsa, blk.ffn
        for name, arr, dt in (("gamma1", m.ln_gamma, np.int8), ("beta1", m.ln_beta, np.int8),
                              ("wqkv", m.wqkv, np.int8), ("bqkv", m.bqkv, "<i4"),
                              ("wproj", m.wproj, np.int8), ("bproj", m.bproj, "<i4"),
                              ("gamma2", f.ln_gamma, np.int8), ("beta2", f.ln_beta, np.int8),
                              ("w1", f.w1, np.int8), ("b1", f.b1, "<i4"),
                              ("w2", f.w2, np.int8), ("b2", f.b2, "<i4")):
            put(getattr(o, name), arr, dt)
    for o, sp in zip(sched.selectors, params.selectors):
        for name, arr, dt in (("local_w", sp.local.w, np.int8), ("local_b", sp.local.b, "<i4"),
                              ("score_w1", sp.score.w1, np.int8), ("score_b1", sp.score.b1, "<i4"),
                              ("score_w2", sp.score.w2, np.int8), ("score_b2", sp.score.b2, "<i4"),
                              ("score_w3", sp.score.w3, np.int8), ("score_b3", sp.score.b3, "<i4"),
                              ("hw_w1", sp.head_weight.w1, np.int8),
                              ("hw_b1", sp.head_weight.b1, "<i4"),
                              ("hw_w2", sp.head_weight.w2, np.int8),
                              ("hw_b2", sp.head_weight.b2, "<i4")):
            put(getattr(o, name), arr, dt)
    put(sched.final_gamma, params.final_gamma, np.int8)
    put(sched.final_beta, params.final_beta, np.int8)
    put(sched.head_w, params.head_w, np.int8)
    put(sched.head_b, params.head_b, "<i4")
    return bytes(buf)


def vector_dir(root, image, weights, checkpoints, logits):
    """An e2e vector directory for one image: checkpoints {name: bytes}."""
    d = Path(root)
    (d / "checkpoints").mkdir(parents=True, exist_ok=True)
    image = np.ascontiguousarray(image, np.int8).tobytes()
    (d / "input.mem").write_text(mem_text(image))
    (d / "weights.mem").write_text(mem_text(weights))
    entries = []
    for name, raw in list(checkpoints.items()) + [("logits", np.asarray(logits, "<i4").tobytes())]:
        (d / "checkpoints" / f"{name}.mem").write_text(mem_text(raw))
        entries.append({"name": name, "bytes": len(raw)})
    manifest = {"regions": {"input": {"valid_bytes": len(image)},
                            "weight": {"valid_bytes": len(weights)}},
                "checkpoints": entries}
    (d / "manifest.json").write_text(json.dumps(manifest, indent=1))
    return d
