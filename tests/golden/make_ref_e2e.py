"""Writes tests/golden/ref_e2e.json: the reference's own seeded synthetic
end-to-end model (verification/heatvit_ref/weights.py build_params on the
image of tools/generate_e2e_vectors.det_image, seed 20260815) and its
golden forward (model.HeatViTModel.infer), by running the reference's
Python in the development container.

The reference commits only the token counts of this model
(sim/generated/e2e_tb_config.sv:18-20); this fixture adds what its golden
model computes: a SHA-256 per parameter tensor, the calibration summary,
the 1000 logits and a SHA-256 per checkpoint.  Run (a few minutes):
    python tests/golden/make_ref_e2e.py
"""

import hashlib
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REFERENCE = Path(os.environ.get("HEATVIT_REFERENCE", "/root/reference"))
OUT = Path(__file__).resolve().parent / "ref_e2e.json"
sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

from golden_io import param_digests  # noqa: E402


def digest(arr, dtype):
    return hashlib.sha256(np.ascontiguousarray(np.asarray(arr), dtype=dtype).tobytes()).hexdigest()


def main():
    sys.path.insert(0, str(REFERENCE))
    from tools.generate_e2e_vectors import det_image
    from verification.heatvit_ref.model import HeatViTModel
    from verification.heatvit_ref.weights import SEED, build_params

    image = det_image(SEED)
    t0 = time.time()
    params, summary, counts = build_params(image)
    t_build = time.time() - t0
    t0 = time.time()
    res = HeatViTModel().infer(image, params)
    t_infer = time.time() - t0
    cks = {k: digest(v, "<i4" if k == "logits" else np.int8)
           for k, v in res.checkpoints.items()}
    rows = {k: len(v) for k, v in res.checkpoints.items() if k != "logits"}
    doc = {
        "seed": SEED,
        "image_sha256": digest(image, np.int8),
        "token_counts": list(counts),
        "summary": list(summary),
        "selector_summary": [dict(s) for s in res.selector_summary],
        "params": param_digests(params),
        "logits": [int(v) for v in res.logits],
        "output_scale_exp": res.output_scale_exp,
        "checkpoints": cks,
        "rows": rows,
        "golden_seconds": {"build_params": round(t_build, 1), "infer": round(t_infer, 1)},
    }
    OUT.write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {OUT}: counts {counts}, build {t_build:.0f} s, infer {t_infer:.0f} s")


if __name__ == "__main__":
    main()
