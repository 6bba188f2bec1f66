"""Writes tests/golden/real.json by running the reference's real-weight
tools on the deterministic real-weight stand-in of tests/real_weights.py:

  * p2_export_weights.golden_params_from_real (tools/p2/p2_export_weights.py:
    110-243) -> SHA-256 and exponents of every HeatViTParams field;
  * p2_export_weights.real_image_list (:246-251) -> the int8 images;
  * p2_sim.forward_image (tools/p2/p2_sim.py:527-...) with prune=True, the
    reference's per-image accuracy engine, over a QuantDeiT built by
    p2_quantize.build_model (tools/p2/p2_quantize.py:123-190) with the
    payload's selectors -> logits and token counts per image;
  * p2_sim_ivit.forward_batch_cfg (tools/p2/p2_sim_ivit.py:563-624) in its
    contract configuration (no pruning) -> logits per image.

Only the reference's public functions are called; the fixture holds digests
and outputs.  Run in the development container (the reference tree is not
present on GPU hosts):
    python tests/golden/make_real.py
"""

import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
REFERENCE = Path(os.environ.get("HEATVIT_REFERENCE", "/root/reference"))
OUT = Path(__file__).resolve().parent / "real.json"
sys.path[:0] = [str(ROOT), str(ROOT / "tests")]

import real_weights  # noqa: E402


def main():
    sys.path.insert(0, str(REFERENCE))
    from tools.p2 import p2_export_weights as pe
    from tools.p2 import p2_quantize as pq
    from tools.p2 import p2_sim, p2_sim_ivit
    from tools.p2.scale_table import ScaleTable

    floats, table, payload, imgs, _ = real_weights.make(4)
    t_floats = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in floats.items()}
    t_payload = {"selectors": [{k: torch.from_numpy(np.ascontiguousarray(v))
                                for k, v in sel.items()} for sel in payload["selectors"]]}
    ref_table = ScaleTable(table.weights, table.activations).validate()

    t0 = time.time()
    params = pe.golden_params_from_real(t_floats, ref_table, t_payload)
    fixture = {"seed": real_weights.SEED, "images": len(imgs),
               "table": {"weights": dict(sorted(table.weights.items())),
                         "activations": dict(sorted(table.activations.items()))},
               "params": real_weights.param_digests(params)}
    timgs = torch.from_numpy(imgs)
    fixture["image_sha256"] = [real_weights.digest(pe.real_image_list(timgs[i], ref_table),
                                                   np.int8)
                               for i in range(len(imgs))]

    model = pq.build_model(t_floats, ref_table, "cpu")
    model.selectors = [p2_sim.SelectorP(**{k: v.to(torch.int8 if "_w" in k else torch.int32)
                                           for k, v in sel.items()})
                       for sel in t_payload["selectors"]]
    fixture["forward_image"] = []
    for i in range(len(imgs)):
        logits, counts, exp = p2_sim.forward_image(model, timgs[i], prune=True)
        fixture["forward_image"].append({"logits": [int(v) for v in logits],
                                         "token_counts": [int(c) for c in counts],
                                         "logits_scale_exp": int(exp)})
    logits, exp = p2_sim_ivit.forward_batch_cfg(model, timgs)
    fixture["forward_batch_unpruned"] = {"logits": logits.to(torch.int64).tolist(),
                                         "logits_scale_exp": int(exp)}
    fixture["reference_seconds"] = round(time.time() - t0, 1)
    OUT.write_text(json.dumps(fixture) + "\n")
    print(f"wrote {OUT} in {fixture['reference_seconds']} s")


if __name__ == "__main__":
    main()
